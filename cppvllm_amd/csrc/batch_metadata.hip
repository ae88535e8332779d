// Per-token metadata of a ragged batch (slot mapping, token->sequence row, causal length) and
// the host-side RoPE tables. Reference: model/model_architecture.cpp:67-75 (RoPE tables) and
// :137-147 (searchsorted / slot / kv_len built from torch ops once per step).
#include <hip/hip_runtime.h>

#include <math.h>

#include "cvh_device.h"

namespace cvh {
namespace {

// One thread per token. seq = number of sequence ends cu_seqlens[1..S] that are <= t
// (torch.searchsorted(ends, t, right=True)), found by binary search over the monotone ends.
__global__ __launch_bounds__(256) void token_metadata_kernel(const int64_t* __restrict__ cu, int64_t S,
                                                             const int64_t* __restrict__ positions, int64_t T,
                                                             const int64_t* __restrict__ tables, int64_t W,
                                                             int log2_bs, int64_t* __restrict__ token_seq,
                                                             int64_t* __restrict__ slots,
                                                             int64_t* __restrict__ kv_len) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    int64_t lo = 0, hi = S;              // count of ends <= t lies in [0, S]
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (cu[mid + 1] <= t) lo = mid + 1;
        else hi = mid;
    }
    const int64_t seq = lo;
    const int64_t pos = positions[t];
    int64_t slot = -1, seq_out = -1, len = 0;
    if (seq < S && pos >= 0) {
        const int64_t b = pos >> log2_bs;
        const int64_t phys = b < W ? tables[seq * W + b] : -1;
        if (phys >= 0) {
            slot = (phys << log2_bs) + (pos & ((int64_t{1} << log2_bs) - 1));
            seq_out = seq;
            len = pos + 1;
        }
    }
    if (token_seq) token_seq[t] = seq_out;
    if (slots) slots[t] = slot;
    if (kv_len) kv_len[t] = len;
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_build_token_metadata(const int64_t* cu_seqlens, int64_t num_seqs, const int64_t* positions,
                                        int64_t num_tokens, const int64_t* block_tables, int64_t table_width,
                                        int block_size, int64_t* token_seq, int64_t* slots, int64_t* token_kv_len,
                                        cvh_stream_t stream) {
    if (num_tokens < 0 || num_seqs < 0 || table_width < 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!cu_seqlens || !positions || (num_seqs > 0 && table_width > 0 && !block_tables)) return CVH_ERR_INVALID_ARG;
    int lg = -1;
    for (int i = 0; i < 31; ++i)
        if ((1 << i) == block_size) lg = i;
    if (lg < 0) return CVH_ERR_UNSUPPORTED;
    const int64_t blocks = (num_tokens + 255) / 256;
    if (blocks > 0x7fffffff) return CVH_ERR_UNSUPPORTED;
    cvh::token_metadata_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            cu_seqlens, num_seqs, positions, num_tokens, block_tables, table_width, lg, token_seq, slots,
            token_kv_len);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

extern "C" int cvh_rope_tables_host(float* cos_t, float* sin_t, int64_t max_position, int head_dim, double theta) {
    if (!cos_t || !sin_t || max_position < 0 || head_dim <= 0 || (head_dim & 1) || !(theta > 0.0))
        return CVH_ERR_INVALID_ARG;
    const int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        // inv_freq_i = 1 / theta^(2i/hd), all in double (model/model_architecture.cpp:69-71)
        const double inv_freq = 1.0 / pow(theta, static_cast<double>(2 * i) / static_cast<double>(head_dim));
        for (int64_t p = 0; p < max_position; ++p) {
            const double a = static_cast<double>(p) * inv_freq;
            cos_t[p * half + i] = static_cast<float>(cos(a));
            sin_t[p * half + i] = static_cast<float>(sin(a));
        }
    }
    return CVH_OK;
}

extern "C" const char* cvh_version(void) { return "cppvllm-mi355x 0.2 (gfx950)"; }
