// gfx950 kernels for the model ops around the attention path: SwiGLU, the token sampler
// (greedy arg-max and Gumbel-max), token feedback and the embedding gather.
//
// These feed or consume the hot path once per layer (SwiGLU) or once per step (the rest); they
// are HBM/launch bound, so each is one coalesced pass with 16-byte accesses.
//
// Numerics (matched bit for bit by the CPU oracle):
//   swiglu : silu = round_T( (float)( g / (1 + exp(-g)) ) evaluated in double ),
//            out = round_T( silu * u ) in float — the reference's rounding points
//            (kernels/fused_ops.cu:210-219) with the exponential evaluated in double so that the
//            result does not depend on the exp implementation's last float ulp.
//   sampler: arg-max with the lowest index winning ties (kernels/fused_ops.cu:302-303); the
//            Gumbel score of a sampling row is (float)(x*inv_t - log(max(-log(u), 1e-10))) in
//            double, u from Philox-4x32-10 (Salmon et al., SC'11) with the counter layout of
//            kernels/fused_ops.cu:327-330.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "cvh_device.h"

namespace cvh {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 ld_nt(const void* p) { return __builtin_nontemporal_load(static_cast<const u32x4*>(p)); }

// ---- SwiGLU ---------------------------------------------------------------------------------

// One thread per 8 consecutive outputs of a row (I % 8 == 0): two 16-byte loads (gate, up) and
// one 16-byte store for 16-bit types.
template <int DT>
__global__ __launch_bounds__(256) void swiglu_kernel(typename Elem<DT>::T* __restrict__ out,
                                                     const typename Elem<DT>::T* __restrict__ gu, int64_t n8, int I) {
    using T = typename Elem<DT>::T;
    const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n8) return;
    const int per_row = I >> 3;
    const int64_t r = k / per_row;
    const int c = static_cast<int>(k - r * per_row) << 3;
    const T* g = gu + r * 2 * I + c;
    const T* u = g + I;
    T* o = out + r * I + c;
    T gv[8], uv[8], ov[8];
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<u32x4*>(gv) = ld_nt(g);
        *reinterpret_cast<u32x4*>(uv) = ld_nt(u);
    } else {
        *reinterpret_cast<uint4*>(gv) = *reinterpret_cast<const uint4*>(g);
        *reinterpret_cast<uint4*>(gv + 4) = *reinterpret_cast<const uint4*>(g + 4);
        *reinterpret_cast<uint4*>(uv) = *reinterpret_cast<const uint4*>(u);
        *reinterpret_cast<uint4*>(uv + 4) = *reinterpret_cast<const uint4*>(u + 4);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ov[j] = Elem<DT>::store(silu_mul<DT>(Elem<DT>::load(gv[j]), Elem<DT>::load(uv[j])));
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint4*>(o) = *reinterpret_cast<const uint4*>(ov);
    } else {
        *reinterpret_cast<uint4*>(o) = *reinterpret_cast<const uint4*>(ov);
        *reinterpret_cast<uint4*>(o + 4) = *reinterpret_cast<const uint4*>(ov + 4);
    }
}

// Any I: one thread per output.
template <int DT>
__global__ __launch_bounds__(256) void swiglu_scalar_kernel(typename Elem<DT>::T* __restrict__ out,
                                                            const typename Elem<DT>::T* __restrict__ gu, int64_t n,
                                                            int I) {
    const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) return;
    const int64_t r = k / I;
    const int i = static_cast<int>(k - r * I);
    out[k] = Elem<DT>::store(silu_mul<DT>(Elem<DT>::load(gu[r * 2 * I + i]), Elem<DT>::load(gu[r * 2 * I + I + i])));
}

// ---- Sampler ----------------------------------------------------------------------------------
constexpr int kSampleThreads = 1024;   // 16 waves per row

// Philox-4x32 with 10 rounds (Random123's philox4x32_10): multipliers 0xD2511F53 / 0xCD9E8D57,
// Weyl key increments 0x9E3779B9 / 0xBB67AE85.
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
        const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = lo1;
        c[2] = n2;
        c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

struct Best {
    float v;
    int i;
};
__device__ __forceinline__ bool better(float v, int i, const Best& b) { return v > b.v || (v == b.v && i < b.i); }

__device__ __forceinline__ float gumbel_score(float x, float inv_t, uint32_t r) {
    const float u = (static_cast<float>(r >> 8) + 0.5f) * (1.0f / 16777216.0f);   // exact
    const double e = fmax(-log(static_cast<double>(u)), 1e-10);
    return static_cast<float>(static_cast<double>(x) * inv_t - log(e));
}

template <int LDT>
__device__ __forceinline__ float load_logit(const void* row, int64_t j) {
    if constexpr (LDT == CVH_DTYPE_F32) return static_cast<const float*>(row)[j];
    else return bf16_bits_to_f32(static_cast<const uint16_t*>(row)[j]);
}

// One workgroup per sampled row. Each thread scans groups of 8 logits (Philox counter = index/4,
// so one group uses two Philox blocks), keeps its best (value, index), then the wave and the
// workgroup reduce with the same tie rule.
template <int LDT>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(int64_t* __restrict__ out, const void* __restrict__ logits,
                                                                const int64_t* __restrict__ rows,
                                                                const float* __restrict__ temps, int V,
                                                                uint64_t seed, uint64_t offset) {
    const int r = blockIdx.x;
    const int64_t src = rows ? rows[r] : r;
    const size_t esz = LDT == CVH_DTYPE_F32 ? 4 : 2;
    const char* row = static_cast<const char*>(logits) + static_cast<size_t>(src) * V * esz;
    const float temp = temps ? temps[r] : 0.f;
    const bool greedy = !(temp > 0.f);
    const float inv_t = 1.0f / fmaxf(temp, 1e-5f);
    const bool vec = (V & 7) == 0;

    Best best{-INFINITY, 0x7fffffff};
    for (int base = threadIdx.x * 8; base < V; base += kSampleThreads * 8) {
        float x[8];
        if (vec && LDT != CVH_DTYPE_F32) {
            const u32x4 w = ld_nt(row + static_cast<size_t>(base) * 2);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[2 * j] = __uint_as_float(ws[j] << 16);
                x[2 * j + 1] = __uint_as_float(ws[j] & 0xffff0000u);
            }
        } else if (vec) {
            const f32x4 a = __builtin_bit_cast(f32x4, ld_nt(row + static_cast<size_t>(base) * 4));
            const f32x4 b = __builtin_bit_cast(f32x4, ld_nt(row + static_cast<size_t>(base) * 4 + 16));
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = base + j < V ? load_logit<LDT>(row, base + j) : -INFINITY;
        }
        if (greedy) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (base + j < V && better(x[j], base + j, best)) best = {x[j], base + j};
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int b4 = base + 4 * h;
                uint32_t c[4] = {static_cast<uint32_t>(b4 >> 2), static_cast<uint32_t>(r), static_cast<uint32_t>(offset),
                                 static_cast<uint32_t>(offset >> 32)};
                philox4x32_10(c, static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32));
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (b4 + j >= V) break;
                    const float s = gumbel_score(x[4 * h + j], inv_t, c[j]);
                    if (better(s, b4 + j, best)) best = {s, b4 + j};
                }
            }
        }
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const float ov = __shfl_xor(best.v, d, 64);
        const int oi = __shfl_xor(best.i, d, 64);
        if (better(ov, oi, best)) best = {ov, oi};
    }
    __shared__ float sv[kSampleThreads / 64];
    __shared__ int si[kSampleThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = best.v;
        si[wave] = best.i;
    }
    __syncthreads();
    if (wave == 0) {
        best = lane < kSampleThreads / 64 ? Best{sv[lane], si[lane]} : Best{-INFINITY, 0x7fffffff};
#pragma unroll
        for (int d = 8; d > 0; d >>= 1) {
            const float ov = __shfl_xor(best.v, d, 64);
            const int oi = __shfl_xor(best.i, d, 64);
            if (better(ov, oi, best)) best = {ov, oi};
        }
        if (lane == 0) out[r] = best.i;
    }
}

// ---- token feedback and embedding -------------------------------------------------------------
__global__ __launch_bounds__(256) void feed_tokens_kernel(int64_t* __restrict__ tokens, const int64_t* __restrict__ src,
                                                          const int64_t* __restrict__ prev, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t s = src[i];
    if (s >= 0) tokens[i] = prev[s];
}

// out[t] = table[ids[t]] for 16-bit rows of D elements (D % 8 == 0): one thread per 16 bytes.
__global__ __launch_bounds__(256) void embedding_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ table,
                                                        const int64_t* __restrict__ ids, int64_t T, int D, int64_t V) {
    const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int per_row = D >> 3;
    if (k >= T * per_row) return;
    const int64_t t = k / per_row;
    const int c = static_cast<int>(k - t * per_row) << 3;
    const int64_t id = ids[t];
    uint4 v = {0u, 0u, 0u, 0u};
    if (id >= 0 && id < V) v = *reinterpret_cast<const uint4*>(table + id * D + c);
    *reinterpret_cast<uint4*>(out + t * D + c) = v;
}

int grid_of(int64_t n, unsigned* g) {
    const int64_t b = (n + 255) / 256;
    if (b > 0x7fffffff) return CVH_ERR_UNSUPPORTED;
    *g = static_cast<unsigned>(b);
    return CVH_OK;
}

int launched() { return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH; }

template <int DT>
int launch_swiglu(void* out, const void* gu, int64_t T, int I, hipStream_t s) {
    using E = typename Elem<DT>::T;
    unsigned g = 0;
    if ((I & 7) == 0) {
        const int64_t n8 = T * (I >> 3);
        if (int rc = grid_of(n8, &g)) return rc;
        swiglu_kernel<DT><<<g, 256, 0, s>>>(static_cast<E*>(out), static_cast<const E*>(gu), n8, I);
    } else {
        if (int rc = grid_of(T * I, &g)) return rc;
        swiglu_scalar_kernel<DT><<<g, 256, 0, s>>>(static_cast<E*>(out), static_cast<const E*>(gu), T * I, I);
    }
    return launched();
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_swiglu(void* out, const void* gate_up, int64_t num_rows, int intermediate, int dtype,
                          cvh_stream_t stream) {
    using namespace cvh;
    if (num_rows < 0 || intermediate <= 0) return CVH_ERR_INVALID_ARG;
    if (num_rows == 0) return CVH_OK;
    if (!out || !gate_up) return CVH_ERR_INVALID_ARG;
    auto s = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case CVH_DTYPE_BF16: return launch_swiglu<CVH_DTYPE_BF16>(out, gate_up, num_rows, intermediate, s);
        case CVH_DTYPE_F16: return launch_swiglu<CVH_DTYPE_F16>(out, gate_up, num_rows, intermediate, s);
        case CVH_DTYPE_F32: return launch_swiglu<CVH_DTYPE_F32>(out, gate_up, num_rows, intermediate, s);
        default: return CVH_ERR_UNSUPPORTED;
    }
}

extern "C" int cvh_sample_tokens(int64_t* out, const void* logits, int logits_dtype, const int64_t* rows,
                                 const float* temps, int64_t num_rows, int vocab, uint64_t seed, uint64_t offset,
                                 cvh_stream_t stream) {
    using namespace cvh;
    if (num_rows < 0 || vocab <= 0) return CVH_ERR_INVALID_ARG;
    if (num_rows == 0) return CVH_OK;
    if (!out || !logits) return CVH_ERR_INVALID_ARG;
    if (num_rows > 0x7fffffff) return CVH_ERR_UNSUPPORTED;
    auto s = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(num_rows));
    if (logits_dtype == CVH_DTYPE_F32)
        sample_kernel<CVH_DTYPE_F32><<<grid, kSampleThreads, 0, s>>>(out, logits, rows, temps, vocab, seed, offset);
    else if (logits_dtype == CVH_DTYPE_BF16)
        sample_kernel<CVH_DTYPE_BF16><<<grid, kSampleThreads, 0, s>>>(out, logits, rows, temps, vocab, seed, offset);
    else
        return CVH_ERR_UNSUPPORTED;
    return launched();
}

extern "C" int cvh_feed_tokens(int64_t* tokens, const int64_t* src, const int64_t* prev, int64_t n,
                               cvh_stream_t stream) {
    using namespace cvh;
    if (n < 0) return CVH_ERR_INVALID_ARG;
    if (n == 0) return CVH_OK;
    if (!tokens || !src || !prev) return CVH_ERR_INVALID_ARG;
    unsigned g = 0;
    if (int rc = grid_of(n, &g)) return rc;
    feed_tokens_kernel<<<g, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(tokens, src, prev, n);
    return launched();
}

extern "C" int cvh_embedding(void* out, const void* table, const int64_t* ids, int64_t num_tokens, int dim,
                             int64_t vocab, cvh_stream_t stream) {
    using namespace cvh;
    if (num_tokens < 0 || dim <= 0 || vocab <= 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!out || !table || !ids) return CVH_ERR_INVALID_ARG;
    if ((dim & 7) != 0) return CVH_ERR_UNSUPPORTED;
    unsigned g = 0;
    if (int rc = grid_of(num_tokens * (dim >> 3), &g)) return rc;
    embedding_kernel<<<g, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            static_cast<uint16_t*>(out), static_cast<const uint16_t*>(table), ids, num_tokens, dim, vocab);
    return launched();
}
