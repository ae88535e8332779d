// Fused pre-attention ops for gfx950: RMSNorm / residual-add+RMSNorm, and per-head
// QK-RMSNorm + neox RoPE + FP8 e4m3 quantise-and-scatter of K/V into the paged cache.
//
// Reference semantics: kernels/fused_ops.cu:61-98 (norms) and :104-207 (qk-norm/rope/kv-write).
// Numerics are pinned to a documented order so that the CPU oracle reproduces every bit:
//   * this translation unit is built with -ffp-contract=off (no silent FMA);
//   * sum of squares: each lane sums its own elements in increasing index order, then an
//     xor-butterfly over the lanes of the row/head (levels 1,2,4,...);
//   * 1/sqrt is IEEE sqrt followed by IEEE division (correctly rounded on gfx950 by default);
//   * RoPE: r_a = a*c - b*s, r_b = b*c + a*s with every product and sum rounded separately.
#include <hip/hip_runtime.h>

#include "cvh_device.h"

namespace cvh {
namespace {

// ---- RMSNorm ---------------------------------------------------------------------------------
// One wavefront per row, 4 rows per 256-thread workgroup. Lane l owns the 8-element chunks
// l, l+64, l+128, ... of the row (one 16-byte load per chunk for bf16/f16, two for f32), and
// keeps them in registers between the sum-of-squares pass and the output pass.
constexpr int kNormWaves = 4;

template <int DT, bool ADD, int MAXC>
__global__ __launch_bounds__(64 * kNormWaves) void rms_norm_kernel(typename Elem<DT>::T* __restrict__ out,
                                                                   typename Elem<DT>::T* resid,
                                                                   const typename Elem<DT>::T* __restrict__ x,
                                                                   const typename Elem<DT>::T* __restrict__ w,
                                                                   int64_t num_rows, int dim, float eps) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
    if (row >= num_rows) return;
    norm_row<DT, ADD, MAXC>(out + row * dim, ADD ? resid + row * dim : nullptr, x + row * dim, w, dim, eps,
                            threadIdx.x & 63, PlainChunk{});
}

// ---- QK-RMSNorm + RoPE + FP8 KV write --------------------------------------------------------
// One 16-lane group per (token, head task), the task body shared with the QKV-projection epilogue
// (qkv_task_load / qkv_task_run).
constexpr int kQkvGroupsPerBlock = 16;   // 256 threads

template <int HD, int SCALE_MODE>
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(const uint16_t* __restrict__ qkv,
                                                              const int64_t* __restrict__ positions,
                                                              const int64_t* __restrict__ slots, QkvDst d) {
    const int gl = threadIdx.x & 15;     // lane inside the 16-lane group
    const int n_tasks = d.H + 2 * d.KV;
    const int task = blockIdx.x * kQkvGroupsPerBlock + (threadIdx.x >> 4);
    if (task >= n_tasks) return;         // whole 16-lane groups exit together
    const int64_t t = blockIdx.y;
    // every global input of the task is requested before the first reduction, so the kernel waits
    // for memory once
    const int64_t slot = slots[t];
    const int64_t pos = positions[t];
    QkvTaskIn<HD> in;
    qkv_task_load_x<HD>(in, qkv + (t * n_tasks + task) * HD, gl);
    qkv_task_load_consts<HD>(in, task, pos, d, gl);
    qkv_task_run<HD, SCALE_MODE>(in, t, task, slot, d, gl);
}

__global__ __launch_bounds__(256) void e4m3_quantize_kernel(uint8_t* __restrict__ dst, const float* __restrict__ src,
                                                            int64_t n, float inv_scale) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = static_cast<uint8_t>(e4m3_encode(src[i] * inv_scale));
}

int ilog2_pow2(int v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

template <int DT, int MAXC>
void launch_norm_c(bool add, void* out, void* resid, const void* x, const void* w, int64_t n, int dim, float eps,
                   hipStream_t stream) {
    using T = typename Elem<DT>::T;
    const dim3 grid(static_cast<unsigned>((n + kNormWaves - 1) / kNormWaves));
    if (add) {
        rms_norm_kernel<DT, true, MAXC><<<grid, 64 * kNormWaves, 0, stream>>>(
                static_cast<T*>(out), static_cast<T*>(resid), static_cast<const T*>(x), static_cast<const T*>(w), n,
                dim, eps);
    } else {
        rms_norm_kernel<DT, false, MAXC><<<grid, 64 * kNormWaves, 0, stream>>>(
                static_cast<T*>(out), nullptr, static_cast<const T*>(x), static_cast<const T*>(w), n, dim, eps);
    }
}

template <int DT>
int launch_norm(bool add, void* out, void* resid, const void* x, const void* w, int64_t n, int dim, float eps,
                hipStream_t stream) {
    const int nchunk = dim / 8;
    if (nchunk <= 64) launch_norm_c<DT, 1>(add, out, resid, x, w, n, dim, eps, stream);
    else if (nchunk <= 128) launch_norm_c<DT, 2>(add, out, resid, x, w, n, dim, eps, stream);
    else if (nchunk <= 256) launch_norm_c<DT, 4>(add, out, resid, x, w, n, dim, eps, stream);
    else launch_norm_c<DT, 16>(add, out, resid, x, w, n, dim, eps, stream);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

int norm_entry(bool add, void* out, void* resid, const void* x, const void* w, int64_t n, int dim, double eps,
               int dtype, hipStream_t stream) {
    if (n < 0) return CVH_ERR_INVALID_ARG;
    if (n == 0) return CVH_OK;
    if (out == nullptr || x == nullptr || w == nullptr || (add && resid == nullptr)) return CVH_ERR_INVALID_ARG;
    if (dim <= 0 || (dim & 7) != 0 || dim > 8192) return CVH_ERR_UNSUPPORTED;
    if (n > (int64_t{1} << 33)) return CVH_ERR_UNSUPPORTED;
    const float e = static_cast<float>(eps);
    switch (dtype) {
        case CVH_DTYPE_BF16: return launch_norm<CVH_DTYPE_BF16>(add, out, resid, x, w, n, dim, e, stream);
        case CVH_DTYPE_F16: return launch_norm<CVH_DTYPE_F16>(add, out, resid, x, w, n, dim, e, stream);
        case CVH_DTYPE_F32: return launch_norm<CVH_DTYPE_F32>(add, out, resid, x, w, n, dim, e, stream);
        default: return CVH_ERR_UNSUPPORTED;
    }
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_rms_norm(void* out, const void* x, const void* w, int64_t num_rows, int dim, double eps, int dtype,
                            cvh_stream_t stream) {
    return cvh::norm_entry(false, out, nullptr, x, w, num_rows, dim, eps, dtype, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cvh_add_rms_norm(void* resid, const void* x, const void* w, void* out, int64_t num_rows, int dim,
                                double eps, int dtype, cvh_stream_t stream) {
    return cvh::norm_entry(true, out, resid, x, w, num_rows, dim, eps, dtype, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cvh_qk_norm_rope_kv_write_fp8(void* q_out, const void* qkv, const void* q_norm, const void* k_norm,
                                             const float* cos_t, const float* sin_t, const int64_t* positions,
                                             const int64_t* slots, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                                             float* v_scale, void* k_dense, void* v_dense, int64_t num_tokens,
                                             int n_heads, int n_kv_heads, int head_dim, int block_size, int scale_mode,
                                             double eps, cvh_stream_t stream) {
    using namespace cvh;
    if (num_tokens < 0 || n_heads <= 0 || n_kv_heads <= 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!q_out || !qkv || !q_norm || !k_norm || !cos_t || !sin_t || !positions || !slots || !k_cache || !v_cache ||
        !k_scale || !v_scale)
        return CVH_ERR_INVALID_ARG;
    const int lg = ilog2_pow2(block_size);
    if (lg < 4 || lg > 12) return CVH_ERR_UNSUPPORTED;
    if (scale_mode != CVH_SCALE_PER_TOKEN_HEAD && scale_mode != CVH_SCALE_PER_TENSOR) return CVH_ERR_UNSUPPORTED;
    if (num_tokens > 0x7fffffff) return CVH_ERR_UNSUPPORTED;
    const int n_tasks = n_heads + 2 * n_kv_heads;
    const dim3 grid(static_cast<unsigned>((n_tasks + kQkvGroupsPerBlock - 1) / kQkvGroupsPerBlock),
                    static_cast<unsigned>(num_tokens));
    auto s = reinterpret_cast<hipStream_t>(stream);
    const float e = static_cast<float>(eps);
    const QkvDst d{static_cast<uint16_t*>(q_out), static_cast<const uint16_t*>(q_norm),
                   static_cast<const uint16_t*>(k_norm), cos_t, sin_t, k_cache, v_cache, k_scale, v_scale,
                   static_cast<uint16_t*>(k_dense), static_cast<uint16_t*>(v_dense), n_heads, n_kv_heads, lg, e};
    auto* in = static_cast<const uint16_t*>(qkv);
#define CVH_QKV_LAUNCH(HD, SM) qk_norm_rope_kv_kernel<HD, SM><<<grid, 256, 0, s>>>(in, positions, slots, d)
    if (head_dim == 128) {
        if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD) CVH_QKV_LAUNCH(128, CVH_SCALE_PER_TOKEN_HEAD);
        else CVH_QKV_LAUNCH(128, CVH_SCALE_PER_TENSOR);
    } else if (head_dim == 64) {
        if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD) CVH_QKV_LAUNCH(64, CVH_SCALE_PER_TOKEN_HEAD);
        else CVH_QKV_LAUNCH(64, CVH_SCALE_PER_TENSOR);
    } else {
        return CVH_ERR_UNSUPPORTED;
    }
#undef CVH_QKV_LAUNCH
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

extern "C" int cvh_fp8_e4m3_quantize(uint8_t* dst, const float* src, int64_t n, float inv_scale,
                                     cvh_stream_t stream) {
    if (n < 0) return CVH_ERR_INVALID_ARG;
    if (n == 0) return CVH_OK;
    if (!dst || !src) return CVH_ERR_INVALID_ARG;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return CVH_ERR_UNSUPPORTED;
    cvh::e4m3_quantize_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            dst, src, n, inv_scale);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}
