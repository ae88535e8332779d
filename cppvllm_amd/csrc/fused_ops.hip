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
// One 16-lane group per (token, head task); task order inside a token row follows the packed
// qkv layout: H query heads, KV key heads, KV value heads (kernels/fused_ops.cu:118-122).
// Lane i of a group owns elements [P*i, P*i+P) and [HALF+P*i, HALF+P*i+P), P = HD/32, so the
// neox RoPE pair (e, e+HALF) lives in one lane and needs no cross-lane exchange.
constexpr int kQkvGroupsPerBlock = 16;   // 256 threads

template <int HD, int SCALE_MODE>
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(
        uint16_t* __restrict__ q_out, const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_norm,
        const uint16_t* __restrict__ k_norm, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
        const int64_t* __restrict__ positions, const int64_t* __restrict__ slots, uint8_t* __restrict__ k_cache,
        uint8_t* __restrict__ v_cache, float* __restrict__ k_scale, float* __restrict__ v_scale,
        uint16_t* __restrict__ k_dense, uint16_t* __restrict__ v_dense, int H, int KV, int log2_bs, float eps) {
    constexpr int HALF = HD / 2;
    constexpr int P = HD / 32;           // elements per lane per half (4 for HD=128, 2 for HD=64)
    const int gl = threadIdx.x & 15;     // lane inside the 16-lane group
    const int n_tasks = H + 2 * KV;
    const int task = blockIdx.x * kQkvGroupsPerBlock + (threadIdx.x >> 4);
    if (task >= n_tasks) return;         // whole 16-lane groups exit together
    const int64_t t = blockIdx.y;
    const uint16_t* src = qkv + (t * n_tasks + task) * HD;
    const int e0 = P * gl;               // first-half element index; partner is e0 + HALF

    // every global input of the task is requested before the first reduction, so the kernel waits
    // for memory once: the head, and for Q/K the norm gains and this position's cos/sin
    const int64_t slot = slots[t];
    const int64_t pos = positions[t];
    const bool is_qk = task < H + KV;
    float x[2 * P], wv[2 * P], cs[P], sn[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        x[j] = bf16_bits_to_f32(src[e0 + j]);
        x[P + j] = bf16_bits_to_f32(src[HALF + e0 + j]);
    }
    if (is_qk) {
        const uint16_t* wn = task < H ? q_norm : k_norm;
        const float* cr = cos_t + pos * HALF + e0;
        const float* sr = sin_t + pos * HALF + e0;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            wv[j] = bf16_bits_to_f32(wn[e0 + j]);
            wv[P + j] = bf16_bits_to_f32(wn[HALF + e0 + j]);
            cs[j] = cr[j];
            sn[j] = sr[j];
        }
    }
    const int bs_mask = (1 << log2_bs) - 1;

    if (!is_qk) {                        // ---- V: quantise (kernels/fused_ops.cu:125-143)
        const int kvh = task - H - KV;
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 2 * P; ++j) amax = fmaxf(amax, fabsf(x[j]));
        amax = xor_max<16>(amax);
        if (v_dense != nullptr) {
            uint16_t* d = v_dense + (t * KV + kvh) * HD;
#pragma unroll
            for (int j = 0; j < P; ++j) { d[e0 + j] = src[e0 + j]; d[HALF + e0 + j] = src[HALF + e0 + j]; }
        }
        if (slot < 0) return;
        float sc, inv;
        if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
            sc = fmaxf(amax, 1e-8f) / 448.0f;
            inv = 1.0f / sc;
        } else {
            inv = 1.0f / v_scale[0];
        }
        uint8_t* dst = v_cache + (slot * KV + kvh) * HD;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            dst[e0 + j] = static_cast<uint8_t>(e4m3_encode(x[j] * inv));
            dst[HALF + e0 + j] = static_cast<uint8_t>(e4m3_encode(x[P + j] * inv));
        }
        if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
            if (gl == 0) v_scale[(((slot >> log2_bs) * KV + kvh) << log2_bs) + (slot & bs_mask)] = sc;
        }
        return;
    }

    // ---- Q / K: per-head RMSNorm (kernels/fused_ops.cu:145-156)
    const bool is_q = task < H;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * P; ++j) ss = ss + x[j] * x[j];
    ss = xor_sum<16>(ss);
    const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(HD) + eps);

    float n[2 * P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        n[j] = round_bf16(round_bf16(x[j] * inv) * wv[j]);
        n[P + j] = round_bf16(round_bf16(x[P + j] * inv) * wv[P + j]);
    }
    // ---- neox RoPE on (e, e+HALF) (kernels/fused_ops.cu:157-166)
    float r[2 * P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const float c = cs[j], s = sn[j];
        const float a = n[j], b = n[P + j];
        const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
        r[j] = ac - bs;
        r[P + j] = bc + as;
    }

    if (is_q) {                          // (kernels/fused_ops.cu:168-173)
        uint16_t* dst = q_out + (t * H + task) * HD;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            dst[e0 + j] = f32_to_bf16_bits(r[j]);
            dst[HALF + e0 + j] = f32_to_bf16_bits(r[P + j]);
        }
        return;
    }

    // ---- K: round to bf16, amax scale, e4m3 (kernels/fused_ops.cu:175-190)
    const int kvh = task - H;
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * P; ++j) { r[j] = round_bf16(r[j]); amax = fmaxf(amax, fabsf(r[j])); }
    amax = xor_max<16>(amax);
    if (k_dense != nullptr) {
        uint16_t* d = k_dense + (t * KV + kvh) * HD;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            d[e0 + j] = f32_to_bf16_bits(r[j]);
            d[HALF + e0 + j] = f32_to_bf16_bits(r[P + j]);
        }
    }
    if (slot < 0) return;
    float sc, sinv;
    if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
        sc = fmaxf(amax, 1e-8f) / 448.0f;
        sinv = 1.0f / sc;
    } else {
        sinv = 1.0f / k_scale[0];
    }
    uint8_t* dst = k_cache + (slot * KV + kvh) * HD;
#pragma unroll
    for (int j = 0; j < P; ++j) {
        dst[e0 + j] = static_cast<uint8_t>(e4m3_encode(r[j] * sinv));
        dst[HALF + e0 + j] = static_cast<uint8_t>(e4m3_encode(r[P + j] * sinv));
    }
    if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
        if (gl == 0) k_scale[(((slot >> log2_bs) * KV + kvh) << log2_bs) + (slot & bs_mask)] = sc;
    }
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
    auto* qo = static_cast<uint16_t*>(q_out);
    auto* in = static_cast<const uint16_t*>(qkv);
    auto* qn = static_cast<const uint16_t*>(q_norm);
    auto* kn = static_cast<const uint16_t*>(k_norm);
    auto* kd = static_cast<uint16_t*>(k_dense);
    auto* vd = static_cast<uint16_t*>(v_dense);
#define CVH_QKV_LAUNCH(HD, SM)                                                                                       \
    qk_norm_rope_kv_kernel<HD, SM><<<grid, 256, 0, s>>>(qo, in, qn, kn, cos_t, sin_t, positions, slots, k_cache,     \
                                                        v_cache, k_scale, v_scale, kd, vd, n_heads, n_kv_heads, lg, e)
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
