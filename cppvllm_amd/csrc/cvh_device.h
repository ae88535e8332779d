// Device helpers shared by the gfx950 kernels: bf16/f16 rounding, OCP e4m3 encode/decode and
// wavefront reductions. Every rounding helper here has a bit-identical host restatement in the
// CPU oracle (oracle/cvh_oracle.c), which is what makes the cache bytes bit-exact.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/cppvllm_hip.h"

namespace cvh {

// ---- bf16 ------------------------------------------------------------------------------------
// float -> bf16 bits, round to nearest even; NaN -> quiet NaN with the sign kept.
// Branch-free (both results computed, one selected), so a wave never splits on a NaN test.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t qnan = (u >> 16) | 0x40u;
    return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? qnan : rne);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---- fp16 (IEEE half), only used by the f16 instantiation of the norm kernels ----------------
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const _Float16 h = static_cast<_Float16>(f);     // v_cvt_f16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// Storage-type traits for the norm kernels (bf16 / f16 / f32 rows).
template <int DT> struct Elem;
template <> struct Elem<CVH_DTYPE_BF16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return bf16_bits_to_f32(v); }
    static __device__ __forceinline__ T store(float f) { return f32_to_bf16_bits(f); }
};
template <> struct Elem<CVH_DTYPE_F16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return f16_bits_to_f32(v); }
    static __device__ __forceinline__ T store(float f) { return f32_to_f16_bits(f); }
};
template <> struct Elem<CVH_DTYPE_F32> {
    using T = float;
    static __device__ __forceinline__ float load(T v) { return v; }
    static __device__ __forceinline__ T store(float f) { return f; }
};

// ---- RMSNorm of one row by one wavefront ---------------------------------------------------------
// 8-element chunks through 16-byte accesses (two for f32).
template <typename T> struct Chunk8;
template <> struct Chunk8<uint16_t> {
    static __device__ __forceinline__ void load(const uint16_t* p, uint16_t (&v)[8]) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) { v[2 * i] = w[i] & 0xffffu; v[2 * i + 1] = w[i] >> 16; }
    }
    static __device__ __forceinline__ void store(uint16_t* p, const uint16_t (&v)[8]) {
        uint4 u;
        u.x = v[0] | (uint32_t(v[1]) << 16); u.y = v[2] | (uint32_t(v[3]) << 16);
        u.z = v[4] | (uint32_t(v[5]) << 16); u.w = v[6] | (uint32_t(v[7]) << 16);
        *reinterpret_cast<uint4*>(p) = u;
    }
};
template <> struct Chunk8<float> {
    static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
        reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
};

// Plain 16-byte row loads for norm_row.
struct PlainChunk {
    template <typename T>
    __device__ __forceinline__ void operator()(const T* p, T (&v)[8]) const { Chunk8<T>::load(p, v); }
};

// ---- DPP helpers (within rows of 16 lanes) ---------------------------------------------------
// All patterns below give every lane a valid source lane, so bound_ctrl (zero for invalid
// sources) never applies; setting it lets the compiler fold the move into the consuming VALU op
// (v_add_f32_dpp / v_max_f32_dpp).
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// lane ^ 1 and lane ^ 2 inside a quad (quad_perm [1,0,3,2] and [2,3,0,1]).
__device__ __forceinline__ float dpp_xor1(float v) { return dpp<0xB1>(v); }
__device__ __forceinline__ float dpp_xor2(float v) { return dpp<0x4E>(v); }
// row_half_mirror: lane i <-> 7-i inside each group of 8. After the xor1/xor2 levels a quad is
// uniform, so this pairs quad 0 with quad 1 exactly like an xor-4 exchange would.
__device__ __forceinline__ float dpp_half_mirror(float v) { return dpp<0x141>(v); }
// row_mirror: lane i <-> 15-i inside each row of 16 (an xor-8 exchange once halves are uniform).
__device__ __forceinline__ float dpp_mirror(float v) { return dpp<0x140>(v); }
// row_ror:8: lane i <-> (i+8) mod 16 inside each row of 16, i.e. exactly lane ^ 8.
__device__ __forceinline__ float dpp_xor8(float v) { return dpp<0x128>(v); }

// The xor butterfly over aligned groups of N lanes (N = 16 or 64; every lane of a group active):
// level m combines lane i with lane i ^ m for m = 1, 2, 4, ..., so the result equals the
// __shfl_xor butterfly bit for bit, but with DPP (xor 4 and 8 as mirrors once quads / halves are
// uniform) and the gfx950 permlane swaps for xor 16 / 32 instead of LDS-routed ds_bpermute.
template <int N, typename Op> __device__ __forceinline__ float xor_butterfly(float v, Op op) {
    static_assert(N == 16 || N == 64, "row or wave");
    v = op(v, dpp_xor1(v));
    v = op(v, dpp_xor2(v));
    v = op(v, dpp_half_mirror(v));
    v = op(v, dpp_mirror(v));
    if constexpr (N == 64) {
        auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
        r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    return v;
}
template <int N> __device__ __forceinline__ float xor_sum(float v) {
    return xor_butterfly<N>(v, [](float a, float b) { return a + b; });
}
template <int N> __device__ __forceinline__ float xor_max(float v) {
    return xor_butterfly<N>(v, [](float a, float b) { return fmaxf(a, b); });
}

// RMSNorm (ADD: after resid <- rnd(resid + x), normalising resid) of one row of `dim` elements
// (dim % 8 == 0, dim <= 512 * MAXC) by the 64 lanes of a wave: lane l owns chunks l, l+64, ...;
// the sum of squares runs over the lane's elements in index order, then an xor butterfly over the
// 64 lanes; inv = 1 / sqrt(ss / dim + eps) with IEEE sqrt and division; out = rnd(rnd(v * inv) * w).
// Every input is requested before the first reduction. Translation units using this are built
// without FMA contraction.
template <int DT, bool ADD, int MAXC, typename XLoad>
__device__ __forceinline__ void norm_row(typename Elem<DT>::T* __restrict__ orow, typename Elem<DT>::T* rr,
                                         const typename Elem<DT>::T* xr, const typename Elem<DT>::T* __restrict__ w,
                                         int dim, float eps, int lane, XLoad xload) {
    using E = Elem<DT>;
    using T = typename E::T;
    using C = Chunk8<T>;
    const int nchunk = dim >> 3;
    T wr[MAXC][8];
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
        if (lane + 64 * j < nchunk) C::load(w + (lane + 64 * j) * 8, wr[j]);
    float v[MAXC][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunk) {
            T raw[8];
            xload(xr + c * 8, raw);
            if constexpr (ADD) {
                T rs[8];
                C::load(rr + c * 8, rs);
#pragma unroll
                for (int e = 0; e < 8; ++e) rs[e] = E::store(E::load(rs[e]) + E::load(raw[e]));
                C::store(rr + c * 8, rs);
#pragma unroll
                for (int e = 0; e < 8; ++e) raw[e] = rs[e];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[j][e] = E::load(raw[e]);
                ss = ss + v[j][e] * v[j][e];
            }
        }
    }
    ss = xor_sum<64>(ss);
    const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunk) {
            T o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float n = E::load(E::store(v[j][e] * inv));
                o[e] = E::store(n * E::load(wr[j][e]));
            }
            C::store(orow + c * 8, o);
        }
    }
}

// ---- SwiGLU element ---------------------------------------------------------------------------
// silu(g) * u with the reference's rounding points (kernels/fused_ops.cu:210-219): silu rounded to
// the storage type, the product left for the caller to round. The exponential is evaluated in
// double so that the result does not depend on a float exp's last ulp. For bf16 the rounded silu
// depends only on the gate's 16 bits: a 64K-entry table (generated at build time with that double
// formula, silu_bf16_lut.inc) replaces the ~45 double-precision operations per element. Shared by
// the SwiGLU kernel and the gate/up GEMM epilogue, which must agree bit for bit.
namespace {
__device__ const uint16_t kSiluBf16[65536] = {
#include "silu_bf16_lut.inc"
};
}  // namespace

template <int DT>
__device__ __forceinline__ float silu_mul(float g, float u) {
    if constexpr (DT == CVH_DTYPE_BF16) {
        return bf16_bits_to_f32(kSiluBf16[f32_to_bf16_bits(g)]) * u;   // g is a bf16 value
    } else {
        const double e = exp(-static_cast<double>(g));
        const float silu = Elem<DT>::load(Elem<DT>::store(static_cast<float>(static_cast<double>(g) / (1.0 + e))));
        return silu * u;
    }
}

// ---- OCP e4m3fn ------------------------------------------------------------------------------
// Encode with round-to-nearest-even and saturation to +-448 (the __NV_SATFINITE behaviour of the
// reference, kernels/fused_ops.cu:42-44). NaN -> 0x7F. Written with integer ops so the exact same
// bytes come out of the host restatement; derived from the OCP 8-bit FP spec (bias 7, 3 mantissa
// bits, max normal 448 = 0x7E, subnormals k*2^-9).
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7fu;                       // NaN
    if (a >= 0x43e00000u) return sign | 0x7eu;               // |x| >= 448 (incl. inf): saturate
    if (a < 0x3c800000u) {                                   // |x| < 2^-6: subnormal grid k*2^-9
        const float k = __builtin_rintf(__uint_as_float(a) * 512.0f);   // exact scale, RNE
        return sign | static_cast<uint32_t>(k);              // k == 8 is the smallest normal 0x08
    }
    const uint32_t e = (a >> 23) - 127u + 7u;                // 1..15
    uint32_t code = (e << 3) | ((a >> 20) & 7u);
    const uint32_t rem = a & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (code & 1u))) ++code;
    if (code > 0x7eu) code = 0x7eu;
    return sign | code;
}

// Hardware OCP e4m3 -> f32 of the four codes of w (byte i -> f[i]).
// gfx950's v_cvt_pk_f32_fp8 is OCP e4m3fn and exact for every finite code.
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float* f) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
    f[0] = lo[0];
    f[1] = lo[1];
    f[2] = hi[0];
    f[3] = hi[1];
}

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

// ---- QK-RMSNorm + neox RoPE + FP8 K/V write of one (token, head) task -----------------------
// Task order in a token's packed qkv row: H query heads, KV key heads, KV value heads
// (kernels/fused_ops.cu:118-122). A task runs on 16 lanes; lane gl owns elements [P*gl, P*gl+P) and
// [HALF+P*gl, HALF+P*gl+P), P = HD/32, so the neox pair (e, e+HALF) sits in one lane. The load
// phases request the task's inputs (head values; norm gains and this position's cos/sin), the run
// phase does the arithmetic, so a caller can issue the loads early or overlap several tasks. Shared by the
// standalone kernel and the QKV-projection epilogue, which must agree bit for bit; callers are
// built without FMA contraction.
// P consecutive 16-bit / 8-bit values of a lane as one store (P = 4: 8 / 4 bytes; P = 2: 4 / 2).
template <int P> __device__ __forceinline__ void store_u16s(uint16_t* dst, const uint32_t (&v)[P]) {
    if constexpr (P == 4) *reinterpret_cast<uint2*>(dst) = make_uint2(v[0] | (v[1] << 16), v[2] | (v[3] << 16));
    else *reinterpret_cast<uint32_t*>(dst) = v[0] | (v[1] << 16);
}
template <int P> __device__ __forceinline__ void store_u8s(uint8_t* dst, const uint32_t (&v)[P]) {
    if constexpr (P == 4) *reinterpret_cast<uint32_t*>(dst) = v[0] | (v[1] << 8) | (v[2] << 16) | (v[3] << 24);
    else *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(v[0] | (v[1] << 8));
}
template <int P> __device__ __forceinline__ void load_u16s(const uint16_t* src, uint32_t (&v)[P]) {
    if constexpr (P == 4) {
        const uint2 w = *reinterpret_cast<const uint2*>(src);
        v[0] = w.x & 0xffffu; v[1] = w.x >> 16; v[2] = w.y & 0xffffu; v[3] = w.y >> 16;
    } else {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
        v[0] = w & 0xffffu; v[1] = w >> 16;
    }
}

struct QkvDst {
    uint16_t* q_out;
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    const float* cos_t;
    const float* sin_t;
    uint8_t* k_cache;
    uint8_t* v_cache;
    float* k_scale;
    float* v_scale;
    uint16_t* k_dense;
    uint16_t* v_dense;
    int H, KV, log2_bs;
    float eps;
};

template <int HD>
struct QkvTaskIn {
    static constexpr int P = HD / 32;
    float x[2 * P], wv[2 * P], cs[P], sn[P];
};

// The head's HD bf16 values (src: global or LDS).
template <int HD>
__device__ __forceinline__ void qkv_task_load_x(QkvTaskIn<HD>& in, const uint16_t* src, int gl) {
    constexpr int HALF = HD / 2, P = HD / 32;
    const int e0 = P * gl;
    uint32_t lo[P], hi[P];
    load_u16s<P>(src + e0, lo);
    load_u16s<P>(src + HALF + e0, hi);
#pragma unroll
    for (int j = 0; j < P; ++j) {
        in.x[j] = bf16_bits_to_f32(lo[j]);
        in.x[P + j] = bf16_bits_to_f32(hi[j]);
    }
}
// Q/K tasks: the norm gains and this position's cos/sin.
template <int HD>
__device__ __forceinline__ void qkv_task_load_consts(QkvTaskIn<HD>& in, int task, int64_t pos, const QkvDst& d,
                                                     int gl) {
    constexpr int HALF = HD / 2, P = HD / 32;
    const int e0 = P * gl;
    if (task < d.H + d.KV) {
        const uint16_t* wn = task < d.H ? d.q_norm : d.k_norm;
        const float* cr = d.cos_t + pos * HALF + e0;
        const float* sr = d.sin_t + pos * HALF + e0;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            in.wv[j] = bf16_bits_to_f32(wn[e0 + j]);
            in.wv[P + j] = bf16_bits_to_f32(wn[HALF + e0 + j]);
            in.cs[j] = cr[j];
            in.sn[j] = sr[j];
        }
    }
}

template <int HD, int SCALE_MODE>
__device__ __forceinline__ void qkv_task_run(const QkvTaskIn<HD>& in, int64_t t, int task, int64_t slot,
                                             const QkvDst& d, int gl) {
    constexpr int HALF = HD / 2, P = HD / 32;
    const int e0 = P * gl;
    const int H = d.H, KV = d.KV;
    const int bs_mask = (1 << d.log2_bs) - 1;
    if (task >= H + KV) {                // ---- V: quantise (kernels/fused_ops.cu:125-143)
        const int kvh = task - H - KV;
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 2 * P; ++j) amax = fmaxf(amax, fabsf(in.x[j]));
        amax = xor_max<16>(amax);
        if (d.v_dense != nullptr) {
            uint16_t* o = d.v_dense + (t * KV + kvh) * HD;
            uint32_t lo[P], hi[P];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                lo[j] = __float_as_uint(in.x[j]) >> 16;      // the input bits
                hi[j] = __float_as_uint(in.x[P + j]) >> 16;
            }
            store_u16s<P>(o + e0, lo);
            store_u16s<P>(o + HALF + e0, hi);
        }
        if (slot < 0) return;
        float sc, inv;
        if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
            sc = fmaxf(amax, 1e-8f) / 448.0f;
            inv = 1.0f / sc;
        } else {
            inv = 1.0f / d.v_scale[0];
        }
        uint8_t* dst = d.v_cache + (slot * KV + kvh) * HD;
        uint32_t lo[P], hi[P];
#pragma unroll
        for (int j = 0; j < P; ++j) {
            lo[j] = e4m3_encode(in.x[j] * inv);
            hi[j] = e4m3_encode(in.x[P + j] * inv);
        }
        store_u8s<P>(dst + e0, lo);
        store_u8s<P>(dst + HALF + e0, hi);
        if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
            if (gl == 0) d.v_scale[(((slot >> d.log2_bs) * KV + kvh) << d.log2_bs) + (slot & bs_mask)] = sc;
        }
        return;
    }

    // ---- Q / K: per-head RMSNorm (kernels/fused_ops.cu:145-156)
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * P; ++j) ss = ss + in.x[j] * in.x[j];
    ss = xor_sum<16>(ss);
    const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(HD) + d.eps);
    float n[2 * P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        n[j] = round_bf16(round_bf16(in.x[j] * inv) * in.wv[j]);
        n[P + j] = round_bf16(round_bf16(in.x[P + j] * inv) * in.wv[P + j]);
    }
    // ---- neox RoPE on (e, e+HALF) (kernels/fused_ops.cu:157-166)
    float r[2 * P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const float c = in.cs[j], s = in.sn[j];
        const float a = n[j], b = n[P + j];
        const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
        r[j] = ac - bs;
        r[P + j] = bc + as;
    }
    if (task < H) {                      // (kernels/fused_ops.cu:168-173)
        uint16_t* dst = d.q_out + (t * H + task) * HD;
        uint32_t lo[P], hi[P];
#pragma unroll
        for (int j = 0; j < P; ++j) {
            lo[j] = f32_to_bf16_bits(r[j]);
            hi[j] = f32_to_bf16_bits(r[P + j]);
        }
        store_u16s<P>(dst + e0, lo);
        store_u16s<P>(dst + HALF + e0, hi);
        return;
    }

    // ---- K: round to bf16, amax scale, e4m3 (kernels/fused_ops.cu:175-190)
    const int kvh = task - H;
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * P; ++j) { r[j] = round_bf16(r[j]); amax = fmaxf(amax, fabsf(r[j])); }
    amax = xor_max<16>(amax);
    if (d.k_dense != nullptr) {
        uint16_t* o = d.k_dense + (t * KV + kvh) * HD;
        uint32_t lo[P], hi[P];
#pragma unroll
        for (int j = 0; j < P; ++j) {
            lo[j] = f32_to_bf16_bits(r[j]);
            hi[j] = f32_to_bf16_bits(r[P + j]);
        }
        store_u16s<P>(o + e0, lo);
        store_u16s<P>(o + HALF + e0, hi);
    }
    if (slot < 0) return;
    float sc, sinv;
    if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
        sc = fmaxf(amax, 1e-8f) / 448.0f;
        sinv = 1.0f / sc;
    } else {
        sinv = 1.0f / d.k_scale[0];
    }
    uint8_t* dst = d.k_cache + (slot * KV + kvh) * HD;
    uint32_t lo[P], hi[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        lo[j] = e4m3_encode(r[j] * sinv);
        hi[j] = e4m3_encode(r[P + j] * sinv);
    }
    store_u8s<P>(dst + e0, lo);
    store_u8s<P>(dst + HALF + e0, hi);
    if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
        if (gl == 0) d.k_scale[(((slot >> d.log2_bs) * KV + kvh) << d.log2_bs) + (slot & bs_mask)] = sc;
    }
}

}  // namespace cvh
