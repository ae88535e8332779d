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

// How a row's input x is read: plainly, or with agent-scope coherent loads (relaxed atomics, the
// sc1 bit) when another workgroup of the same kernel wrote it (see the GEMM's fused norm).
struct PlainChunk {
    template <typename T>
    __device__ __forceinline__ void operator()(const T* p, T (&v)[8]) const { Chunk8<T>::load(p, v); }
};
struct AgentChunk {
    __device__ __forceinline__ void operator()(const uint16_t* p, uint16_t (&v)[8]) const {
        const uint64_t a = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t b = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p) + 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = static_cast<uint16_t>(a >> (16 * i));
            v[4 + i] = static_cast<uint16_t>(b >> (16 * i));
        }
    }
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
// double so that the result does not depend on a float exp's last ulp. Shared by the SwiGLU kernel
// and the gate/up GEMM epilogue, which must agree bit for bit.
template <int DT>
__device__ __forceinline__ float silu_mul(float g, float u) {
    const double e = exp(-static_cast<double>(g));
    const float silu = Elem<DT>::load(Elem<DT>::store(static_cast<float>(static_cast<double>(g) / (1.0 + e))));
    return silu * u;
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

}  // namespace cvh
