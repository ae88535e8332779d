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
//            kernels/fused_ops.cu:327-330 (index/4, row, offset).
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
// Design: every candidate becomes one 64-bit key whose unsigned order is the selection order,
//   key = order32(score) << 32 | (0xFFFFFFFF - index),
// so "largest score, lowest index on ties" is a plain unsigned max and a row's winner is the max
// over all its keys. order32 maps float bit patterns to an unsigned order (negatives bit-flipped,
// positives with the sign bit set) and sends NaN below every number, so a NaN never wins. The
// search starts from the key of (-inf, index 0x7FFFFFFF): an all -inf row then gives index 0 and
// an all-NaN row 0x7FFFFFFF, as the reference's (value, index) scan does (kernels/fused_ops.cu:
// 300-306).
// Work split: one workgroup of kSampleWaves waves per row; wave w owns the contiguous slice
// [w*S, (w+1)*S) of the vocab (S a multiple of 8), and its lanes read 8 logits (16 bytes of bf16)
// at a time, lane-consecutive, so one load instruction of a wave covers 1 KB contiguous. Each
// lane folds its keys with a 64-bit max; the wave folds them with a DPP/permlane butterfly on the
// two 32-bit halves; wave leaders fold into one LDS word with ds_max_u64.
constexpr int kSampleWaves = 16;

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

__device__ __forceinline__ uint64_t rank_key(float s, uint32_t index) {
    uint32_t b = __float_as_uint(s);
    if (b == 0x80000000u) b = 0u;                  // -0.0 ties with +0.0 (lower index wins)
    uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    if ((b & 0x7fffffffu) > 0x7f800000u) o = 0u;   // NaN: below -inf
    return (static_cast<uint64_t>(o) << 32) | (0xFFFFFFFFu - index);
}
__device__ __forceinline__ uint32_t key_index(uint64_t k) { return 0xFFFFFFFFu - static_cast<uint32_t>(k); }
__device__ __forceinline__ uint64_t kmax(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Gumbel perturbation of logit x with the 32-bit uniform word r: u = ((r >> 8) + 0.5) / 2^24 (exact
// in float), score = x / t - log(max(-log u, 1e-10)) evaluated in double and rounded to float.
__device__ __forceinline__ float perturbed(float x, float inv_t, uint32_t r) {
    const float u = (static_cast<float>(r >> 8) + 0.5f) * (1.0f / 16777216.0f);
    const double g = -log(fmax(-log(static_cast<double>(u)), 1e-10));
    return static_cast<float>(static_cast<double>(x) * inv_t + g);
}

template <int CTRL> __device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(v)), CTRL, 0xF, 0xF, true);
    const uint32_t hi = __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(v >> 32)), CTRL, 0xF, 0xF, true);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
// Max over the 64 lanes (every lane active): quad DPP, then mirrors (exact once quads / halves are
// uniform), then the gfx950 permlane16/32 swaps across rows.
__device__ __forceinline__ uint64_t wave_kmax(uint64_t v) {
    v = kmax(v, dpp64<0xB1>(v));
    v = kmax(v, dpp64<0x4E>(v));
    v = kmax(v, dpp64<0x141>(v));
    v = kmax(v, dpp64<0x140>(v));
    uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
    auto l16 = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    auto h16 = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = kmax((static_cast<uint64_t>(h16[0]) << 32) | l16[0], (static_cast<uint64_t>(h16[1]) << 32) | l16[1]);
    lo = static_cast<uint32_t>(v);
    hi = static_cast<uint32_t>(v >> 32);
    auto l32 = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    auto h32 = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return kmax((static_cast<uint64_t>(h32[0]) << 32) | l32[0], (static_cast<uint64_t>(h32[1]) << 32) | l32[1]);
}

// The 8 logits at [j, j+8) of a row as float; positions past V read as -inf (never selected:
// the caller does not fold them).
template <int LDT>
__device__ __forceinline__ void logits8(const char* row, int j, int V, float* x) {
    if (j + 8 <= V && (V & 7) == 0) {
        if constexpr (LDT == CVH_DTYPE_F32) {
            const u32x4 a = ld_nt(row + static_cast<size_t>(j) * 4);
            const u32x4 b = ld_nt(row + static_cast<size_t>(j) * 4 + 16);
            x[0] = __uint_as_float(a.x); x[1] = __uint_as_float(a.y); x[2] = __uint_as_float(a.z); x[3] = __uint_as_float(a.w);
            x[4] = __uint_as_float(b.x); x[5] = __uint_as_float(b.y); x[6] = __uint_as_float(b.z); x[7] = __uint_as_float(b.w);
        } else {
            const u32x4 a = ld_nt(row + static_cast<size_t>(j) * 2);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = bf16_bits_to_f32(w[e] & 0xffffu);
                x[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (j + e >= V) { x[e] = -INFINITY; continue; }
            if constexpr (LDT == CVH_DTYPE_F32) x[e] = reinterpret_cast<const float*>(row)[j + e];
            else x[e] = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(row)[j + e]);
        }
    }
}

template <int LDT, bool GUMBEL>
__device__ __forceinline__ uint64_t scan_slice(const char* row, int lo, int hi, int V, int lane, int r, float inv_t,
                                               uint64_t seed, uint64_t offset) {
    uint64_t best = rank_key(-INFINITY, 0x7fffffffu);
    for (int j = lo + 8 * lane; j < hi; j += 8 * 64) {
        float x[8];
        logits8<LDT>(row, j, V, x);
        uint32_t rnd[8];
        if constexpr (GUMBEL) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // Philox counter (index / 4, row, offset): one block gives the words of 4 indices
                uint32_t c[4] = {static_cast<uint32_t>((j >> 2) + h), static_cast<uint32_t>(r),
                                 static_cast<uint32_t>(offset), static_cast<uint32_t>(offset >> 32)};
                philox4x32_10(c, static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32));
#pragma unroll
                for (int e = 0; e < 4; ++e) rnd[4 * h + e] = c[e];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (j + e >= hi) break;
            const float s = GUMBEL ? perturbed(x[e], inv_t, rnd[e]) : x[e];
            best = kmax(best, rank_key(s, static_cast<uint32_t>(j + e)));
        }
    }
    return best;
}

template <int LDT>
__global__ __launch_bounds__(64 * kSampleWaves) void sample_kernel(int64_t* __restrict__ out,
                                                                   const void* __restrict__ logits,
                                                                   const int64_t* __restrict__ rows,
                                                                   const float* __restrict__ temps, int V,
                                                                   uint64_t seed, uint64_t offset) {
    __shared__ unsigned long long winner;
    const int r = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x == 0) winner = 0ull;
    const int64_t src = rows ? rows[r] : r;
    const char* row = static_cast<const char*>(logits) + static_cast<size_t>(src) * V * (LDT == CVH_DTYPE_F32 ? 4 : 2);
    const float t = temps ? temps[r] : 0.f;
    // contiguous slice of this wave, a multiple of 8 so a Philox block never straddles slices
    const int slice = ((V + kSampleWaves * 8 - 1) / (kSampleWaves * 8)) * 8;
    const int lo = wave * slice, hi = min(V, lo + slice);
    uint64_t k = t > 0.f ? scan_slice<LDT, true>(row, lo, hi, V, lane, r, 1.0f / fmaxf(t, 1e-5f), seed, offset)
                         : scan_slice<LDT, false>(row, lo, hi, V, lane, r, 0.f, seed, offset);
    k = wave_kmax(k);
    __syncthreads();
    if (lane == 0) atomicMax(&winner, static_cast<unsigned long long>(k));
    __syncthreads();
    if (threadIdx.x == 0) out[r] = key_index(winner);
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
        sample_kernel<CVH_DTYPE_F32><<<grid, 64 * kSampleWaves, 0, s>>>(out, logits, rows, temps, vocab, seed, offset);
    else if (logits_dtype == CVH_DTYPE_BF16)
        sample_kernel<CVH_DTYPE_BF16><<<grid, 64 * kSampleWaves, 0, s>>>(out, logits, rows, temps, vocab, seed, offset);
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
