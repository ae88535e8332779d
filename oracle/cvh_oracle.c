/*
 * cvh_oracle.c — CPU restatement of cppvllm's FP8 paged-decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP library and the CPU
 * baseline timed by bench.py. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product path (cppvllm_amd) never does.
 *
 * Every function cites the reference code it restates (paths relative to the cppvllm source).
 * Where the reference leaves the floating-point order open (warp-shuffle reductions under
 * --use_fast_math), this restatement fixes one documented order, and the gfx950 kernels follow
 * the same order, so that FP8 cache bytes and scales are bit-exact:
 *   - sum of squares: lane-partial sums in increasing element order, then xor-butterfly levels
 *     1,2,4,... over the lanes (16 lanes per head for QK-norm, 64 lanes per row for RMSNorm);
 *   - 1/sqrt(v) = 1.0f / sqrtf(v) (IEEE sqrt and division, both correctly rounded);
 *   - no fused multiply-add anywhere (built with -ffp-contract=off).
 *
 * Pinning status (what checks each function independently of this code) is listed in the
 * header of oracle/__init__.py and enforced by tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_PER_TOKEN_HEAD 0
#define ORC_PER_TENSOR 1
#define ORC_BF16 0
#define ORC_F16 1
#define ORC_F32 2

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- bf16: round to nearest even (the rounding of __float2bfloat16 used by the reference,
 *      kernels/fused_ops.cu:25,27). NaN -> quiet NaN keeping the sign. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }
static inline float rbf16(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* ---- IEEE binary16, round to nearest even (fused_ops.cu:24 __float2half). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                            /* < 2^-14: subnormal grid 2^-24 */
        float k = rintf(u2f(a) * 16777216.0f);                        /* exact power-of-two scale */
        return (uint16_t)(sign | (uint32_t)k);
    }
    uint32_t e = (a >> 23) - 127u + 15u;
    uint32_t code = (e << 10) | ((a >> 13) & 0x3ffu);
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (code & 1u))) ++code;
    return (uint16_t)(sign | code);
}
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

/* ---- OCP e4m3fn encode: RNE, saturate to +-448, NaN -> 0x7F.
 *      Restates __nv_cvt_float_to_fp8(x, __NV_SATFINITE, __NV_E4M3) (kernels/fused_ops.cu:42-44)
 *      from the OCP 8-bit floating point specification (bias 7, max 448, subnormals k*2^-9). */
uint8_t orc_e4m3_encode(float x) {
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7f;
    if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu);
    if (a < 0x3c800000u) {
        float k = rintf(u2f(a) * 512.0f);
        return (uint8_t)(sign | (uint32_t)k);
    }
    uint32_t e = (a >> 23) - 127u + 7u;
    uint32_t code = (e << 3) | ((a >> 20) & 7u);
    uint32_t rem = a & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (code & 1u))) ++code;
    if (code > 0x7eu) code = 0x7eu;
    return (uint8_t)(sign | code);
}

/* ---- OCP e4m3fn decode, spec formula. The reference's bit trick (paged_attention.cu:21-30)
 *      yields this value times 2^-8 for every finite code and is compensated there by *256. */
float orc_e4m3_decode(uint8_t c) {
    int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

void orc_e4m3_quantize(uint8_t* dst, const float* src, int64_t n, float inv_scale) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_e4m3_encode(src[i] * inv_scale);
}

/* ---- element load/store for the norm dtypes */
static inline float ld(const void* p, int64_t i, int dt) {
    if (dt == ORC_BF16) return orc_bf16_to_f32(((const uint16_t*)p)[i]);
    if (dt == ORC_F16) return orc_f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}
static inline void st(void* p, int64_t i, int dt, float v) {
    if (dt == ORC_BF16) ((uint16_t*)p)[i] = orc_f32_to_bf16(v);
    else if (dt == ORC_F16) ((uint16_t*)p)[i] = orc_f32_to_f16(v);
    else ((float*)p)[i] = v;
}
static inline float rnd(float v, int dt) {
    if (dt == ORC_BF16) return rbf16(v);
    if (dt == ORC_F16) return orc_f16_to_f32(orc_f32_to_f16(v));
    return v;
}

/* xor-butterfly over n lanes (n a power of two): after it every lane holds the same sum. */
static float butterfly_sum(float* p, int n) {
    float tmp[64];
    for (int m = 1; m < n; m <<= 1) {
        for (int i = 0; i < n; ++i) tmp[i] = p[i] + p[i ^ m];
        for (int i = 0; i < n; ++i) p[i] = tmp[i];
    }
    return p[0];
}

/* ---- rms_norm / add_rms_norm: restates rms_norm_kernel<T,ADD> (kernels/fused_ops.cu:61-88).
 *      v = rnd(resid + x) (ADD; resid <- v), inv = 1/sqrt(sum(v^2)/D + eps),
 *      out = rnd(rnd(v*inv) * w). Reduction order: 64 lanes, lane l owns 8-element chunks
 *      l, l+64, ... in increasing order; then butterfly over 64 lanes. */
static void norm_rows(void* out, void* resid, const void* x, const void* w, int64_t N, int D, float eps, int dt,
                      int add) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < N; ++r) {
        float part[64];
        int nchunk = D / 8;
        for (int l = 0; l < 64; ++l) {
            float ss = 0.f;
            for (int c = l; c < nchunk; c += 64)
                for (int e = 0; e < 8; ++e) {
                    int64_t i = r * (int64_t)D + c * 8 + e;
                    float v = ld(x, i, dt);
                    if (add) v = rnd(ld(resid, i, dt) + v, dt);
                    ss = ss + v * v;
                }
            part[l] = ss;
        }
        float ss = butterfly_sum(part, 64);
        float inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (int d = 0; d < D; ++d) {
            int64_t i = r * (int64_t)D + d;
            float v = ld(x, i, dt);
            if (add) {
                v = rnd(ld(resid, i, dt) + v, dt);
                st(resid, i, dt, v);
            }
            float n = rnd(v * inv, dt);
            st(out, i, dt, n * ld(w, d, dt));
        }
    }
}
void orc_rms_norm(void* out, const void* x, const void* w, int64_t N, int D, double eps, int dt) {
    norm_rows(out, 0, x, w, N, D, (float)eps, dt, 0);
}
void orc_add_rms_norm(void* resid, const void* x, const void* w, void* out, int64_t N, int D, double eps, int dt) {
    norm_rows(out, resid, x, w, N, D, (float)eps, dt, 1);
}

/* ---- QK-RMSNorm + neox RoPE + FP8 quantise-and-scatter.
 *      Restates qk_norm_rope_kv_fp8_kernel<bf16,HD> (kernels/fused_ops.cu:104-191), with
 *      block_size as a parameter (the reference hard-codes 16, :136,185) and slot < 0 skipped.
 *      Sum-of-squares order: 16 lanes per head; lane i owns elements [P*i, P*i+P) then
 *      [HD/2+P*i, HD/2+P*i+P) (P = HD/32), summed in that order; butterfly over 16 lanes. */
void orc_qk_norm_rope_kv_write_fp8(uint16_t* q_out, const uint16_t* qkv, const uint16_t* q_norm,
                                   const uint16_t* k_norm, const float* cos_t, const float* sin_t,
                                   const int64_t* positions, const int64_t* slots, uint8_t* k_cache, uint8_t* v_cache,
                                   float* k_scale, float* v_scale, uint16_t* k_dense, uint16_t* v_dense, int64_t T,
                                   int H, int KV, int HD, int BS, int scale_mode, double eps_d) {
    const float eps = (float)eps_d;
    const int n_tasks = H + 2 * KV, HALF = HD / 2, P = HD / 32;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        const int64_t slot = slots[t];
        const int64_t pos = positions[t];
        for (int task = 0; task < n_tasks; ++task) {
            const uint16_t* src = qkv + (t * n_tasks + task) * HD;
            float x[256];
            for (int e = 0; e < HD; ++e) x[e] = orc_bf16_to_f32(src[e]);
            if (task >= H + KV) {                         /* V (fused_ops.cu:125-143) */
                int kvh = task - H - KV;
                float amax = 0.f;
                for (int e = 0; e < HD; ++e) amax = fmaxf(amax, fabsf(x[e]));
                if (v_dense)
                    for (int e = 0; e < HD; ++e) v_dense[(t * KV + kvh) * HD + e] = src[e];
                if (slot < 0) continue;
                float sc = 0.f, inv;
                if (scale_mode == ORC_PER_TOKEN_HEAD) { sc = fmaxf(amax, 1e-8f) / 448.0f; inv = 1.0f / sc; }
                else inv = 1.0f / v_scale[0];
                for (int e = 0; e < HD; ++e) v_cache[(slot * KV + kvh) * HD + e] = orc_e4m3_encode(x[e] * inv);
                if (scale_mode == ORC_PER_TOKEN_HEAD)
                    v_scale[((slot / BS) * KV + kvh) * BS + slot % BS] = sc;
                continue;
            }
            const int is_q = task < H;
            const uint16_t* wn = is_q ? q_norm : k_norm;
            float part[16];
            for (int i = 0; i < 16; ++i) {
                float ss = 0.f;
                for (int j = 0; j < P; ++j) ss = ss + x[P * i + j] * x[P * i + j];
                for (int j = 0; j < P; ++j) ss = ss + x[HALF + P * i + j] * x[HALF + P * i + j];
                part[i] = ss;
            }
            float ss = butterfly_sum(part, 16);
            float inv = 1.0f / sqrtf(ss / (float)HD + eps);
            float n[256], r[256];
            for (int e = 0; e < HD; ++e) n[e] = rbf16(rbf16(x[e] * inv) * orc_bf16_to_f32(wn[e]));
            for (int e = 0; e < HALF; ++e) {              /* neox RoPE (fused_ops.cu:157-166) */
                float c = cos_t[pos * HALF + e], s = sin_t[pos * HALF + e];
                float a = n[e], b = n[e + HALF];
                float ac = a * c, bs = b * s, bc = b * c, as = a * s;
                r[e] = ac - bs;
                r[e + HALF] = bc + as;
            }
            if (is_q) {
                for (int e = 0; e < HD; ++e) q_out[(t * H + task) * HD + e] = orc_f32_to_bf16(r[e]);
                continue;
            }
            int kvh = task - H;                           /* K (fused_ops.cu:175-190) */
            float amax = 0.f;
            for (int e = 0; e < HD; ++e) { r[e] = rbf16(r[e]); amax = fmaxf(amax, fabsf(r[e])); }
            if (k_dense)
                for (int e = 0; e < HD; ++e) k_dense[(t * KV + kvh) * HD + e] = orc_f32_to_bf16(r[e]);
            if (slot < 0) continue;
            float sc = 0.f, sinv;
            if (scale_mode == ORC_PER_TOKEN_HEAD) { sc = fmaxf(amax, 1e-8f) / 448.0f; sinv = 1.0f / sc; }
            else sinv = 1.0f / k_scale[0];
            for (int e = 0; e < HD; ++e) k_cache[(slot * KV + kvh) * HD + e] = orc_e4m3_encode(r[e] * sinv);
            if (scale_mode == ORC_PER_TOKEN_HEAD) k_scale[((slot / BS) * KV + kvh) * BS + slot % BS] = sc;
        }
    }
}

/* ---- Paged FP8 attention: restates paged_attention_fp8_kernel + merge
 *      (kernels/paged_attention.cu:89-393) as one exact softmax per (token, head):
 *        s_j = (q . k_j) * scale * ks_j  (q bf16, k_j decoded e4m3, fp32 dot in element order)
 *        out = bf16( sum_j exp(s_j - max) * vs_j * v_j / sum_j exp(s_j - max) )
 *      over the token's first kv_len keys, key j at slot table[seq][j/BS]*BS + j%BS.
 *      The reference's online/split evaluation is the same quantity up to fp32 reassociation.
 *      kv_len <= 0 gives a zero row (the reference would produce 0/0). Parallel over
 *      (token, kv head) units with OpenMP (the CPU baseline). */
void orc_paged_attention_fp8(uint16_t* out, const uint16_t* q, const uint8_t* k_cache, const uint8_t* v_cache,
                             const float* k_scale, const float* v_scale, const int64_t* block_tables,
                             int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len, int64_t T,
                             int H, int KV, int HD, int BS, int scale_mode, double scale_d) {
    static float lut[256];
    static int lut_ready = 0;
    if (!lut_ready) {
        for (int c = 0; c < 256; ++c) lut[c] = orc_e4m3_decode((uint8_t)c);
        lut_ready = 1;
    }
    const float scale = (float)scale_d;
    const int REP = H / KV;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t u = 0; u < T * KV; ++u) {
        const int64_t t = u / KV;
        const int g = (int)(u % KV);
        int64_t L = token_kv_len[t];
        if (L > table_width * BS) L = table_width * BS;
        if (token_seq[t] < 0) L = 0;                       /* padding token (token_seq -1): zero row */
        if (L <= 0) {
            for (int r = 0; r < REP; ++r)
                for (int d = 0; d < HD; ++d) out[(t * H + g * REP + r) * HD + d] = 0;
            continue;
        }
        const int64_t* table = block_tables + token_seq[t] * table_width;
        for (int r = 0; r < REP; ++r) {
            const int h = g * REP + r;
            float qf[256];
            for (int d = 0; d < HD; ++d) qf[d] = orc_bf16_to_f32(q[(t * H + h) * HD + d]);
            float mx = -INFINITY;
            float acc[256];
            for (int d = 0; d < HD; ++d) acc[d] = 0.f;
            /* pass 1: max score */
            for (int64_t j = 0; j < L; ++j) {
                const int64_t slot = table[j / BS] * BS + j % BS;
                const uint8_t* kr = k_cache + (slot * KV + g) * HD;
                float p8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int d = 0; d < HD; d += 8)
                    for (int i = 0; i < 8; ++i) p8[i] += qf[d + i] * lut[kr[d + i]];
                float dot = ((p8[0] + p8[1]) + (p8[2] + p8[3])) + ((p8[4] + p8[5]) + (p8[6] + p8[7]));
                float ks = scale_mode == ORC_PER_TOKEN_HEAD ? k_scale[((slot / BS) * KV + g) * BS + slot % BS]
                                                            : k_scale[0];
                float s = dot * scale * ks;
                if (s > mx) mx = s;
            }
            /* pass 2: exp-weights and weighted V sum */
            float den = 0.f;
            for (int64_t j = 0; j < L; ++j) {
                const int64_t slot = table[j / BS] * BS + j % BS;
                const uint8_t* kr = k_cache + (slot * KV + g) * HD;
                const uint8_t* vr = v_cache + (slot * KV + g) * HD;
                float p8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int d = 0; d < HD; d += 8)
                    for (int i = 0; i < 8; ++i) p8[i] += qf[d + i] * lut[kr[d + i]];
                float dot = ((p8[0] + p8[1]) + (p8[2] + p8[3])) + ((p8[4] + p8[5]) + (p8[6] + p8[7]));
                int64_t sidx = ((slot / BS) * KV + g) * BS + slot % BS;
                float ks = scale_mode == ORC_PER_TOKEN_HEAD ? k_scale[sidx] : k_scale[0];
                float vs = scale_mode == ORC_PER_TOKEN_HEAD ? v_scale[sidx] : v_scale[0];
                float p = expf(dot * scale * ks - mx);
                den += p;
                float pv = p * vs;
                for (int d = 0; d < HD; ++d) acc[d] += pv * lut[vr[d]];
            }
            for (int d = 0; d < HD; ++d) out[(t * H + h) * HD + d] = orc_f32_to_bf16(acc[d] / den);
        }
    }
}

/* ---- per-token metadata: restates model/model_architecture.cpp:137-147
 *      (searchsorted(cu[1:], t, right) ; slot = table[seq][pos/BS]*BS + pos%BS ; kv_len = pos+1),
 *      with padding tokens (t >= cu[S]) and negative table entries mapped to (-1, -1, 0). */
void orc_token_metadata(const int64_t* cu, int64_t S, const int64_t* positions, int64_t T, const int64_t* tables,
                        int64_t W, int BS, int64_t* token_seq, int64_t* slots, int64_t* kv_len) {
    for (int64_t t = 0; t < T; ++t) {
        int64_t seq = 0;
        while (seq < S && cu[seq + 1] <= t) ++seq;
        int64_t pos = positions[t], slot = -1, so = -1, len = 0;
        if (seq < S && pos >= 0) {
            int64_t b = pos / BS;
            int64_t phys = b < W ? tables[seq * W + b] : -1;
            if (phys >= 0) { slot = phys * BS + pos % BS; so = seq; len = pos + 1; }
        }
        token_seq[t] = so;
        slots[t] = slot;
        kv_len[t] = len;
    }
}

/* ---- SwiGLU: restates kernels/fused_ops.cu:210-219 (silu rounded to the row dtype, then the
 *      product rounded), with g/(1+exp(-g)) evaluated in double (the build's documented order). */
void orc_swiglu(void* out, const void* gu, int64_t N, int I, int dt) {
    for (int64_t r = 0; r < N; ++r)
        for (int i = 0; i < I; ++i) {
            float g = ld(gu, r * 2 * I + i, dt), u = ld(gu, r * 2 * I + I + i, dt);
            float silu = rnd((float)((double)g / (1.0 + exp(-(double)g))), dt);
            st(out, r * I + i, dt, silu * u);
        }
}

/* ---- Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
 *      SC'11): 10 rounds of the 4x32 bijection with multipliers 0xD2511F53, 0xCD9E8D57 and the key
 *      schedule k += (0x9E3779B9, 0xBB67AE85). Used by the sampler of kernels/fused_ops.cu:287-299. */
void orc_philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int i = 0; i < 10; ++i) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c[0], p1 = (uint64_t)0xCD9E8D57u * c[2];
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1, n3 = (uint32_t)p0;
        c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
}

/* ---- token sampler: restates kernels/fused_ops.cu:309-365 as a plain scan in index order:
 *      greedy (temp <= 0) = arg-max, lowest index on ties; otherwise Gumbel-max with
 *      u = ((r >> 8) + 0.5) / 2^24 from Philox counter (j/4, row, offset) and the score
 *      x/temp - log(max(-log u, 1e-10)) evaluated in double, rounded to float. logits are f32
 *      (dt == ORC_F32) or bf16 bit patterns. */
void orc_sample_tokens(int64_t* out, const void* logits, int dt, const int64_t* rows, const float* temps, int64_t R,
                       int V, uint64_t seed, uint64_t offset) {
    for (int64_t r = 0; r < R; ++r) {
        int64_t src = rows ? rows[r] : r;
        float temp = temps ? temps[r] : 0.f;
        int greedy = !(temp > 0.f);
        float inv_t = 1.0f / fmaxf(temp, 1e-5f);
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        uint32_t c[4] = {0, 0, 0, 0};
        for (int j = 0; j < V; ++j) {
            float x = ld(logits, src * (int64_t)V + j, dt == ORC_F32 ? ORC_F32 : ORC_BF16), s = x;
            if (!greedy) {
                if ((j & 3) == 0) {
                    c[0] = (uint32_t)(j >> 2); c[1] = (uint32_t)r;
                    c[2] = (uint32_t)offset; c[3] = (uint32_t)(offset >> 32);
                    orc_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
                }
                float u = ((float)(c[j & 3] >> 8) + 0.5f) * (1.0f / 16777216.0f);
                double e = fmax(-log((double)u), 1e-10);
                s = (float)((double)x * inv_t - log(e));
            }
            /* kernels/fused_ops.cu:303: larger, or equal with a lower index (so an all -inf row
             * gives index 0; NaN never wins) */
            if (s > bv || (s == bv && j < bi)) { bv = s; bi = j; }
        }
        out[r] = bi;
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
