// FP8-e4m3 paged decode attention for gfx950 (CDNA4), one wavefront per
// (query token, kv head, split).
//
// Reference semantics: kernels/paged_attention.cu:89-393 (per-token causal length, GQA heads
// sharing each K/V row, per-(token,head) FP8 scales, online softmax in fp32, split-K partials
// merged with a log-sum-exp combine). The decomposition here is designed for wave64:
//
//   * lane = (grp, sub): grp = lane/8 picks one of 8 keys of a step, sub = lane%8 owns a
//     16-byte (HD=128) or 8-byte (HD=64) slice of the 128-byte K and V rows, so each load
//     instruction covers 8 full key rows (8 x 128 B cache lines, no partial lines);
//   * a tile is 4 steps = 32 keys; tile t+1's K/V/scale loads are issued before tile t is
//     computed (register double buffer) to keep >= 8 KB in flight per wave;
//   * FP8 -> f32 with the hardware OCP converter (v_cvt_pk_f32_fp8, exact for finite codes);
//   * q.k partial dots reduce over the 8 lanes of a key with DPP (quad_perm, half-mirror);
//   * softmax in base 2 (scale*log2(e) folded into q) with a lazy running max: the
//     accumulator is only rescaled when a tile's max exceeds the running max by 8 (p <= 256),
//     which is exact because the final normalisation uses the same max for l and acc;
//   * the running max is wave-uniform, so the cross-key-group combine at the end is a plain
//     sum (no per-group rescale);
//   * split-K: each token's context is cut into chunks of split_tiles*32 keys; a token with one
//     chunk writes bf16 directly, others write (acc, m, l) partials for the merge kernel.
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>

#include "cvh_device.h"

namespace cvh {
namespace {

constexpr int kTileKeys = 32;      // keys per wave per tile (4 steps x 8 key groups)
constexpr int kSteps = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;   // log2 units: stale max tolerated up to p = 2^8

template <int HD> struct KvVec;
template <> struct KvVec<128> {
    using T = uint4;
    static constexpr int kElems = 16;
    static __device__ __forceinline__ void to_f32(const uint4& u, float (&f)[16]) {
        fp8x4_to_f32(u.x, f + 0);
        fp8x4_to_f32(u.y, f + 4);
        fp8x4_to_f32(u.z, f + 8);
        fp8x4_to_f32(u.w, f + 12);
    }
};
template <> struct KvVec<64> {
    using T = uint2;
    static constexpr int kElems = 8;
    static __device__ __forceinline__ void to_f32(const uint2& u, float (&f)[8]) {
        fp8x4_to_f32(u.x, f + 0);
        fp8x4_to_f32(u.y, f + 4);
    }
};

// Sum over the 8 lanes of a key group (lanes 8k..8k+7); result in every lane of the group.
__device__ __forceinline__ float group8_sum(float v) {
    v = v + dpp_xor1(v);
    v = v + dpp_xor2(v);
    v = v + dpp_half_mirror(v);
    return v;
}
// xor-8 exchange inside a row of 16 (row_ror:8).
__device__ __forceinline__ float dpp_ror8(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
}
// Combine the 8 key groups (sum), result in every lane; lanes with equal sub get equal values.
__device__ __forceinline__ float across_groups_sum(float v) {
    v = v + dpp_ror8(v);
    v = v + shfl_xor(v, 16);
    v = v + shfl_xor(v, 32);
    return v;
}
// Max over the whole wave of a value that is already uniform inside each key group.
__device__ __forceinline__ float across_groups_max(float v) {
    v = fmaxf(v, dpp_ror8(v));
    v = fmaxf(v, shfl_xor(v, 16));
    v = fmaxf(v, shfl_xor(v, 32));
    return v;
}

template <int HD, int REP, int SM>
__global__ __launch_bounds__(64) void paged_decode_kernel(
        uint16_t* __restrict__ out, float* __restrict__ part_acc, float* __restrict__ part_ml,
        const uint16_t* __restrict__ q, const uint8_t* __restrict__ k_cache, const uint8_t* __restrict__ v_cache,
        const float* __restrict__ k_scale, const float* __restrict__ v_scale, const int64_t* __restrict__ block_tables,
        int64_t table_width, const int64_t* __restrict__ token_seq, const int64_t* __restrict__ token_kv_len,
        int n_kv, int log2_bs, int split_tiles, int max_splits, float q_scale) {
    using V = KvVec<HD>;
    using VT = typename V::T;
    constexpr int E = V::kElems;                 // elements of HD owned per lane
    const int t = blockIdx.x;
    const int g = blockIdx.y;
    const int split = blockIdx.z;
    const int lane = threadIdx.x;
    const int grp = lane >> 3;
    const int sub = lane & 7;
    const int H = n_kv * REP;

    int64_t kv_len = token_kv_len[t];
    const int64_t cap = table_width << log2_bs;  // never read past the block table row
    if (kv_len > cap) kv_len = cap;
    if (kv_len <= 0) {                           // empty context: zero output (reference: 0/0)
        if (split == 0) {
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                uint16_t* o = out + ((int64_t)t * H + g * REP + r) * HD;
                for (int d = lane; d < HD; d += 64) o[d] = 0;
            }
        }
        return;
    }
    const int64_t ntiles = (kv_len + kTileKeys - 1) / kTileKeys;
    const int64_t nsplit = (ntiles + split_tiles - 1) / split_tiles;
    if (split >= nsplit) return;
    const int64_t tile_begin = (int64_t)split * split_tiles;
    const int64_t tile_end = min(ntiles, tile_begin + split_tiles);
    const int64_t* table = block_tables + token_seq[t] * table_width;
    const int64_t row_bytes = (int64_t)n_kv * HD;    // bytes of one cache slot (all kv heads)
    const int bs_mask = (1 << log2_bs) - 1;

    // ---- q slice for the REP heads of this kv head, pre-scaled by scale*log2(e) [*k_scale]
    const float qsc = (SM == CVH_SCALE_PER_TENSOR) ? q_scale * k_scale[0] : q_scale;
    float qf[REP][E];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const uint16_t* qr = q + ((int64_t)t * H + g * REP + r) * HD + sub * E;
#pragma unroll
        for (int c = 0; c < E / 8; ++c) {
            const uint4 u = reinterpret_cast<const uint4*>(qr)[c];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qf[r][c * 8 + 2 * i] = bf16_bits_to_f32(w[i] & 0xffffu) * qsc;
                qf[r][c * 8 + 2 * i + 1] = bf16_bits_to_f32(w[i] >> 16) * qsc;
            }
        }
    }

    float m[REP], l[REP], acc[REP][E];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[r][e] = 0.f;
    }

    // ---- tile loader: K/V slices and per-key scales for keys tile*32 + 8*s + grp
    struct Tile {
        VT k[kSteps], v[kSteps];
        float ks[kSteps], vs[kSteps];
    };
    auto load_tile = [&](int64_t tile, Tile& tl) {
        const int64_t p0 = tile * kTileKeys;
        const int64_t last = min(p0 + kTileKeys - 1, kv_len - 1);
        const int64_t bi_lo = p0 >> log2_bs, bi_hi = last >> log2_bs;   // block_size >= 16: <= 2 blocks
        const int64_t ph_lo = max(table[bi_lo], int64_t{0});
        const int64_t ph_hi = max(table[bi_hi], int64_t{0});
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int64_t pos = min(p0 + 8 * s + grp, kv_len - 1);         // masked keys re-read a valid row
            const int64_t ph = ((pos >> log2_bs) == bi_lo) ? ph_lo : ph_hi;
            const int off = static_cast<int>(pos & bs_mask);
            const int64_t byte = (((ph << log2_bs) + off) * row_bytes) + g * HD + sub * E;
            tl.k[s] = *reinterpret_cast<const VT*>(k_cache + byte);
            tl.v[s] = *reinterpret_cast<const VT*>(v_cache + byte);
            if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) {
                const int64_t sidx = ((ph * n_kv + g) << log2_bs) + off;
                tl.ks[s] = k_scale[sidx];
                tl.vs[s] = v_scale[sidx];
            } else {
                tl.ks[s] = 1.f;
                tl.vs[s] = 1.f;
            }
        }
    };

    auto compute_tile = [&](int64_t tile, const Tile& tl) {
        const int64_t p0 = tile * kTileKeys;
        float sc[REP][kSteps];
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            float kf[E];
            V::to_f32(tl.k[s], kf);
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) d += qf[r][e] * kf[e];
                sc[r][s] = d;
            }
        }
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const bool valid = (p0 + 8 * s + grp) < kv_len;
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                const float d = group8_sum(sc[r][s]);
                sc[r][s] = valid ? d * tl.ks[s] : -INFINITY;
            }
        }
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            float mt = fmaxf(fmaxf(sc[r][0], sc[r][1]), fmaxf(sc[r][2], sc[r][3]));
            mt = across_groups_max(mt);
            if (mt > m[r] + kRescaleThreshold) {
                const float c = exp2f(m[r] - mt);
                l[r] *= c;
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] *= c;
                m[r] = mt;
            }
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const float p = exp2f(sc[r][s] - m[r]);
                l[r] += p;
                sc[r][s] = p * tl.vs[s];
            }
        }
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            float vf[E];
            V::to_f32(tl.v[s], vf);
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                const float w = sc[r][s];
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] += w * vf[e];
            }
        }
    };

    // Register double buffer, unrolled by two so no tile is ever copied between buffers.
    Tile ta, tb;
    load_tile(tile_begin, ta);
    for (int64_t tile = tile_begin; tile < tile_end; tile += 2) {
        if (tile + 1 < tile_end) load_tile(tile + 1, tb);
        compute_tile(tile, ta);
        if (tile + 1 >= tile_end) break;
        if (tile + 2 < tile_end) load_tile(tile + 2, ta);
        compute_tile(tile + 1, tb);
    }

    // ---- combine the 8 key groups (shared running max => plain sums)
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        // l is uniform inside a group (every lane of a group sums the same p's); sum over groups.
        l[r] = across_groups_sum(l[r]);
#pragma unroll
        for (int e = 0; e < E; ++e) acc[r][e] = across_groups_sum(acc[r][e]);
    }
    if (grp != 0) return;

    const float v_fin = (SM == CVH_SCALE_PER_TENSOR) ? v_scale[0] : 1.f;
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const int64_t head = (int64_t)t * H + g * REP + r;
        if (nsplit == 1) {
            const float f = v_fin / l[r];
            uint16_t* o = out + head * HD + sub * E;
#pragma unroll
            for (int c = 0; c < E / 8; ++c) {
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    w[i] = f32_to_bf16_bits(acc[r][c * 8 + 2 * i] * f) |
                           (uint32_t(f32_to_bf16_bits(acc[r][c * 8 + 2 * i + 1] * f)) << 16);
                }
                reinterpret_cast<uint4*>(o)[c] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        } else {
            const int64_t slot = head * max_splits + split;
            float* pa = part_acc + slot * HD + sub * E;
#pragma unroll
            for (int c = 0; c < E / 4; ++c)
                reinterpret_cast<float4*>(pa)[c] =
                        make_float4(acc[r][4 * c], acc[r][4 * c + 1], acc[r][4 * c + 2], acc[r][4 * c + 3]);
            if (sub == 0) reinterpret_cast<float2*>(part_ml)[slot] = make_float2(m[r], l[r]);
        }
    }
}

// Log-sum-exp merge of the split partials (reference: kernels/paged_attention.cu:361-393).
// One wave per (token, head); lane d handles dims d and d+64.
template <int HD, int SM>
__global__ __launch_bounds__(64) void paged_merge_kernel(uint16_t* __restrict__ out, const float* __restrict__ part_acc,
                                                         const float* __restrict__ part_ml,
                                                         const int64_t* __restrict__ token_kv_len,
                                                         const float* __restrict__ v_scale, int64_t table_width,
                                                         int log2_bs, int n_heads, int split_tiles, int max_splits) {
    const int h = blockIdx.x;
    const int t = blockIdx.y;
    int64_t kv_len = token_kv_len[t];
    const int64_t cap = table_width << log2_bs;
    if (kv_len > cap) kv_len = cap;
    if (kv_len <= 0) return;
    const int64_t ntiles = (kv_len + kTileKeys - 1) / kTileKeys;
    const int nsplit = static_cast<int>((ntiles + split_tiles - 1) / split_tiles);
    if (nsplit <= 1) return;
    const int64_t head = (int64_t)t * n_heads + h;
    const float2* ml = reinterpret_cast<const float2*>(part_ml) + head * max_splits;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ml[s].x);
    float L = 0.f;
    constexpr int PER = HD / 64;
    float A[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) A[i] = 0.f;
    for (int s = 0; s < nsplit; ++s) {
        const float2 v = ml[s];
        const float c = exp2f(v.x - M);
        L += v.y * c;
        const float* pa = part_acc + (head * max_splits + s) * HD;
#pragma unroll
        for (int i = 0; i < PER; ++i) A[i] += pa[threadIdx.x + 64 * i] * c;
    }
    const float f = ((SM == CVH_SCALE_PER_TENSOR) ? v_scale[0] : 1.f) / L;
    uint16_t* o = out + head * HD;
#pragma unroll
    for (int i = 0; i < PER; ++i) o[threadIdx.x + 64 * i] = f32_to_bf16_bits(A[i] * f);
}

int ilog2_pow2(int64_t v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int l = 0;
    while ((int64_t{1} << l) < v) ++l;
    return l;
}

int64_t max_context(int64_t table_width, int block_size) { return table_width * block_size; }

int auto_split_tokens(int64_t num_tokens, int n_kv, int64_t table_width, int block_size) {
    // Aim for >= 2048 waves (8 per CU on 256 CUs) when the longest possible context allows it,
    // with chunks no shorter than 64 keys; 512-key chunks otherwise (64 KB of K+V per wave).
    const int64_t ctx = std::max<int64_t>(1, max_context(table_width, block_size));
    int chunk = 512;
    while (chunk > 64 && num_tokens * n_kv * ((ctx + chunk - 1) / chunk) < 2048) chunk >>= 1;
    return chunk;
}

bool valid_split(int split_tokens) { return split_tokens >= 64 && split_tokens % kTileKeys == 0; }

int64_t num_splits_max(int64_t table_width, int block_size, int split_tokens) {
    const int64_t ctx = max_context(table_width, block_size);
    return std::max<int64_t>(1, (ctx + split_tokens - 1) / split_tokens);
}

size_t ws_bytes(int64_t T, int H, int HD, int64_t splits) {
    if (splits <= 1) return 0;
    return static_cast<size_t>(T) * H * splits * (HD + 2) * sizeof(float);
}

template <int HD, int REP, int SM>
void launch(dim3 grid, hipStream_t s, void* out, float* pa, float* pm, const void* q, const uint8_t* kc,
            const uint8_t* vc, const float* ks, const float* vs, const int64_t* bt, int64_t tw, const int64_t* ts,
            const int64_t* tl, int n_kv, int lg, int split_tiles, int max_splits, float qs) {
    paged_decode_kernel<HD, REP, SM><<<grid, 64, 0, s>>>(static_cast<uint16_t*>(out), pa, pm,
                                                         static_cast<const uint16_t*>(q), kc, vc, ks, vs, bt, tw, ts,
                                                         tl, n_kv, lg, split_tiles, max_splits, qs);
}

template <int HD, int SM>
bool launch_rep(int rep, dim3 grid, hipStream_t s, void* out, float* pa, float* pm, const void* q,
                const uint8_t* kc, const uint8_t* vc, const float* ks, const float* vs, const int64_t* bt, int64_t tw,
                const int64_t* ts, const int64_t* tl, int n_kv, int lg, int st, int ms, float qs) {
    switch (rep) {
        case 1: launch<HD, 1, SM>(grid, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        case 2: launch<HD, 2, SM>(grid, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        case 4: launch<HD, 4, SM>(grid, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        case 8: launch<HD, 8, SM>(grid, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        default: return false;
    }
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_paged_attention_split_tokens(int64_t num_tokens, int n_kv_heads, int64_t table_width,
                                                int block_size) {
    if (num_tokens <= 0 || n_kv_heads <= 0 || table_width <= 0 || block_size <= 0) return 512;
    return cvh::auto_split_tokens(num_tokens, n_kv_heads, table_width, block_size);
}

extern "C" size_t cvh_paged_attention_workspace_bytes(int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                                      int64_t table_width, int block_size, int split_tokens) {
    if (num_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width <= 0 || block_size <= 0) return 0;
    if (split_tokens == 0) split_tokens = cvh::auto_split_tokens(num_tokens, n_kv_heads, table_width, block_size);
    if (!cvh::valid_split(split_tokens)) return 0;
    return cvh::ws_bytes(num_tokens, n_heads, head_dim,
                                cvh::num_splits_max(table_width, block_size, split_tokens));
}

extern "C" int cvh_paged_attention_fp8_ex(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                          const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                          int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                          int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                          int block_size, int scale_mode, double scale, int split_tokens,
                                          void* workspace, size_t workspace_bytes, cvh_stream_t stream) {
    using namespace cvh;
    if (num_tokens < 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width < 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!out || !q || !k_cache || !v_cache || !k_scale || !v_scale || !block_tables || !token_seq || !token_kv_len)
        return CVH_ERR_INVALID_ARG;
    if (table_width == 0) return CVH_ERR_INVALID_ARG;
    if (n_heads % n_kv_heads != 0) return CVH_ERR_UNSUPPORTED;
    const int rep = n_heads / n_kv_heads;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return CVH_ERR_UNSUPPORTED;
    const int lg = ilog2_pow2(block_size);
    if (lg < 4 || lg > 12) return CVH_ERR_UNSUPPORTED;
    if (head_dim != 64 && head_dim != 128) return CVH_ERR_UNSUPPORTED;
    if (scale_mode != CVH_SCALE_PER_TOKEN_HEAD && scale_mode != CVH_SCALE_PER_TENSOR) return CVH_ERR_UNSUPPORTED;
    if (num_tokens > 0x7fffffff || n_kv_heads > 65535) return CVH_ERR_UNSUPPORTED;
    if (split_tokens == 0) split_tokens = auto_split_tokens(num_tokens, n_kv_heads, table_width, block_size);
    if (!valid_split(split_tokens)) return CVH_ERR_INVALID_ARG;
    const int64_t ms = num_splits_max(table_width, block_size, split_tokens);
    if (ms > 65535) return CVH_ERR_UNSUPPORTED;
    const size_t need = ws_bytes(num_tokens, n_heads, head_dim, ms);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return CVH_ERR_WORKSPACE;
    float* pa = static_cast<float*>(workspace);
    float* pm = need > 0 ? pa + static_cast<size_t>(num_tokens) * n_heads * ms * head_dim : nullptr;

    // The softmax scale is folded into q with log2(e) (base-2 softmax); a per-tensor K scale is a
    // device float, so the kernel folds it into q after reading it.
    const float qs = static_cast<float>(scale) * kLog2e;
    auto s = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(num_tokens), static_cast<unsigned>(n_kv_heads), static_cast<unsigned>(ms));
    const int st = split_tokens / kTileKeys;
    bool ok;
    if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD) {
        ok = head_dim == 128 ? launch_rep<128, CVH_SCALE_PER_TOKEN_HEAD>(rep, grid, s, out, pa, pm, q, k_cache, v_cache,
                                                                        k_scale, v_scale, block_tables, table_width,
                                                                        token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                        static_cast<int>(ms), qs)
                             : launch_rep<64, CVH_SCALE_PER_TOKEN_HEAD>(rep, grid, s, out, pa, pm, q, k_cache, v_cache,
                                                                       k_scale, v_scale, block_tables, table_width,
                                                                       token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                       static_cast<int>(ms), qs);
    } else {
        ok = head_dim == 128 ? launch_rep<128, CVH_SCALE_PER_TENSOR>(rep, grid, s, out, pa, pm, q, k_cache, v_cache,
                                                                    k_scale, v_scale, block_tables, table_width,
                                                                    token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                    static_cast<int>(ms), qs)
                             : launch_rep<64, CVH_SCALE_PER_TENSOR>(rep, grid, s, out, pa, pm, q, k_cache, v_cache,
                                                                   k_scale, v_scale, block_tables, table_width,
                                                                   token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                   static_cast<int>(ms), qs);
    }
    if (!ok) return CVH_ERR_UNSUPPORTED;
    if (hipGetLastError() != hipSuccess) return CVH_ERR_LAUNCH;
    if (ms > 1) {
        const dim3 mgrid(static_cast<unsigned>(n_heads), static_cast<unsigned>(num_tokens));
        auto* o = static_cast<uint16_t*>(out);
        if (head_dim == 128) {
            if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
                paged_merge_kernel<128, CVH_SCALE_PER_TOKEN_HEAD><<<mgrid, 64, 0, s>>>(o, pa, pm, token_kv_len, v_scale, table_width, lg, n_heads, st, static_cast<int>(ms));
            else
                paged_merge_kernel<128, CVH_SCALE_PER_TENSOR><<<mgrid, 64, 0, s>>>(o, pa, pm, token_kv_len, v_scale, table_width, lg, n_heads, st, static_cast<int>(ms));
        } else {
            if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
                paged_merge_kernel<64, CVH_SCALE_PER_TOKEN_HEAD><<<mgrid, 64, 0, s>>>(o, pa, pm, token_kv_len, v_scale, table_width, lg, n_heads, st, static_cast<int>(ms));
            else
                paged_merge_kernel<64, CVH_SCALE_PER_TENSOR><<<mgrid, 64, 0, s>>>(o, pa, pm, token_kv_len, v_scale, table_width, lg, n_heads, st, static_cast<int>(ms));
        }
        if (hipGetLastError() != hipSuccess) return CVH_ERR_LAUNCH;
    }
    return CVH_OK;
}

extern "C" int cvh_paged_attention_fp8(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                       const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                       int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                       int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                       int scale_mode, double scale, void* workspace, size_t workspace_bytes,
                                       cvh_stream_t stream) {
    return cvh_paged_attention_fp8_ex(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq,
                                      token_kv_len, num_tokens, n_heads, n_kv_heads, head_dim, block_size, scale_mode,
                                      scale, 0, workspace, workspace_bytes, stream);
}
