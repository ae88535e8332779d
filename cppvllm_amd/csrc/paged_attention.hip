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
//   * K/V loads are non-temporal (streamed once), and a workgroup carries the waves of 4
//     consecutive kv heads of one (token, split) so whole 1 KB slot rows are read together;
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
#include <type_traits>

#include "cvh_device.h"

namespace cvh {
namespace {

constexpr int kTileKeys = 32;      // keys per wave per tile (4 steps x 8 key groups)
constexpr int kSteps = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;   // log2 units: stale max tolerated up to p = 2^8
constexpr float kMinusHuge = -1e30f;

// K/V rows and scales go through raw buffer loads: the descriptor's record count bounds every
// access, so a tile that must not be read (the prefetch issued past a split's last tile) is given
// a zero-size descriptor and returns zeros without touching memory. All K/V/scale loads carry the
// non-temporal hint: each byte is read once per launch, so it should not displace reusable lines
// (block tables, q, partials) in L2 / MALL (measured: -8% kernel time at config 3).
constexpr int kBufferWord3 = 0x00020000;      // raw buffer, 32-bit data format (gfx9 encoding)
constexpr int kNonTemporal = 2;               // cache-policy bits of the load: nt
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}
template <typename VT> __device__ __forceinline__ VT buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ uint4 buf_load<uint4>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNonTemporal);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ uint2 buf_load<uint2>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNonTemporal);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kNonTemporal));
}

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
// Exchange across rows of 16 / halves of 32 lanes with the gfx950 permlane swaps (no LDS, no
// LGKM counter traffic): with both operands = v, the pair returned holds, per lane, its own
// value and its xor-16 (resp. xor-32) partner's value.
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Combine the 8 key groups (sum), result in every lane; lanes with equal sub get equal values.
__device__ __forceinline__ float across_groups_sum(float v) {
    v = v + dpp_xor8(v);
    v = xor16_sum(v);
    return xor32_sum(v);
}
// Max over the whole wave of a value that is already uniform inside each key group.
__device__ __forceinline__ float across_groups_max(float v) {
    v = fmaxf(v, dpp_xor8(v));
    v = xor16_max(v);
    return xor32_max(v);
}

// ONE_BLOCK: block_size >= 32, so a 32-key tile never straddles two cache blocks and one
// block-table lookup serves the whole tile. Otherwise (block_size 16) each 8-key step still lies
// in a single block, looked up per step. Lookups are wave-uniform scalar loads; the per-lane
// address is a 32-bit offset from a scalar block base.
template <int HD, int REP, int SM, bool ONE_BLOCK>
__global__ __launch_bounds__(256) void paged_decode_kernel(
        uint16_t* __restrict__ out, float* __restrict__ part_acc, float* __restrict__ part_ml,
        const uint16_t* __restrict__ q, const uint8_t* __restrict__ k_cache, const uint8_t* __restrict__ v_cache,
        const float* __restrict__ k_scale, const float* __restrict__ v_scale, const int64_t* __restrict__ block_tables,
        int64_t table_width, const int64_t* __restrict__ token_seq, const int64_t* __restrict__ token_kv_len,
        int n_kv, int log2_bs, int split_tiles, int max_splits, float q_scale) {
    using V = KvVec<HD>;
    using VT = typename V::T;
    constexpr int E = V::kElems;                 // elements of HD owned per lane
    // A workgroup holds the waves of (blockDim.x/64) consecutive kv heads of one (token, split):
    // together they read whole slot rows, so the HBM pages they touch are read at the same time.
    const int t = blockIdx.x;
    // wave-uniform by construction; readfirstlane tells the compiler so (scalar descriptors)
    const int g = __builtin_amdgcn_readfirstlane(blockIdx.y * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const int split = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int grp = lane >> 3;
    const int sub = lane & 7;
    const int H = n_kv * REP;

    int64_t kv64 = token_kv_len[t];
    const int64_t cap = table_width << log2_bs;  // never read past the block table row
    if (kv64 > cap) kv64 = cap;
    if (kv64 <= 0) {                             // empty context: zero output (reference: 0/0)
        if (split == 0) {
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                uint16_t* o = out + ((int64_t)t * H + g * REP + r) * HD;
                for (int d = lane; d < HD; d += 64) o[d] = 0;
            }
        }
        return;
    }
    const int kv_len = static_cast<int>(kv64);   // the host limits table_width*block_size < 2^31
    const int ntiles = (kv_len + kTileKeys - 1) / kTileKeys;
    const int nsplit = (ntiles + split_tiles - 1) / split_tiles;
    if (split >= nsplit) return;
    const int tile_begin = split * split_tiles;
    const int tile_end = min(ntiles, tile_begin + split_tiles);
    const int64_t* table = block_tables + token_seq[t] * table_width;
    const uint32_t row_bytes = static_cast<uint32_t>(n_kv) * HD;    // bytes of one slot (all kv heads)
    const int64_t blk_bytes = static_cast<int64_t>(row_bytes) << log2_bs;
    const int bs_mask = (1 << log2_bs) - 1;
    const uint32_t lane_col = g * HD + sub * E;  // byte column of this lane inside a slot row

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

    // Running max per key group (lanes 8k..8k+7 agree on it): no cross-group exchange per tile.
    // Starts at a finite floor so that a group whose keys are all masked gives exp2(-inf) = 0.
    float m[REP], l[REP], acc[REP][E];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        m[r] = kMinusHuge;
        l[r] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[r][e] = 0.f;
    }

    // ---- tile loader: K/V slices and per-key scales for keys tile*32 + 8*s + grp.
    // Keys past kv_len (last tile only) are clamped to key kv_len-1: a valid, finite row whose
    // score is masked, so no garbage (possibly NaN) cache byte ever reaches the accumulator.
    struct Tile {
        VT k[kSteps], v[kSteps];
        float ks[kSteps], vs[kSteps];
    };
    // Physical blocks of a tile: `lo` for its first 16 keys, `hi` for the last 16 (equal unless
    // block_size == 16). Both wave-uniform (scalar loads); looked up one tile ahead of use.
    struct Phys {
        int64_t lo, hi;
    };
    auto lookup = [&](int tile) -> Phys {
        tile = min(tile, tile_end - 1);
        const int p0 = tile * kTileKeys;
        const int64_t lo = max(table[p0 >> log2_bs], int64_t{0});
        if constexpr (ONE_BLOCK) return {lo, lo};
        const int64_t hi = max(table[min(p0 + 16, kv_len - 1) >> log2_bs], int64_t{0});
        return {lo, hi};
    };
    // live = false: the prefetch past the split's last tile; zero-size descriptors, no traffic.
    const uint32_t blk_bytes32 = static_cast<uint32_t>(blk_bytes);
    const uint32_t srow_bytes = 4u << log2_bs;                      // scale row of one (block, head)
    auto load_tile = [&](int tile, Tile& tl, Phys ph2, bool live) {
        const int p0 = tile * kTileKeys;
        const uint32_t lv = static_cast<uint32_t>(live);               // arithmetic, not a branch
        const uint32_t kv_rec = blk_bytes32 * lv, s_rec = srow_bytes * lv;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int64_t ph = (ONE_BLOCK || s < 2) ? ph2.lo : ph2.hi;
            const int pos = min(p0 + 8 * s + grp, kv_len - 1);
            const uint32_t in_blk = static_cast<uint32_t>(pos & bs_mask);
            const uint32_t off = in_blk * row_bytes + lane_col;
            const __amdgpu_buffer_rsrc_t kr = make_rsrc(k_cache + ph * blk_bytes, kv_rec);
            const __amdgpu_buffer_rsrc_t vr = make_rsrc(v_cache + ph * blk_bytes, kv_rec);
            tl.k[s] = buf_load<VT>(kr, off);
            tl.v[s] = buf_load<VT>(vr, off);
            if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) {
                const int64_t sbase = (ph * n_kv + g) << log2_bs;
                const __amdgpu_buffer_rsrc_t ksr = make_rsrc(k_scale + sbase, s_rec);
                const __amdgpu_buffer_rsrc_t vsr = make_rsrc(v_scale + sbase, s_rec);
                tl.ks[s] = buf_load_f32(ksr, in_blk * 4u);
                tl.vs[s] = buf_load_f32(vsr, in_blk * 4u);
            } else {
                tl.ks[s] = 1.f;
                tl.vs[s] = 1.f;
            }
        }
    };

    auto compute = [&](int tile, const Tile& tl) {
        const int p0 = tile * kTileKeys;
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
                float d = group8_sum(sc[r][s]);
                if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) d *= tl.ks[s];
                sc[r][s] = valid ? d : -INFINITY;
            }
        }
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float mt = fmaxf(fmaxf(sc[r][0], sc[r][1]), fmaxf(sc[r][2], sc[r][3]));
            const bool need = mt > m[r] + kRescaleThreshold;    // per key group
            if (__builtin_amdgcn_ballot_w64(need) != 0) {      // wave-uniform; rare after tile 0
                const float mn = need ? mt : m[r];
                const float c = __builtin_amdgcn_exp2f(m[r] - mn);
                l[r] *= c;
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] *= c;
                m[r] = mn;
            }
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const float p = __builtin_amdgcn_exp2f(sc[r][s] - m[r]);
                l[r] += p;
                if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) sc[r][s] = p * tl.vs[s];
                else sc[r][s] = p;
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

    // Register double buffer, unrolled by two so no tile is ever copied between buffers; the
    // block-table lookup runs one tile ahead of the loads that use it. The prefetch is issued
    // unconditionally (past the end with zero-size descriptors) so that it sits in straight-line
    // code and the wait before each compute only covers the tile it consumes.
    Tile ta, tb;
    Phys pa_ = lookup(tile_begin);
    Phys pb_ = lookup(tile_begin + 1);
    load_tile(tile_begin, ta, pa_, true);
    for (int tile = tile_begin;; tile += 2) {
        load_tile(min(tile + 1, tile_end - 1), tb, pb_, tile + 1 < tile_end);
        pa_ = lookup(tile + 2);
        compute(tile, ta);
        if (tile + 1 >= tile_end) break;
        load_tile(min(tile + 2, tile_end - 1), ta, pa_, tile + 2 < tile_end);
        pb_ = lookup(tile + 3);
        compute(tile + 1, tb);
        if (tile + 2 >= tile_end) break;
    }

    // ---- combine the 8 key groups: rescale each to the wave max, then sum
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const float M = across_groups_max(m[r]);
        const float c = __builtin_amdgcn_exp2f(m[r] - M);
        m[r] = M;
        // l is uniform inside a group (every lane of a group sums the same p's); sum over groups.
        l[r] = across_groups_sum(l[r] * c);
#pragma unroll
        for (int e = 0; e < E; ++e) acc[r][e] = across_groups_sum(acc[r][e] * c);
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
void launch(dim3 grid, int threads, hipStream_t s, void* out, float* pa, float* pm, const void* q, const uint8_t* kc,
            const uint8_t* vc, const float* ks, const float* vs, const int64_t* bt, int64_t tw, const int64_t* ts,
            const int64_t* tl, int n_kv, int lg, int split_tiles, int max_splits, float qs) {
    if (lg >= 5)
        paged_decode_kernel<HD, REP, SM, true><<<grid, threads, 0, s>>>(static_cast<uint16_t*>(out), pa, pm,
                                                                   static_cast<const uint16_t*>(q), kc, vc, ks, vs, bt,
                                                                   tw, ts, tl, n_kv, lg, split_tiles, max_splits, qs);
    else
        paged_decode_kernel<HD, REP, SM, false><<<grid, threads, 0, s>>>(static_cast<uint16_t*>(out), pa, pm,
                                                                    static_cast<const uint16_t*>(q), kc, vc, ks, vs,
                                                                    bt, tw, ts, tl, n_kv, lg, split_tiles, max_splits,
                                                                    qs);
}

template <int HD, int SM>
bool launch_rep(int rep, dim3 grid, int threads, hipStream_t s, void* out, float* pa, float* pm, const void* q,
                const uint8_t* kc, const uint8_t* vc, const float* ks, const float* vs, const int64_t* bt, int64_t tw,
                const int64_t* ts, const int64_t* tl, int n_kv, int lg, int st, int ms, float qs) {
    switch (rep) {
        case 1: launch<HD, 1, SM>(grid, threads, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        case 2: launch<HD, 2, SM>(grid, threads, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        case 4: launch<HD, 4, SM>(grid, threads, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
        case 8: launch<HD, 8, SM>(grid, threads, s, out, pa, pm, q, kc, vc, ks, vs, bt, tw, ts, tl, n_kv, lg, st, ms, qs); return true;
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

namespace cvh {
namespace {
enum Phase { kPhaseSplit = 1, kPhaseMerge = 2, kPhaseBoth = 3 };

int paged_attention(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache, const float* k_scale,
                    const float* v_scale, const int64_t* block_tables, int64_t table_width, const int64_t* token_seq,
                    const int64_t* token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                    int block_size, int scale_mode, double scale, int split_tokens, void* workspace,
                    size_t workspace_bytes, cvh_stream_t stream, int phase) {
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
    if (table_width > (int64_t{0x7fffffff} >> lg)) return CVH_ERR_UNSUPPORTED;   // contexts < 2^31 keys
    const size_t need = ws_bytes(num_tokens, n_heads, head_dim, ms);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return CVH_ERR_WORKSPACE;
    float* pa = static_cast<float*>(workspace);
    float* pm = need > 0 ? pa + static_cast<size_t>(num_tokens) * n_heads * ms * head_dim : nullptr;

    // The softmax scale is folded into q with log2(e) (base-2 softmax); a per-tensor K scale is a
    // device float, so the kernel folds it into q after reading it.
    const float qs = static_cast<float>(scale) * kLog2e;
    auto s = reinterpret_cast<hipStream_t>(stream);
    const int wpg = (n_kv_heads % 4 == 0) ? 4 : (n_kv_heads % 2 == 0) ? 2 : 1;   // waves (kv heads) per group
    const dim3 grid(static_cast<unsigned>(num_tokens), static_cast<unsigned>(n_kv_heads / wpg),
                    static_cast<unsigned>(ms));
    const int st = split_tokens / kTileKeys;
    bool ok = true;
    if (phase & kPhaseSplit) {
    if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD) {
        ok = head_dim == 128 ? launch_rep<128, CVH_SCALE_PER_TOKEN_HEAD>(rep, grid, 64 * wpg, s, out, pa, pm, q, k_cache, v_cache,
                                                                        k_scale, v_scale, block_tables, table_width,
                                                                        token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                        static_cast<int>(ms), qs)
                             : launch_rep<64, CVH_SCALE_PER_TOKEN_HEAD>(rep, grid, 64 * wpg, s, out, pa, pm, q, k_cache, v_cache,
                                                                       k_scale, v_scale, block_tables, table_width,
                                                                       token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                       static_cast<int>(ms), qs);
    } else {
        ok = head_dim == 128 ? launch_rep<128, CVH_SCALE_PER_TENSOR>(rep, grid, 64 * wpg, s, out, pa, pm, q, k_cache, v_cache,
                                                                    k_scale, v_scale, block_tables, table_width,
                                                                    token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                    static_cast<int>(ms), qs)
                             : launch_rep<64, CVH_SCALE_PER_TENSOR>(rep, grid, 64 * wpg, s, out, pa, pm, q, k_cache, v_cache,
                                                                   k_scale, v_scale, block_tables, table_width,
                                                                   token_seq, token_kv_len, n_kv_heads, lg, st,
                                                                   static_cast<int>(ms), qs);
    }
    }
    if (!ok) return CVH_ERR_UNSUPPORTED;
    if (hipGetLastError() != hipSuccess) return CVH_ERR_LAUNCH;
    if (ms > 1 && (phase & kPhaseMerge)) {
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
}  // namespace
}  // namespace cvh

#define CVH_PA_ARGS                                                                                                   \
    out, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq, token_kv_len, num_tokens,      \
            n_heads, n_kv_heads, head_dim, block_size, scale_mode, scale, split_tokens, workspace, workspace_bytes,  \
            stream
#define CVH_PA_PARAMS                                                                                                 \
    void *out, const void *q, const uint8_t *k_cache, const uint8_t *v_cache, const float *k_scale,                 \
            const float *v_scale, const int64_t *block_tables, int64_t table_width, const int64_t *token_seq,        \
            const int64_t *token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,              \
            int block_size, int scale_mode, double scale, int split_tokens, void *workspace, size_t workspace_bytes, \
            cvh_stream_t stream

extern "C" int cvh_paged_attention_fp8_ex(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseBoth);
}
extern "C" int cvh_paged_attention_fp8_split_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseSplit);
}
extern "C" int cvh_paged_attention_fp8_merge_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseMerge);
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
