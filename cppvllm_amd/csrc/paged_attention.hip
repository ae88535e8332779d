// FP8-e4m3 paged decode attention for gfx950 (CDNA4).
//
// Reference semantics: kernels/paged_attention.cu:89-393 — per query token causal length,
// GQA query heads sharing each K/V row, per-(token, kv head) FP8 scales, online softmax in fp32,
// split partials merged with a log-sum-exp combine.
//
// Work decomposition (persistent, balanced — "stream-K" over the key axis):
//   * a *row* is (query token t, group of WPG consecutive kv heads); it has
//     ntiles(t) = ceil(kv_len(t) / 32) tiles of 32 keys. Rows are laid end to end in (t, group)
//     order, giving U tiles in total. Every workgroup builds the prefix sum of the row tile counts
//     in LDS from token_kv_len (no host knowledge of the lengths is needed, so the launch is
//     capture-safe), and processes exactly the tiles [w*U/G, (w+1)*U/G) for its index w of G.
//     Ragged contexts therefore cost no load imbalance and there is no tail of short items.
//   * a workgroup has WPG waves, one per kv head of the row group; they walk the same tiles, so
//     whole 1 KB slot rows (all heads of a token) are read together.
//   * a row piece that is cut by a workgroup boundary is written as an (acc, max, sum) partial to
//     one of two per-workgroup slots (0: the piece containing the workgroup's first tile, 1: the
//     one containing its last); whole rows are finished in place. paged_merge2_kernel combines
//     the pieces of cut rows.
//   * shared-prefix units (planned shared launches): the plan groups tokens whose block tables
//     start with the same shared blocks (prefix-cache hits) and appends one row per unit of up to
//     16 / REP such tokens after the real rows; a unit's tiles are the group's shared keys, multiplied
//     on matrix cores against the 16 query columns of its tokens (16 / REP tokens x REP heads), so the
//     prefix is read once per unit instead of once per token. Members' own rows start after the
//     shared keys; member rows and units always end as partials, which the merge combines.
//
// Per wave (one kv head, REP query heads), designed for wave64:
//   * lane = (grp, sub): grp = lane/8 picks one of 8 keys of a step, sub = lane%8 owns a 16-byte
//     (HD=128) or 8-byte (HD=64) slice of the 128-byte K and V rows, so each load instruction
//     covers 8 full key rows (8 x 128 B cache lines);
//   * a tile is 4 steps = 32 keys; the next two tiles' K/V/scale loads are in flight while one is
//     computed (register triple buffer, unrolled by three; the GQA-4/8 MFMA path: two tiles, one in
//     flight). The tile loops exit only at their bottom and prefetch straight-line, so the wait
//     before each compute covers only its own tile; block-table lookups run one tile ahead;
//   * raw buffer loads with the non-temporal hint; a prefetch past the piece's end gets a
//     zero-size descriptor and returns zeros without memory traffic;
//   * FP8 -> f32 with the hardware OCP converter (v_cvt_pk_f32_fp8, exact for finite codes);
//   * q.k partial dots reduce over the 8 lanes of a key with DPP (quad_perm, half-mirror);
//   * softmax in base 2 (scale*log2(e) folded into q) with a running max per key group and a
//     lazy rescale (only when a tile's max exceeds the running max by 2^8), exact because l and
//     acc share the stale max; groups are combined once per piece by a reduce-scatter (permlane
//     swaps, DPP row_ror:8), each lane ending with a few finished dims to convert and store.
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <cstddef>
#include <mutex>
#include <type_traits>

#include "cvh_device.h"

namespace cvh {
namespace {

constexpr int kSteps = 4;                  // 8-key steps per tile
constexpr int kTileKeys = 8 * kSteps;      // 32 keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units: stale max tolerated up to p = 2^8
constexpr float kMinusHuge = -1e30f;
constexpr int kMaxRows = 8192;             // rows (tokens x head groups) per launch: LDS prefix
constexpr size_t kLdsBytes = 160 * 1024;   // LDS of one gfx950 workgroup
constexpr int kQStageBytes = 16384;        // LDS for the q of a workgroup's first rows
// Full-row-group MFMA launches: each wave's K tile passes through LDS (32 rows of 128 bytes, rows
// 144 bytes apart so both the full-row writes and the MFMA-layout reads are bank-conflict free)
constexpr int kKtRowBytes = 144;
constexpr int kKtWaveBytes = 32 * kKtRowBytes;
constexpr int kMaxQRows = 8;
constexpr int kPreQRows = 4;               // q rows a planned launch fetches ahead of its first tiles
constexpr int kDeferMinTiles = 16;          // ranges this long hold their first cut piece's partial (MFMA path)
constexpr int kResidentWaves = 2048;       // MI355X: 256 CUs x 4 SIMDs x 2 waves (<= 256 VGPRs each)

// ---- buffer loads ------------------------------------------------------------------------------
// K/V rows and scales go through raw buffer loads: the descriptor's record count bounds every
// access, so a tile that must not be read is given a zero-size descriptor and returns zeros
// without touching memory. All K/V/scale loads carry the non-temporal hint: each byte is read
// once per launch and should not displace reusable lines (block tables, q, partials).
constexpr int kBufferWord3 = 0x00020000;   // raw buffer, 32-bit data format (gfx9 encoding)
constexpr int kNonTemporal = 2;            // cache-policy bits of the load: nt
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}
// The shared-prefix units read their group's blocks with the default policy instead, so the
// group's other units find them in L2 / the last-level cache.
constexpr int kTemporal = 0;
template <typename VT, int POL = kNonTemporal> __device__ __forceinline__ VT buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ uint4 buf_load<uint4, kNonTemporal>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNonTemporal);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ uint2 buf_load<uint2, kNonTemporal>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNonTemporal);
    return make_uint2(v[0], v[1]);
}
template <> __device__ __forceinline__ uint4 buf_load<uint4, kTemporal>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kTemporal);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ uint2 buf_load<uint2, kTemporal>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kTemporal);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kNonTemporal));
}
template <int POL> __device__ __forceinline__ uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---- GQA 4 / 8 on matrix cores (head_dim 128) ----------------------------------------------------
// One wave per (query token, kv head) as in the VALU path, but the REP query heads of the kv head are
// the 16 columns of v_mfma_f32_16x16x32_bf16 tiles (padded with zero columns):
//   S^T[key][head] = K . Q^T : A = K (16 keys x 32 d, e4m3 -> bf16 exact), B = Q^T (bf16)
//   O[head][d]    += P . V   : A = P (16 heads x 32 keys, bf16, V scale folded in), B = V (32 keys x 16 d)
// Lane (i16 = lane % 16, g = lane / 16). In S^T a lane holds one head (column i16) for keys
// {kb*16 + 4g + r}; those 8 keys are exactly the contraction slots 8g..8g+7 of the PV product's A
// operand, so P never leaves its lane. V's B operand wants 8 keys of one d per lane: the lane loads
// 8 bytes (d = 8*i16 .. +8) of each of its 8 keys, transposes the 4 key x 4 d byte blocks with
// v_perm_b32, and feeds d = 8*i16 + j to the MFMA j (j = 0..7), whose output holds heads 4g..4g+3 of
// that d in the lane. Softmax state is per S^T column (one head per lane, combined over the 4 lane
// groups with permlane swaps); the rare rescale of O rows and the final normalisation fetch the 4
// heads' factors with ds_bpermute. Loads per lane and 32-key tile: 4 x 16 B of K, 8 x 8 B of V and
// 4 scales (lane r of each row of 16 loads key 4g + r's; the row reads them with DPP broadcasts).
struct MfTile {
    uint4 k[2][2];          // [kb][h]: key kb*16 + i16, bytes h*64 + g*16 .. +16 of the head's row
                            // (with the LDS transpose: [kb][j]: key kb*16 + 8j + lane/8, bytes (lane%8)*16 .. +16)
    uint2 v[2][4];          // [kb][r]: key kb*16 + 4g + r, bytes 8*i16 .. +8
    float ks[2], vs[2];     // [kb]: key kb*16 + 4g + (i16 & 3); lane r of each row of 16 is broadcast
};
// value of lane r of this lane's row of 16 (DPP row_newbcast)
template <int R> __device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + R, 0xF, 0xF, false));
}
template <bool HI> __device__ __forceinline__ uint32_t fp8x2_bf16(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}
// 8 e4m3 codes (bytes of lo, then hi) -> bf16x8, exact
__device__ __forceinline__ bf16x8_t fp8x8_bf16(uint32_t lo, uint32_t hi) {
    const uint4 u = make_uint4(fp8x2_bf16<false>(lo), fp8x2_bf16<true>(lo), fp8x2_bf16<false>(hi), fp8x2_bf16<true>(hi));
    return __builtin_bit_cast(bf16x8_t, u);
}
// 4x4 byte transpose: w[r] holds bytes (r, 0..3); returns u[j] with bytes (0..3, j)
__device__ __forceinline__ void transpose4x4(const uint32_t (&w)[4], uint32_t (&u)[4]) {
    const uint32_t a = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);   // w0b0 w1b0 w0b1 w1b1
    const uint32_t b = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);   // w0b2 w1b2 w0b3 w1b3
    const uint32_t c = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
    const uint32_t d = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
    u[0] = __builtin_amdgcn_perm(c, a, 0x05040100u);
    u[1] = __builtin_amdgcn_perm(c, a, 0x07060302u);
    u[2] = __builtin_amdgcn_perm(d, b, 0x05040100u);
    u[3] = __builtin_amdgcn_perm(d, b, 0x07060302u);
}
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

template <int HD> struct KvVec;
template <> struct KvVec<128> {
    using T = uint4;
    static constexpr int kElems = 16;
    static __device__ __forceinline__ void words(const uint4& u, uint32_t (&w)[4]) {
        w[0] = u.x;
        w[1] = u.y;
        w[2] = u.z;
        w[3] = u.w;
    }
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
    static __device__ __forceinline__ void words(const uint2& u, uint32_t (&w)[2]) {
        w[0] = u.x;
        w[1] = u.y;
    }
    static __device__ __forceinline__ void to_f32(const uint2& u, float (&f)[8]) {
        fp8x4_to_f32(u.x, f + 0);
        fp8x4_to_f32(u.y, f + 4);
    }
};

// ---- cross-lane reductions ------------------------------------------------------------------------
// Sum over the 8 lanes of a key group (lanes 8k..8k+7); result in every lane of the group.
__device__ __forceinline__ float group8_sum(float v) {
    v = v + dpp_xor1(v);
    v = v + dpp_xor2(v);
    v = v + dpp_half_mirror(v);
    return v;
}
// Exchange across rows of 16 / halves of 32 lanes with the gfx950 permlane swaps (no LDS): with
// both operands = v, the returned pair holds, per lane, its own value and its xor-16 (resp.
// xor-32) partner's value.
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
// Sum over the 8 key groups; lanes with equal sub end with equal values.
__device__ __forceinline__ float across_groups_sum(float v) {
    v = v + dpp_xor8(v);
    v = xor16_sum(v);
    return xor32_sum(v);
}
// Max over the whole wave of a value that is uniform inside each key group.
__device__ __forceinline__ float across_groups_max(float v) {
    v = fmaxf(v, dpp_xor8(v));
    v = xor16_max(v);
    return xor32_max(v);
}

// Wave-uniform read of kernel-constant data (block tables, token metadata) through the constant
// address space, which makes it a scalar load (s_load) even though the pointer cannot be proven
// free of aliasing with the kernel's stores; vector loads here would share the vmcnt counter with
// the K/V stream and force full waits.
template <typename T> __device__ __forceinline__ T ld_uniform(const T* ptr, int64_t i) {
    typedef const T __attribute__((address_space(4)))* cptr;
    return ((cptr)(uintptr_t)ptr)[i];
}

// Per-workgroup start of the decode stream, written by the plan kernel once per batch layout
// (shared by every layer of a step): the first piece of the workgroup's first batch of rows and
// the physical blocks of its first two tiles, so a planned launch issues them before anything
// else. row < 0: no preload.
constexpr int kPlanWin = 8;                // rows of a workgroup's window carried in its plan record
struct PlanRec {
    int row, lt, le, kv_len, seq, b_ok, r_s, r_e;   // r_e: one past the last row holding a tile of the range
    int64_t a_lo, a_hi, b_lo, b_hi;
    // win = 1: every prefix entry and token record the workgroup reads lies in the window below, so
    // its launch needs neither the LDS copies of the prefix and token metadata nor the barrier
    // that publishes them. pre[i] = prefix[min(r_s + i, rows)]; tok[j] = token metadata of token
    // r_s / (n_kv / wpg) + j (clamped); U = prefix[rows].
    int win, U;
    int pre[kPlanWin + 1];
    int tkl[kPlanWin], tsq[kPlanWin];
    int pad[3];
};

constexpr int kUnitTokens = 16;            // most member tokens of a shared-prefix unit (16 MFMA columns, GQA 1)
struct UnitRec {
    int seq;                               // block-table row of the group's first member
    int keys;                              // shared keys (a multiple of the block size, or a whole context)
    int n;                                 // member tokens in this unit
    int tok[kUnitTokens];
    int pad;
};

struct Params {
    uint16_t* out;
    const PlanRec* plan;     // [G] (planned launches)
    int2* plan_tok;          // [T] (kv_len, block-table row) per token, written by the plan kernel
    int* shared_tok;         // [T] keys of token t in blocks shared with another sequence (plan kernel)
    const int32_t* shared_blocks;   // [table rows] leading shared blocks per row (plan input), or null
    // Shared-prefix units (planned shared launches at head_dim 128, one row group per token):
    // sequences whose block tables start with the same shared blocks are grouped; each group's
    // shared keys are read once per unit of up to unit_tokens member tokens (16 MFMA columns:
    // unit_tokens tokens x the query heads of one kv head), and each member's own row starts after them.
    UnitRec* units;          // [max_units] unit records (plan output)
    int* unit_count;         // [1] number of units (plan output)
    int2* tok_unit;          // [T] (unit, column) of a member token, (-1, 0) otherwise
    float* ptok_acc;         // [T][H][HD] partial of a member token's own row when one range held all of it
    float* ptok_ml;          // [T][H][2]
    float* punit_acc;        // [max_units][WPG][16][HD] partial of a unit held whole by one range
    float* punit_ml;         // [max_units][WPG][16][2]
    float* psh_acc;          // [G][2][WPG][16][HD] partials of units cut by a range boundary
    float* psh_ml;           // [G][2][WPG][16][2]
    int max_units;
    int unit_tokens;         // member tokens per unit: 16 MFMA columns / query heads per kv head
    float* part_acc;         // [G][2][WPG][REP][HD]
    float* part_ml;          // [G][2][WPG][REP][2]
    int* prefix_out;         // [rows + 1] row tile prefix, written by workgroup 0 for the merge
    const uint16_t* q;
    const uint8_t* k_cache;
    const uint8_t* v_cache;
    const float* k_scale;
    const float* v_scale;
    const int64_t* block_tables;
    int64_t table_width;
    const int64_t* token_seq;
    const int64_t* token_kv_len;
    int num_tokens;
    int n_kv;                // kv heads as the kernel sees them (virtual: physical << kv_shift)
    int kv_shift;            // log2 of the virtual kv heads per physical kv head
    int wpg;                 // kv heads (waves) per row group
    int pack;                // row-group ranges per workgroup (wpg * pack waves; 1 unless wpg < 4)
    int G;                   // tile ranges (workgroups x pack)
    int qrows;               // rows per workgroup whose q is staged in LDS by the prologue
    int log2_bs;
    float q_scale;           // softmax scale * log2(e)
};

// Causal length of token t, clamped to what its block-table row can address. A padding token
// (token_seq < 0) has length 0 whatever its kv_len says, so its output row is zero.
__device__ __forceinline__ int token_len(const Params& p, int t, int64_t seq) {
    if (seq < 0) return 0;
    int64_t kv = p.token_kv_len[t];
    const int64_t cap = p.table_width << p.log2_bs;
    if (kv > cap) kv = cap;
    return kv > 0 ? static_cast<int>(kv) : 0;
}

// Dynamic LDS: row tile prefix (int [rows + 1]); per-token (clamped kv_len, block-table row)
// (int2 [T]); the q staging area (bf16 [qrows][WPG][REP][HD]) on a 16-byte boundary.
__host__ __device__ inline size_t lds_tok_offset(int rows) {
    return ((static_cast<size_t>(rows) + 1) * 4 + 7) & ~size_t{7};
}
__host__ __device__ inline size_t lds_q_offset(int rows, int tokens) {
    return (lds_tok_offset(rows) + static_cast<size_t>(tokens) * 8 + 15) & ~size_t{15};
}
inline int q_stage_rows(int wpg, int rep, int hd) {
    const int per_row = wpg * rep * hd * 2;
    // the MFMA path (rep >= 4) stages up to 4 rows of 8 heads x 8 waves (64 KiB)
    const int budget = rep >= 4 ? 4 * kQStageBytes : kQStageBytes;
    return std::max(1, std::min(kMaxQRows, budget / per_row));
}
// GQA 4 and 8 run on MFMA at head_dim 128; elsewhere (head_dim 64) as 2 / 4 virtual kv heads of 2
// query heads (VALU path). Returns the number of virtual kv heads per physical one.
inline int virtual_kv_split(int rep, int head_dim) { return (rep > 2 && head_dim != 128) ? rep / 2 : 1; }

// Token metadata and the exclusive prefix of row tile counts into LDS (prefix[0..rows]); all
// threads of the block. kv_len and the block-table row of every token are fetched together (one
// memory round trip), so later lookups of a piece's token read LDS.
__device__ __forceinline__ void fill_tokens(const Params& p, int2* tok) {
    for (int t = threadIdx.x; t < p.num_tokens; t += blockDim.x) {
        const int64_t sq = p.token_seq[t];
        tok[t] = make_int2(token_len(p, t, sq), static_cast<int>(sq > 0 ? sq : 0));
    }
    __syncthreads();
}
// Exclusive prefix of the tile counts ntiles(r) of rows [0, rows) into LDS (prefix[0..rows]).
template <typename F>
__device__ __forceinline__ void scan_rows(int rows, F ntiles, int* prefix) {
    __shared__ int wave_tot[16];
    const int nthreads = blockDim.x;
    const int tid = threadIdx.x;
    const int per = (rows + nthreads - 1) / nthreads;
    const int beg = min(rows, tid * per), end = min(rows, beg + per);
    int s = 0;
    for (int r = beg; r < end; ++r) s += ntiles(r);
    // inclusive scan over the wave
    const int lane = tid & 63, wv = tid >> 6;
    int incl = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wave_tot[wv] = incl;
    __syncthreads();
    int off = 0;
    for (int i = 0; i < wv; ++i) off += wave_tot[i];
    int run = off + incl - s;            // exclusive prefix of this thread's chunk
    for (int r = beg; r < end; ++r) {
        prefix[r] = run;
        run += ntiles(r);
    }
    if (tid == nthreads - 1) {
        int tot = 0;
        for (int i = 0; i < nthreads / 64; ++i) tot += wave_tot[i];
        prefix[rows] = tot;
    }
    __syncthreads();
}
__device__ __forceinline__ void build_row_prefix(const Params& p, int rows, int hg_count, int* prefix, int2* tok) {
    fill_tokens(p, tok);
    scan_rows(rows, [&](int r) { return (tok[r / hg_count].x + kTileKeys - 1) / kTileKeys; }, prefix);
}

// Shared-prefix units (plan kernel, one workgroup). A token whose block-table row starts with
// blocks other rows also hold (shared_blocks) has s = min(kv_len, shared_blocks * block_size)
// shared keys. Tokens with the same first physical block, the same s and the same first
// ceil(s / block_size) table entries form a group; a group of two or more is split in token order
// into units of up to kUnitTokens members. Each member's own row then covers keys [s, kv_len)
// only (tok.x -= s; shared_tok = s), and unit u becomes row rows_real + u of the tile space, with
// ceil(s / 32) tiles over the group's shared keys. Returns the number of units.
__device__ int build_units(const Params& p, int2* tok) {
    __shared__ int n_units;
    const int T = p.num_tokens, tid = threadIdx.x, nth = blockDim.x;
    const int log2_bs = p.log2_bs;
    const int64_t W = p.table_width;
    const int ut = p.unit_tokens;
    if (tid == 0) n_units = 0;
    for (int i = tid; i < p.max_units; i += nth) p.units[i].n = 0;
    auto keys_of = [&](int t) -> int {
        const int64_t nb = p.shared_blocks[tok[t].y];
        return static_cast<int>(min(static_cast<int64_t>(tok[t].x), max(nb, int64_t{0}) << log2_bs));
    };
    auto same_prefix = [&](int a, int b, int keys) {
        const int64_t* ta = p.block_tables + static_cast<int64_t>(tok[a].y) * W;
        const int64_t* tb = p.block_tables + static_cast<int64_t>(tok[b].y) * W;
        const int nb = (keys + (1 << log2_bs) - 1) >> log2_bs;
        for (int i = 0; i < nb; ++i)
            if (ta[i] != tb[i]) return false;
        return true;
    };
    // pass 1: the group leader of every token (the first token with the same key), or -1
    for (int t = tid; t < T; t += nth) {
        const int st = (p.token_seq[t] >= 0) ? keys_of(t) : 0;
        int lead = -1;
        if (st > 0) {
            const int64_t first = p.block_tables[static_cast<int64_t>(tok[t].y) * W];
            for (int u = 0; u <= t && lead < 0; ++u)
                if (p.token_seq[u] >= 0 && keys_of(u) == st &&
                    p.block_tables[static_cast<int64_t>(tok[u].y) * W] == first && same_prefix(u, t, st))
                    lead = u;
        }
        p.tok_unit[t] = make_int2(lead, 0);
    }
    __syncthreads();
    // pass 2: index within the group; the leader also counts its group
    for (int t = tid; t < T; t += nth) {
        const int lead = p.tok_unit[t].x;
        int j = 0, size = 0;
        if (lead >= 0) {
            for (int u = lead; u < T; ++u)
                if (p.tok_unit[u].x == lead) {
                    if (u < t) ++j;
                    ++size;
                }
        }
        p.shared_tok[t] = (lead == t) ? size : 0;
        p.tok_unit[t].y = j;
    }
    __syncthreads();
    // pass 3: unit ids (units ordered by leader token, then member index)
    int my_unit[8], my_col[8], my_keys[8];
    int k = 0;
    for (int t = tid; t < T; t += nth, ++k) {
        const int lead = p.tok_unit[t].x;
        my_unit[k & 7] = -1;
        my_col[k & 7] = 0;
        my_keys[k & 7] = 0;
        if (lead < 0 || p.shared_tok[lead] < 2) continue;
        int base = 0;
        for (int u = 0; u < lead; ++u)
            if (p.tok_unit[u].x == u && p.shared_tok[u] >= 2) base += (p.shared_tok[u] + ut - 1) / ut;
        const int j = p.tok_unit[t].y;
        my_unit[k & 7] = base + j / ut;
        my_col[k & 7] = j % ut;
        my_keys[k & 7] = keys_of(t);
        if (lead == t) atomicAdd(&n_units, (p.shared_tok[t] + ut - 1) / ut);
    }
    __syncthreads();
    k = 0;
    for (int t = tid; t < T; t += nth, ++k) {
        const int u = my_unit[k & 7];
        p.tok_unit[t] = make_int2(u, my_col[k & 7]);
        p.shared_tok[t] = u >= 0 ? my_keys[k & 7] : 0;
        if (u >= 0) {
            UnitRec& rec = p.units[u];
            rec.tok[my_col[k & 7]] = t;
            if (my_col[k & 7] == 0) {
                rec.seq = tok[t].y;
                rec.keys = my_keys[k & 7];
            }
            tok[t].x -= my_keys[k & 7];
        }
    }
    __syncthreads();
    // member counts of the units (a unit's members are the columns written above)
    for (int t = tid; t < T; t += nth) {
        const int2 tu = p.tok_unit[t];
        if (tu.x >= 0) atomicMax(&p.units[tu.x].n, tu.y + 1);
    }
    __syncthreads();
    return n_units;
}

// First row a workgroup visits for tile range [u0, ...): the row holding tile u0, or the first
// empty row sitting at u0 (so empty rows at a range boundary get zeroed exactly once).
template <typename F> __device__ __forceinline__ int first_row(F pfx, int rows, int64_t u0) {
    int lo = 0, hi = rows;               // last r with prefix[r] <= u0
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pfx(mid) <= u0) lo = mid;
        else hi = mid;
    }
    int r = lo;
    if (pfx(r) == u0) {                  // rewind over empty rows that also start at u0
        int a = 0, b = r;
        while (a < b) {
            const int mid = (a + b) >> 1;
            if (pfx(mid) < u0) a = mid + 1;
            else b = mid;
        }
        r = a;
    }
    return r;
}

// One past the last row holding a tile of [u0, u1) (r_s when the range is empty): the rows a
// workgroup stages q for and walks are [r_s, end_row).
template <typename F> __device__ __forceinline__ int end_row(F pfx, int rows, int64_t u0, int64_t u1, int r_s) {
    if (u1 <= u0) return r_s;
    int lo = 0, hi = rows;               // last r with prefix[r] <= u1 - 1
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pfx(mid) <= u1 - 1) lo = mid;
        else hi = mid;
    }
    return lo + 1;
}

// One piece of work of a workgroup: tiles [lt, le) of row `row` (token t, kv head g of this wave).
// row < 0 marks "no more work" (its other fields are safe dummies: loads made for it use zero-size
// descriptors, and its table lookups stay inside block-table row 0).
struct Piece {
    int row, t, g, kv_len, lt, le;
    int shared_keys;   // keys [0, shared_keys) sit in blocks shared with other sequences
    int64_t seq;   // block-table row of token t
};

// DEFER (MFMA path, full 8-kv-head row groups): the range's first cut piece is stored after the
// range's tile stream (see `deferred` below), and K rows are loaded whole and passed through LDS
// into the MFMA layout (see `mf_load`); a separate instantiation because both slow the short
// ranges of the one-kv-head shares down.
template <int HD, int REP, int SM, bool ONE_BLOCK, bool PLANNED, bool SHARED = false, bool DEFER = false>
__global__ __launch_bounds__(512, 1) void paged_decode_kernel(Params p) {
    using V = KvVec<HD>;
    using VT = typename V::T;
    constexpr int E = V::kElems;
    extern __shared__ int prefix[];
    const int wpg = p.wpg;
    const int hg_count = p.n_kv / wpg;
    // shared-prefix units run on the MFMA path at head_dim 128 (16 columns: 16 / REP tokens x REP heads)
    constexpr bool UNITS = SHARED && HD == 128;
    const int rows_real = p.num_tokens * hg_count;
    const int rows = rows_real + ((UNITS && p.units != nullptr) ? ld_uniform(p.unit_count, 0) : 0);
    int2* tok = reinterpret_cast<int2*>(reinterpret_cast<char*>(prefix) + lds_tok_offset(rows_real + p.max_units));
    // values that are the same for every lane; uniform() makes that visible to the compiler so
    // all the piece bookkeeping below stays in scalar registers
    auto uniform = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    // A workgroup runs `pack` independent tile ranges of wpg waves each (pack > 1 only for row
    // groups of one kv head: the hardware spreads a 4-wave workgroup over the 4 SIMDs of a
    // CU, where one-wave workgroups were seen stacked two deep on some SIMDs while
    // others of the same CU stayed empty). They share the LDS prefix and token tables (identical
    // content) and have separate q staging areas.
    const int64_t G = p.G;
    // wave-uniform by construction; readfirstlane tells the compiler so (scalar descriptors)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wi = wave % wpg, vg = wave / wpg;
    const int w = static_cast<int>(blockIdx.x) * p.pack + vg;
    const bool last_wg = (w == G - 1);
    const int lane = threadIdx.x & 63;
    const int grp = lane >> 3;
    const int sub = lane & 7;
    const int H = p.n_kv * REP;
    const int log2_bs = p.log2_bs;
    const int kv_shift = p.kv_shift;
    const int n_kv_phys = p.n_kv >> kv_shift;
    const uint32_t row_bytes = static_cast<uint32_t>(n_kv_phys) * HD;   // bytes of one slot (all kv heads)
    const int64_t blk_bytes = static_cast<int64_t>(row_bytes) << log2_bs;
    const uint32_t blk_bytes32 = static_cast<uint32_t>(blk_bytes);
    const uint32_t srow_bytes = 4u << log2_bs;                      // scale row of one (block, head)
    const int bs_mask = (1 << log2_bs) - 1;

    constexpr bool MF = REP >= 4;                   // GQA 4 / 8: score and PV products on MFMA
    constexpr bool DEF = MF && DEFER;
    constexpr bool KT = DEF;                        // K through the per-wave LDS transpose area
    static_assert(!MF || HD == 128, "the MFMA path is laid out for head_dim 128");
    struct VTile {
        VT k[kSteps], v[kSteps];
        float ks[kSteps], vs[kSteps];
    };
    using Tile = std::conditional_t<MF, MfTile, VTile>;
    const int i16 = lane & 15, g4 = lane >> 4;      // MFMA lane coordinates
    // Physical blocks of a tile: `lo` for its first 16 keys, `hi` for the last 16 (equal unless
    // block_size == 16). Wave-uniform scalar loads, issued one tile ahead of the loads using them.
    struct Phys {
        int64_t lo, hi;
    };
    // With whole tiles inside one block (block_size >= 32) consecutive tiles mostly share a block:
    // the last (sequence, block) -> physical block pair is kept in scalar registers, so a tile in
    // the same block as the previous lookup issues no load (7 of 8 tiles at 256-token blocks) and
    // nothing later waits on one.
    int64_t memo_seq = -1, memo_phys = 0;
    int memo_blk = -1;
    auto lookup = [&](const Piece& pc, int tile) -> Phys {
        const int64_t seq = static_cast<int64_t>(uniform(static_cast<int>(pc.seq)));
        const int64_t* table = p.block_tables + seq * p.table_width;
        const int p0 = uniform(tile * kTileKeys);
        const int off = SHARED ? uniform(pc.shared_keys) : 0;   // a member row starts after its shared keys
        if constexpr (ONE_BLOCK) {
            const int blk = (off + p0) >> log2_bs;
            if (seq != memo_seq || blk != memo_blk) {
                memo_phys = max(ld_uniform(table, blk), int64_t{0});
                memo_seq = seq;
                memo_blk = blk;
            }
            return {memo_phys, memo_phys};
        }
        const int64_t lo = max(ld_uniform(table, (off + p0) >> log2_bs), int64_t{0});
        const int64_t hi = max(ld_uniform(table, uniform((off + min(p0 + kTileKeys / 2, pc.kv_len - 1)) >> log2_bs)),
                               int64_t{0});
        return {lo, hi};
    };
    // MFMA-layout tile loads (GQA 4 / 8 rows and shared-prefix units)
    auto mf_load = [&](auto pol, const Piece& pc, int tile, MfTile& tl, Phys ph2, bool live) {
        constexpr int POL = decltype(pol)::value;
        const int p0 = tile * kTileKeys;
        const uint32_t lv = static_cast<uint32_t>(live);             // arithmetic, not a branch
        const uint32_t kv_rec = blk_bytes32 * lv, s_rec = srow_bytes * lv;
            const uint32_t col = static_cast<uint32_t>(pc.g) * HD;   // the kv head's 128 bytes in a slot row
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int64_t ph = (ONE_BLOCK || kb == 0) ? ph2.lo : ph2.hi;
                const auto rk = make_rsrc(p.k_cache + ph * blk_bytes, kv_rec);
                const auto rv = make_rsrc(p.v_cache + ph * blk_bytes, kv_rec);
                if constexpr (KT) {
                    // K as full 128-byte rows, 8 per load (8 lanes a row): the MFMA layout reads each
                    // row as two 64-byte halves (~3% slower at GQA 8); mf_compute moves it through LDS
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t kin =
                                static_cast<uint32_t>(min(p0 + kb * 16 + 8 * j + (lane >> 3), pc.kv_len - 1) & bs_mask);
                        tl.k[kb][j] = buf_load<uint4, POL>(rk, kin * row_bytes + col + (lane & 7) * 16);
                    }
                } else {
                    const uint32_t kin = static_cast<uint32_t>(min(p0 + kb * 16 + i16, pc.kv_len - 1) & bs_mask);
                    const uint32_t koff = kin * row_bytes + col + g4 * 16;
                    tl.k[kb][0] = buf_load<uint4, POL>(rk, koff);
                    tl.k[kb][1] = buf_load<uint4, POL>(rk, koff + 64);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t vin = static_cast<uint32_t>(min(p0 + kb * 16 + 4 * g4 + r, pc.kv_len - 1) & bs_mask);
                    tl.v[kb][r] = buf_load<uint2, POL>(rv, vin * row_bytes + col + 8 * i16);
                }
                if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) {
                    const int64_t sbase = (ph * n_kv_phys + pc.g) << log2_bs;
                    const uint32_t sin = static_cast<uint32_t>(min(p0 + kb * 16 + 4 * g4 + (i16 & 3), pc.kv_len - 1) & bs_mask);
                    tl.ks[kb] = buf_load_f32(make_rsrc(p.k_scale + sbase, s_rec), sin * 4u);
                    tl.vs[kb] = buf_load_f32(make_rsrc(p.v_scale + sbase, s_rec), sin * 4u);
                } else {
                    tl.ks[kb] = 1.f;
                    tl.vs[kb] = 1.f;
                }
            }
    };
    // Keys past kv_len (a row's last tile) are clamped to key kv_len-1: a valid, finite row whose
    // score is masked. live = false (no work left): zero-size descriptors, no memory traffic.
    auto load_tile_pol = [&](auto pol, const Piece& pc, int tile, Tile& tl, Phys ph2, bool live) {
        constexpr int POL = decltype(pol)::value;
        const int p0 = tile * kTileKeys;
        const uint32_t lv = static_cast<uint32_t>(live);             // arithmetic, not a branch
        const uint32_t kv_rec = blk_bytes32 * lv, s_rec = srow_bytes * lv;
        if constexpr (MF) {
            mf_load(pol, pc, tile, tl, ph2, live);
        } else {
        const uint32_t lane_col = (pc.g >> kv_shift) * HD + sub * E;   // byte column inside a slot row
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int64_t ph = (ONE_BLOCK || s < kSteps / 2) ? ph2.lo : ph2.hi;
            const int pos = min(p0 + 8 * s + grp, pc.kv_len - 1);
            const uint32_t in_blk = static_cast<uint32_t>(pos & bs_mask);
            const uint32_t off = in_blk * row_bytes + lane_col;
            tl.k[s] = buf_load<VT, POL>(make_rsrc(p.k_cache + ph * blk_bytes, kv_rec), off);
            tl.v[s] = buf_load<VT, POL>(make_rsrc(p.v_cache + ph * blk_bytes, kv_rec), off);
            if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) {
                const int64_t sbase = (ph * n_kv_phys + (pc.g >> kv_shift)) << log2_bs;
                tl.ks[s] = buf_load_f32(make_rsrc(p.k_scale + sbase, s_rec), in_blk * 4u);
                tl.vs[s] = buf_load_f32(make_rsrc(p.v_scale + sbase, s_rec), in_blk * 4u);
            } else {
                tl.ks[s] = 1.f;
                tl.vs[s] = 1.f;
            }
        }
        }
    };

    auto load_tile = [&](const Piece& pc, int tile, Tile& tl, Phys ph2, bool live) {
        load_tile_pol(std::integral_constant<int, kNonTemporal>{}, pc, tile, tl, ph2, live);
    };

    Tile A, B, C;
    // A planned launch starts its first two K/V tiles from the plan record before it builds
    // anything, then copies the prefix and token metadata of the plan into LDS; otherwise the
    // workgroup derives them from token_kv_len itself (one memory round trip more, then the
    // block-table round trip before its first K/V load).
    bool preA = false, preB = false, preQ = false;
    int plan_row = -1, plan_lt = 0, plan_rs = -1, plan_re = -1;
    constexpr int QB = REP * HD * 2;                 // bytes of one row's q slice for one wave
    char* q_lds_b = reinterpret_cast<char*>(prefix) + lds_q_offset(rows_real + p.max_units, p.num_tokens) +
                    static_cast<size_t>(vg) * p.qrows * wpg * QB;
    constexpr int QL = (QB + 1023) / 1024;           // 16-byte loads per lane per row
    // this wave's K transpose area (used by the DEFER instantiation), after the workgroup's q staging
    char* kt_lds = reinterpret_cast<char*>(prefix) + lds_q_offset(rows_real + p.max_units, p.num_tokens) +
                   static_cast<size_t>(p.pack) * p.qrows * wpg * QB + static_cast<size_t>(threadIdx.x >> 6) * kKtWaveBytes;
    if constexpr (PLANNED) {
        // Everything the prologue waits for (q of the first rows, prefix, token metadata) is
        // requested before the first two tiles, so the in-order vmcnt wait for it leaves the
        // tiles in flight. Out-of-range entries use zero-size descriptors: straight-line code.
        const PlanRec* rp = p.plan + w;
        plan_row = ld_uniform(&rp->row, 0);
        plan_rs = ld_uniform(&rp->r_s, 0);
        plan_re = ld_uniform(&rp->r_e, 0);
        uint4 qv[kPreQRows][QL];
#pragma unroll
        for (int r = 0; r < kPreQRows; ++r) {
            const bool live = r < p.qrows && plan_rs + r < min(plan_re, rows_real);   // unit rows stage no q
            const int rr = live ? plan_rs + r : 0;
            const int t = rr / hg_count, g = (rr % hg_count) * wpg + wi;
            const auto rs = make_rsrc(p.q + (static_cast<int64_t>(t) * H + g * REP) * HD, live ? QB : 0);
#pragma unroll
            for (int j = 0; j < QL; ++j) qv[r][j] = buf_load<uint4>(rs, lane * 16 + j * 1024);
        }
        // the plan's row window, one entry per lane (lanes 0..8 prefix, 0..7 token records)
        const auto rec_rs = make_rsrc(rp, sizeof(PlanRec));
        const int wpre = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(
                rec_rs, static_cast<int>(offsetof(PlanRec, pre)) + 4 * min(lane, kPlanWin), 0, 0));
        const int wtkl = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(
                rec_rs, static_cast<int>(offsetof(PlanRec, tkl)) + 4 * min(lane, kPlanWin - 1), 0, 0));
        const int wtsq = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(
                rec_rs, static_cast<int>(offsetof(PlanRec, tsq)) + 4 * min(lane, kPlanWin - 1), 0, 0));
        const int wU = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(
                rec_rs, static_cast<int>(offsetof(PlanRec, U)), 0, 0));
        const bool win = ld_uniform(&rp->win, 0) != 0;
        const int bd = blockDim.x, tid = threadIdx.x;
        const auto pre_rs = make_rsrc(p.prefix_out, (rows + 1) * 4);
        const auto tok_rs = make_rsrc(p.plan_tok, p.num_tokens * 8);
        const int pv0 = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(pre_rs, tid * 4, 0, 0));
        const int pv1 = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(pre_rs, (tid + bd) * 4, 0, 0));
        const u32x2_t tv0 = __builtin_amdgcn_raw_buffer_load_b64(tok_rs, tid * 8, 0, 0);
        const u32x2_t tv1 = __builtin_amdgcn_raw_buffer_load_b64(tok_rs, (tid + bd) * 8, 0, 0);
        {
            const bool live = plan_row >= 0;
            Piece pc;
            pc.row = live ? plan_row : 0;
            pc.t = pc.row / hg_count;
            pc.g = (pc.row % hg_count) * wpg + wi;
            plan_lt = ld_uniform(&rp->lt, 0);
            pc.lt = plan_lt;
            pc.le = ld_uniform(&rp->le, 0);
            pc.kv_len = live ? ld_uniform(&rp->kv_len, 0) : 1;
            pc.seq = ld_uniform(&rp->seq, 0);
            pc.shared_keys = (SHARED && live) ? ld_uniform(p.shared_tok, pc.t) : 0;
            const bool b_ok = live && ld_uniform(&rp->b_ok, 0) != 0;
            const int64_t a_lo = ld_uniform(&rp->a_lo, 0), b_lo = ld_uniform(&rp->b_lo, 0);
            load_tile(pc, plan_lt, A, {a_lo, ld_uniform(&rp->a_hi, 0)}, live);
            load_tile(pc, plan_lt + 1, B, {b_lo, ld_uniform(&rp->b_hi, 0)}, b_ok);
            preA = live;
            preB = b_ok;
            if (ONE_BLOCK && live) {         // the newest tile's block seeds the lookup memo
                memo_seq = uniform(static_cast<int>(pc.seq));
                memo_blk = ((b_ok ? plan_lt + 1 : plan_lt) * kTileKeys + pc.shared_keys) >> log2_bs;
                memo_phys = b_ok ? b_lo : a_lo;
            }
        }
#pragma unroll
        for (int r = 0; r < kPreQRows; ++r)
#pragma unroll
            for (int j = 0; j < QL; ++j)
                if (r < p.qrows && lane * 16 + j * 1024 < QB)
                    *reinterpret_cast<uint4*>(q_lds_b + (r * wpg + wi) * QB + lane * 16 + j * 1024) = qv[r][j];
        if (win) {
            // Every wave writes the whole window, the same values at the same places, and reads only
            // inside it after its own writes (LDS operations of a wave complete in order): no barrier.
            if (lane <= kPlanWin) prefix[min(plan_rs + lane, rows)] = wpre;
            if (lane == 0) prefix[rows] = wU;
            if (lane < kPlanWin)
                tok[min(plan_rs / hg_count + lane, p.num_tokens - 1)] = make_int2(wtkl, wtsq);
        } else {
            if (tid <= rows) prefix[tid] = pv0;
            if (tid + bd <= rows) prefix[tid + bd] = pv1;
            if (tid < p.num_tokens) tok[tid] = make_int2(static_cast<int>(tv0[0]), static_cast<int>(tv0[1]));
            if (tid + bd < p.num_tokens) tok[tid + bd] = make_int2(static_cast<int>(tv1[0]), static_cast<int>(tv1[1]));
            for (int i = tid + 2 * bd; i <= rows; i += bd) prefix[i] = p.prefix_out[i];
            for (int t = tid + 2 * bd; t < p.num_tokens; t += bd) tok[t] = p.plan_tok[t];
            __syncthreads();
        }
    } else {
        build_row_prefix(p, rows, hg_count, prefix, tok);
        if (blockIdx.x == 0)
            for (int i = threadIdx.x; i <= rows; i += blockDim.x) p.prefix_out[i] = prefix[i];
    }

    auto pfx = [&](int i) { return uniform(prefix[i]); };
    const int64_t U = pfx(rows);
    const int64_t u0 = w * U / G, u1 = (w + 1) * U / G;

    // ---- first row to visit, and one past the last row holding a tile of the range (a planned
    // launch has both in its plan record)
    const int r_s = PLANNED ? plan_rs : first_row(pfx, rows, u0);
    const int r_e = PLANNED ? plan_re : end_row(pfx, rows, u0, u1, r_s);
    // ---- empty rows of the range (kv_len <= 0): zero output (the reference would give 0/0)
    for (int r = r_s; r < rows_real; ++r) {
        const int64_t pr0 = pfx(r), pr1 = pfx(r + 1);
        if (!(pr0 < u1 || (last_wg && pr0 == U))) break;
        if (pr1 != pr0) continue;
        const int t = r / hg_count, g = (r % hg_count) * wpg + wi;
#pragma unroll
        for (int rr = 0; rr < REP; ++rr) {
            uint16_t* o = p.out + ((int64_t)t * H + g * REP + rr) * HD;
            for (int dd = lane; dd < HD; dd += 64) o[dd] = 0;
        }
    }

    // ---- pieces: the non-empty rows of [u0, u1), in order
    auto piece_from = [&](int r, int rlim) -> Piece {
        for (; r < rlim; ++r) {
            const int64_t pr0 = pfx(r), pr1 = pfx(r + 1);
            if (pr0 >= u1) break;
            if (pr1 == pr0) continue;
            Piece pc;
            pc.row = r;
            pc.t = r / hg_count;
            pc.g = (r % hg_count) * wpg + wi;
            const int2 tm = tok[pc.t];
            pc.kv_len = uniform(tm.x);
            pc.shared_keys = SHARED ? ld_uniform(p.shared_tok, pc.t) : 0;
            pc.lt = static_cast<int>(max(u0, pr0) - pr0);
            pc.le = static_cast<int>(min(u1, pr1) - pr0);
            pc.seq = uniform(tm.y);
            return pc;
        }
        Piece none;
        none.row = -1;
        none.t = 0;
        none.g = wi;
        none.kv_len = 1;
        none.lt = 0;
        none.le = 1;
        none.seq = 0;
        none.shared_keys = 0;
        return none;
    };

    // q slice for the REP heads of the piece's kv head, kept as raw bf16 pairs: the scores are
    // bf16 x bf16 dot products (v_dot2c_f32_bf16) against K converted fp8 -> bf16, both exact, and
    // scale*log2(e) [*k_scale] is applied to each score. Rows are processed in batches of up to
    // qrows rows whose q is first staged in LDS (each wave its own head), so starting a piece
    // reads LDS and never waits behind the K/V loads in flight.
    const float qsc = (SM == CVH_SCALE_PER_TENSOR) ? p.q_scale * p.k_scale[0] : p.q_scale;
    constexpr int QW = E / 2;                       // 32-bit words of bf16 pairs per head per lane
    uint16_t* q_lds = reinterpret_cast<uint16_t*>(q_lds_b);
    int rb = r_s;                        // first row of the current batch of up to qrows rows
    // a planned launch has staged the first kPreQRows rows of its first batch already
    preQ = PLANNED && r_s == plan_rs;
    auto stage_q = [&](int r0, int rlim) {   // q of rows [r0, rlim) -> LDS, this wave's head
        for (int r = r0; r < rlim; ++r) {
            const int t = r / hg_count, g = (r % hg_count) * wpg + wi;
            const uint16_t* src = p.q + ((int64_t)t * H + g * REP) * HD;
            uint16_t* dst = q_lds + ((r - rb) * wpg + wi) * (REP * HD);
            for (int o = lane * 8; o < REP * HD; o += 64 * 8)
                *reinterpret_cast<uint4*>(dst + o) = *reinterpret_cast<const uint4*>(src + o);
        }
    };
    uint32_t qf[MF ? 1 : REP][QW];
    bf16x8_t qm[(MF || UNITS) ? 4 : 1];                        // MFMA B operands: step st covers d = (st>>1)*64 + g*16 + (st&1)*8 .. +8
    auto take_q = [&](const Piece& pc) {
        const uint16_t* src = q_lds + ((pc.row - rb) * wpg + wi) * (REP * HD);
        if constexpr (MF) {
            const bool head = i16 < REP;            // columns past REP are zero padding
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                uint4 u = make_uint4(0u, 0u, 0u, 0u);
                if (head) u = *reinterpret_cast<const uint4*>(src + i16 * HD + (st >> 1) * 64 + g4 * 16 + (st & 1) * 8);
                qm[st] = __builtin_bit_cast(bf16x8_t, u);
            }
        } else {
#pragma unroll
            for (int r = 0; r < REP; ++r)
#pragma unroll
                for (int c = 0; c < E / 8; ++c) {
                    const uint4 u = *reinterpret_cast<const uint4*>(src + r * HD + sub * E + 8 * c);
                    qf[r][4 * c] = u.x;
                    qf[r][4 * c + 1] = u.y;
                    qf[r][4 * c + 2] = u.z;
                    qf[r][4 * c + 3] = u.w;
                }
        }
    };
    // running max per key group; a finite floor so an all-masked group gives exp2(-inf) = 0
    float m[MF ? 1 : REP], l[MF ? 1 : REP], acc[MF ? 1 : REP][E];
    // MFMA path: softmax state of this lane's S^T column (one head), O rows of heads 4g..4g+3
    float mm = kMinusHuge, lm = 0.f;
    f32x4_t om[(MF || UNITS) ? 8 : 1];                         // [j]: d = 8*i16 + j, rows = heads 4g..4g+3
    // MFMA path: the partial of the range's first piece when a boundary cuts it (slot 0), held in
    // registers until the range's tile stream has ended. A store issued inside the stream would be
    // waited for by the next tile's loads (one in-order vector-memory counter), and its write
    // acknowledgement queues behind the saturating K/V reads. Short ranges store at once: there
    // the deferred store would sit in the launch's tail instead.
    f32x4_t dom[DEF ? 8 : 1];
    float dmm = 0.f, dL = 0.f;
    bool deferred = false;
    auto reset = [&]() {
        if constexpr (MF) {
            mm = kMinusHuge;
            lm = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) om[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                m[r] = kMinusHuge;
                l[r] = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] = 0.f;
            }
        }
    };
    auto mf_compute = [&](const Piece& pc, int tile, const MfTile& tl) {
        const int p0 = tile * kTileKeys;
            // K rows -> LDS (full rows), back in the MFMA layout: key kb*16 + i16, bytes h*64 + g*16 .. +16
            // (a wave's LDS operations complete in order, so the reads see this tile's writes and
            // the next tile's writes come after these reads)
            uint4 kt[2][2];
            if constexpr (KT) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        *reinterpret_cast<uint4*>(kt_lds + (kb * 16 + 8 * j + (lane >> 3)) * kKtRowBytes + (lane & 7) * 16) =
                                tl.k[kb][j];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        kt[kb][h] = *reinterpret_cast<const uint4*>(kt_lds + (kb * 16 + i16) * kKtRowBytes + h * 64 + g4 * 16);
            } else {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int h = 0; h < 2; ++h) kt[kb][h] = tl.k[kb][h];
            }
            // S^T for keys kb*16 + 4g + r (rows) x heads (columns)
            float sv[2][4];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                f32x4_t sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const uint4 kw = kt[kb][st >> 1];
                    const bf16x8_t ka = (st & 1) ? fp8x8_bf16(kw.z, kw.w) : fp8x8_bf16(kw.x, kw.y);
                    sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qm[st], sa, 0, 0, 0);
                }
                const float ksr[4] = {row_bcast<0>(tl.ks[kb]), row_bcast<1>(tl.ks[kb]), row_bcast<2>(tl.ks[kb]),
                                      row_bcast<3>(tl.ks[kb])};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool valid = p0 + kb * 16 + 4 * g4 + r < pc.kv_len;
                    const float f = (SM == CVH_SCALE_PER_TOKEN_HEAD) ? ksr[r] * qsc : qsc;
                    sv[kb][r] = valid ? sa[r] * f : -INFINITY;
                }
            }
            float mt = fmaxf(fmaxf(fmaxf(sv[0][0], sv[0][1]), fmaxf(sv[0][2], sv[0][3])),
                             fmaxf(fmaxf(sv[1][0], sv[1][1]), fmaxf(sv[1][2], sv[1][3])));
            mt = xor32_max(xor16_max(mt));            // the column's (head's) tile max over the 4 lane groups
            const bool need = mt > mm + kRescaleThreshold;
            if (__builtin_amdgcn_ballot_w64(need) != 0) {
                const float mn = need ? mt : mm;
                const float c = __builtin_amdgcn_exp2f(mm - mn);
                lm *= c;
                mm = mn;
                // O rows are heads 4g..4g+3: their factors live in the S^T columns (lanes) 4g + r
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float cr = __shfl(c, 4 * g4 + r, 64);
#pragma unroll
                    for (int j = 0; j < 8; ++j) om[j][r] *= cr;
                }
            }
            // p (with the V scale) as a bf16 pair hi + lo: hi = bf16(w), lo = bf16(w - hi), so the two
            // PV products carry w to ~16 significant bits (the fp32 weights of the VALU path; a
            // single bf16 rounding of w lets 20x-outlier rows drift by several output ulps)
            uint32_t pw[4], pl[4];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const float vsr[4] = {row_bcast<0>(tl.vs[kb]), row_bcast<1>(tl.vs[kb]), row_bcast<2>(tl.vs[kb]),
                                      row_bcast<3>(tl.vs[kb])};
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    const float p0v = __builtin_amdgcn_exp2f(sv[kb][r] - mm);
                    const float p1v = __builtin_amdgcn_exp2f(sv[kb][r + 1] - mm);
                    lm += p0v + p1v;
                    const float w0 = (SM == CVH_SCALE_PER_TOKEN_HEAD) ? p0v * vsr[r] : p0v;
                    const float w1 = (SM == CVH_SCALE_PER_TOKEN_HEAD) ? p1v * vsr[r + 1] : p1v;
                    const uint32_t h = pack_bf16x2_rne(w0, w1);
                    pw[kb * 2 + r / 2] = h;
                    pl[kb * 2 + r / 2] = pack_bf16x2_rne(w0 - __uint_as_float(h << 16), w1 - __uint_as_float(h & 0xffff0000u));
                }
            }
            const bf16x8_t pa = __builtin_bit_cast(bf16x8_t, make_uint4(pw[0], pw[1], pw[2], pw[3]));
            const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, make_uint4(pl[0], pl[1], pl[2], pl[3]));
#pragma unroll
            for (int hw = 0; hw < 2; ++hw) {        // d = 8*i16 + 4*hw + jj
                uint32_t t0[4], t1[4];
                const uint32_t w0[4] = {hw ? tl.v[0][0].y : tl.v[0][0].x, hw ? tl.v[0][1].y : tl.v[0][1].x,
                                        hw ? tl.v[0][2].y : tl.v[0][2].x, hw ? tl.v[0][3].y : tl.v[0][3].x};
                const uint32_t w1[4] = {hw ? tl.v[1][0].y : tl.v[1][0].x, hw ? tl.v[1][1].y : tl.v[1][1].x,
                                        hw ? tl.v[1][2].y : tl.v[1][2].x, hw ? tl.v[1][3].y : tl.v[1][3].x};
                transpose4x4(w0, t0);               // t0[jj]: keys 4g..4g+3 at d = 8*i16 + 4*hw + jj
                transpose4x4(w1, t1);               // t1[jj]: keys 16+4g..
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const bf16x8_t vb = fp8x8_bf16(t0[jj], t1[jj]);
                    om[4 * hw + jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, om[4 * hw + jj], 0, 0, 0);
                    om[4 * hw + jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pb, vb, om[4 * hw + jj], 0, 0, 0);
                }
            }
    };
    auto compute = [&](const Piece& pc, int tile, const Tile& tl) {
        const int p0 = tile * kTileKeys;
        if constexpr (MF) {
            mf_compute(pc, tile, tl);
        } else {
        float sc[REP][kSteps];
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            uint32_t kw[E / 4];
            V::words(tl.k[s], kw);
#pragma unroll
            for (int r = 0; r < REP; ++r) sc[r][s] = 0.f;
#pragma unroll
            for (int j = 0; j < E / 4; ++j) {
                const bf16x2_t k01 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kw[j], 1.0f, false);
                const bf16x2_t k23 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kw[j], 1.0f, true);
#pragma unroll
                for (int r = 0; r < REP; ++r) {
                    sc[r][s] = __builtin_amdgcn_fdot2_f32_bf16(k01, __builtin_bit_cast(bf16x2_t, qf[r][2 * j]),
                                                               sc[r][s], false);
                    sc[r][s] = __builtin_amdgcn_fdot2_f32_bf16(k23, __builtin_bit_cast(bf16x2_t, qf[r][2 * j + 1]),
                                                               sc[r][s], false);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const bool valid = (p0 + 8 * s + grp) < pc.kv_len;
            const float f = (SM == CVH_SCALE_PER_TOKEN_HEAD) ? tl.ks[s] * qsc : qsc;
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                const float dsum = group8_sum(sc[r][s]) * f;
                sc[r][s] = valid ? dsum : -INFINITY;
            }
        }
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            float mt = sc[r][0];
#pragma unroll
            for (int s = 1; s < kSteps; ++s) mt = fmaxf(mt, sc[r][s]);
            const bool need = mt > m[r] + kRescaleThreshold;    // per key group
            if (__builtin_amdgcn_ballot_w64(need) != 0) {      // wave-uniform; rare after a piece's first tile
                const float mn = need ? mt : m[r];
                const float c = __builtin_amdgcn_exp2f(m[r] - mn);
                l[r] *= c;
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] *= c;
                m[r] = mn;
            }
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const float pr = __builtin_amdgcn_exp2f(sc[r][s] - m[r]);
                l[r] += pr;
                if constexpr (SM == CVH_SCALE_PER_TOKEN_HEAD) sc[r][s] = pr * tl.vs[s];
                else sc[r][s] = pr;
            }
        }
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            float vf[E];
            V::to_f32(tl.v[s], vf);
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                const float wgt = sc[r][s];
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] += wgt * vf[e];
            }
        }
        }
    };
    // End of a piece: combine the 8 key groups (rescale each to the wave max, then sum) and
    // write the finished row, or the partial of a cut row to slot 0 (holds u0) / 1 (holds u1-1).
    // The 8 key groups are combined by a reduce-scatter: each lane starts with REP*E partial
    // values (REP heads x E dims) and ends with NV/8 of them summed over the 8 groups, so every
    // lane converts and stores NV/8 consecutive dims of one head instead of group 0 handling all.
    // Levels: xor 16 and xor 32 with the permlane swaps (one swap exchanges a pair of halves:
    // swap(vdst = upper, src = lower) leaves even rows / lower lanes the two upper halves and the
    // others the two lower halves, so one add finishes the pair), then xor 8 with DPP.
    constexpr int NV = REP * E, NV8 = NV / 8;
    static_assert(NV8 >= 1 && E % NV8 == 0, "each lane's share lies in one head");
    const int b3 = (lane >> 3) & 1, b4 = (lane >> 4) & 1, b5 = (lane >> 5) & 1;
    const int v_own = (b4 ? 0 : NV / 2) + (b5 ? 0 : NV / 4) + (b3 ? NV8 : 0);   // first value index kept
    const int r_own = v_own / E, e_own = v_own % E;
    auto finish = [&](const Piece& pc) {
        const int64_t pr0 = pfx(pc.row), pr1 = pfx(pc.row + 1);
        if constexpr (MF) {
            const float L = xor32_sum(xor16_sum(lm));   // the column's (head's) sum over all its keys
            float Lr[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) Lr[r] = __shfl(L, 4 * g4 + r, 64);   // heads of this lane's O rows
            if (UNITS && pc.shared_keys > 0 && pc.lt == 0 && pc.le == pr1 - pr0) {
                // a member row held whole: its partial joins the unit's in the merge
                const int64_t base = (int64_t)pc.t * H + pc.g * REP;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int head = 4 * g4 + r;
                    if (head >= REP) continue;
                    float* pa = p.ptok_acc + (base + head) * HD + 8 * i16;
                    *reinterpret_cast<float4*>(pa) = make_float4(om[0][r], om[1][r], om[2][r], om[3][r]);
                    *reinterpret_cast<float4*>(pa + 4) = make_float4(om[4][r], om[5][r], om[6][r], om[7][r]);
                }
                if (g4 == 0 && i16 < REP) reinterpret_cast<float2*>(p.ptok_ml)[base + i16] = make_float2(mm, L);
            } else if (pc.lt == 0 && pc.le == pr1 - pr0) {
                const float vfin = (SM == CVH_SCALE_PER_TENSOR) ? p.v_scale[0] : 1.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int head = 4 * g4 + r;
                    if (head >= REP) continue;
                    const float f = vfin / Lr[r];
                    uint16_t* o = p.out + ((int64_t)pc.t * H + pc.g * REP + head) * HD + 8 * i16;
                    *reinterpret_cast<uint4*>(o) = make_uint4(pack_bf16x2_rne(om[0][r] * f, om[1][r] * f),
                                                              pack_bf16x2_rne(om[2][r] * f, om[3][r] * f),
                                                              pack_bf16x2_rne(om[4][r] * f, om[5][r] * f),
                                                              pack_bf16x2_rne(om[6][r] * f, om[7][r] * f));
                }
            } else if (DEF && pr0 <= u0 && u1 - u0 >= kDeferMinTiles) {   // slot 0 of a long range: stored later
#pragma unroll
                for (int j = 0; j < (DEF ? 8 : 1); ++j) dom[j] = om[j];
                dmm = mm;
                dL = L;
                deferred = true;
            } else {
                const int slot = (pr0 <= u0) ? 0 : 1;
                const int64_t base = ((static_cast<int64_t>(w) * 2 + slot) * wpg + wi) * REP;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int head = 4 * g4 + r;
                    if (head >= REP) continue;
                    float* pa = p.part_acc + (base + head) * HD + 8 * i16;
                    *reinterpret_cast<float4*>(pa) = make_float4(om[0][r], om[1][r], om[2][r], om[3][r]);
                    *reinterpret_cast<float4*>(pa + 4) = make_float4(om[4][r], om[5][r], om[6][r], om[7][r]);
                }
                if (g4 == 0 && i16 < REP) reinterpret_cast<float2*>(p.part_ml)[base + i16] = make_float2(mm, L);
            }
        } else {
        float cs[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float M = across_groups_max(m[r]);
            cs[r] = __builtin_amdgcn_exp2f(m[r] - M);
            m[r] = M;
            l[r] = across_groups_sum(l[r] * cs[r]);   // l is uniform inside a group
        }
        float a16[NV / 2];
#pragma unroll
        for (int i = 0; i < NV / 2; ++i) {
            const float lo = acc[i / E][i % E] * cs[i / E];
            const float hi = acc[(NV / 2 + i) / E][(NV / 2 + i) % E] * cs[(NV / 2 + i) / E];
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(hi), __float_as_uint(lo), false, false);
            a16[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        float a32[NV / 4];
#pragma unroll
        for (int i = 0; i < NV / 4; ++i) {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a16[NV / 4 + i]), __float_as_uint(a16[i]),
                                                             false, false);
            a32[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        float res[NV8];
#pragma unroll
        for (int i = 0; i < NV8; ++i) {
            const float x = a32[i], y = a32[NV8 + i];
            const float keep = b3 ? y : x, send = b3 ? x : y;
            res[i] = keep + dpp_xor8(send);
        }
        float l_own = l[0], m_own = m[0];
#pragma unroll
        for (int r = 1; r < REP; ++r)
            if (r_own == r) {
                l_own = l[r];
                m_own = m[r];
            }
        if (UNITS && pc.shared_keys > 0 && pc.lt == 0 && pc.le == pr1 - pr0) {
            // a member row held whole: its partial joins the unit's in the merge
            const int64_t idx = (int64_t)pc.t * H + pc.g * REP + r_own;
            float* pa = p.ptok_acc + idx * HD + sub * E + e_own;
#pragma unroll
            for (int i = 0; i < NV8; ++i) pa[i] = res[i];
            if (sub == 0 && e_own == 0) reinterpret_cast<float2*>(p.ptok_ml)[idx] = make_float2(m_own, l_own);
        } else if (pc.lt == 0 && pc.le == pr1 - pr0) {
            const float vfin = (SM == CVH_SCALE_PER_TENSOR) ? p.v_scale[0] : 1.f;
            const float f = vfin / l_own;
            uint16_t* o = p.out + ((int64_t)pc.t * H + pc.g * REP + r_own) * HD + sub * E + e_own;
            if constexpr (NV8 == 1) {
                *o = f32_to_bf16_bits(res[0] * f);
            } else {
                uint32_t wd[NV8 / 2];
#pragma unroll
                for (int i = 0; i < NV8 / 2; ++i)
                    wd[i] = f32_to_bf16_bits(res[2 * i] * f) | (uint32_t(f32_to_bf16_bits(res[2 * i + 1] * f)) << 16);
                if constexpr (NV8 == 4) *reinterpret_cast<uint2*>(o) = make_uint2(wd[0], wd[1]);
                else *reinterpret_cast<uint32_t*>(o) = wd[0];
            }
        } else {
            const int slot = (pr0 <= u0) ? 0 : 1;
            const int64_t idx = ((static_cast<int64_t>(w) * 2 + slot) * wpg + wi) * REP + r_own;
            float* pa = p.part_acc + idx * HD + sub * E + e_own;
#pragma unroll
            for (int i = 0; i < NV8; ++i) pa[i] = res[i];
            if (sub == 0 && e_own == 0) reinterpret_cast<float2*>(p.part_ml)[idx] = make_float2(m_own, l_own);
        }
        }
    };

    // ---- per batch: one tile stream over its pieces, two tiles in flight ahead of the one being
    // computed (register triple buffer, unrolled by three so no tile is copied between buffers)
    for (;;) {
        if (rb >= min(r_e, rows_real) || pfx(rb) >= u1) break;   // rlim > rb below: the loop always advances
        const int rlim = min(min(r_e, rows_real), rb + p.qrows);
        Piece pa_ = piece_from(rb, rlim);
        if (pa_.row >= 0) {
            int ta_ = pa_.lt;
            Piece pb_, pc_;
            int tb_, tc_;
            Piece lp = pa_;              // load cursor (the tile after the newest buffered one)
            int lt = ta_;
            auto advance = [&]() {
                if (lt + 1 < lp.le) ++lt;
                else if (lp.row >= 0) {
                    lp = piece_from(lp.row + 1, rlim);
                    lt = lp.lt;
                }
            };
            // the first two tiles are in flight before q is staged: their latency covers it (a
            // planned launch issued them at its start when they are the plan's)
            preA = preA && pa_.row == plan_row && ta_ == plan_lt;
            const Phys ph_a = preA ? Phys{0, 0} : lookup(pa_, ta_);
            advance();
            pb_ = lp;
            tb_ = lt;
            preB = preB && preA && pb_.row == pa_.row && tb_ == ta_ + 1;
            // B's loads follow A's on every path through this code (a fresh A always takes a fresh
            // B), so the compiler's waits for A's registers leave B's loads in flight
            if (!preA) {
                load_tile(pa_, ta_, A, ph_a, true);
                load_tile(pb_, tb_, B, lookup(pb_, tb_), pb_.row >= 0);
            } else if (!preB) {
                load_tile(pb_, tb_, B, lookup(pb_, tb_), pb_.row >= 0);
            }
            preA = preB = false;
            advance();
            Phys ph = lookup(lp, lt);
            stage_q(preQ ? min(rlim, rb + kPreQRows) : rb, rlim);
            preQ = false;
            take_q(pa_);
            reset();
            if constexpr (MF) {
                // one tile in flight while one is computed (two register tiles): the MFMA tiles
                // are larger than the VALU ones and three do not fit the register budget. The loop
                // has a single exit at the bottom (B's loads are issued, as zero-size loads, also
                // after the last tile): every path back to the loop head then issues A's loads
                // before B's, so the compiler's wait for a tile leaves the other tile's loads in
                // flight (an exit from inside the finish makes the compiler's loop flow add paths
                // without B's loads, and its waits for A then cover B's loads as well).
                for (;;) {
                    compute(pa_, ta_, A);
                    if (ta_ + 1 == pa_.le) {
                        finish(pa_);
                        if (pb_.row >= 0) {
                            reset();
                            take_q(pb_);
                        }
                    }
                    pa_ = lp;
                    ta_ = lt;
                    load_tile(pa_, ta_, A, ph, pa_.row >= 0);
                    advance();
                    ph = lookup(lp, lt);
                    const bool live_b = pb_.row >= 0;
                    if (live_b) {
                        compute(pb_, tb_, B);
                        if (tb_ + 1 == pb_.le) {
                            finish(pb_);
                            if (pa_.row >= 0) {
                                reset();
                                take_q(pa_);
                            }
                        }
                    }
                    pb_ = lp;
                    tb_ = lt;
                    load_tile(pb_, tb_, B, ph, pb_.row >= 0);
                    advance();
                    ph = lookup(lp, lt);
                    if (pa_.row < 0) break;     // the tile after B's: none means B's was the last
                }
            } else
            // the same single bottom exit with three register tiles
            for (;;) {
                pc_ = lp;
                tc_ = lt;
                load_tile(pc_, tc_, C, ph, pc_.row >= 0);
                advance();
                ph = lookup(lp, lt);
                compute(pa_, ta_, A);
                if (ta_ + 1 == pa_.le) {
                    finish(pa_);
                    if (pb_.row >= 0) {
                        reset();
                        take_q(pb_);
                    }
                }
                pa_ = lp;
                ta_ = lt;
                load_tile(pa_, ta_, A, ph, pa_.row >= 0);
                advance();
                ph = lookup(lp, lt);
                if (pb_.row >= 0) {
                    compute(pb_, tb_, B);
                    if (tb_ + 1 == pb_.le) {
                        finish(pb_);
                        if (pc_.row >= 0) {
                            reset();
                            take_q(pc_);
                        }
                    }
                }
                pb_ = lp;
                tb_ = lt;
                load_tile(pb_, tb_, B, ph, pb_.row >= 0);
                advance();
                ph = lookup(lp, lt);
                if (pc_.row >= 0) {
                    compute(pc_, tc_, C);
                    if (tc_ + 1 == pc_.le) {
                        finish(pc_);
                        if (pa_.row >= 0) {
                            reset();
                            take_q(pa_);
                        }
                    }
                }
                if (pa_.row < 0) break;         // the tile after C's: none means C's was the last
            }
        }
        rb = rlim;
        preQ = false;
    }
    if constexpr (DEF) {
        if (deferred) {                    // the range's first cut piece, slot 0
            const int64_t base = (static_cast<int64_t>(w) * 2 * wpg + wi) * REP;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int head = 4 * g4 + r;
                if (head >= REP) continue;
                float* pa = p.part_acc + (base + head) * HD + 8 * i16;
                *reinterpret_cast<float4*>(pa) = make_float4(dom[0][r], dom[1][r], dom[2][r], dom[3][r]);
                *reinterpret_cast<float4*>(pa + 4) = make_float4(dom[4][r], dom[5][r], dom[6][r], dom[7][r]);
            }
            if (g4 == 0 && i16 < REP) reinterpret_cast<float2*>(p.part_ml)[base + i16] = make_float2(dmm, dL);
        }
    }
    if constexpr (UNITS) {
        // ---- shared-prefix units of the range: each wave multiplies its kv head's K/V tiles of the
        // group's shared keys against 16 query columns (16 / REP member tokens x REP heads), one pass per unit
        // instead of one per member; the tiles are read with the default cache policy so the other
        // units of the group find them in L2 / the last-level cache
        if (p.units != nullptr) {
            const auto pol = std::integral_constant<int, kTemporal>{};
            for (int r = max(r_s, rows_real); r < r_e; ++r) {
                const int64_t pr0 = pfx(r), pr1 = pfx(r + 1);
                if (pr0 >= u1) break;
                if (pr1 == pr0) continue;
                const int u = r - rows_real;
                const UnitRec* ur = p.units + u;
                Piece pc;
                pc.row = r;
                pc.t = 0;
                pc.g = wi;
                pc.kv_len = ld_uniform(&ur->keys, 0);
                pc.seq = ld_uniform(&ur->seq, 0);
                pc.shared_keys = 0;
                pc.lt = static_cast<int>(max(u0, pr0) - pr0);
                pc.le = static_cast<int>(min(u1, pr1) - pr0);
                const int n = ld_uniform(&ur->n, 0);
                MfTile TA, TB;
                int tile = pc.lt;
                // q before the first two tiles (the first compute's wait for q then leaves the tiles
                // in flight), loaded unconditionally (member 0's row past the unit's members) and
                // zeroed after: column c = REP j + h is member j's query head REP wi + h
                uint4 qv[4];
                const int qj = i16 / REP;
                {
                    const int tj = ur->tok[qj < n ? qj : 0];
                    const uint16_t* src = p.q + ((int64_t)tj * H + REP * wi + i16 % REP) * HD;
#pragma unroll
                    for (int st = 0; st < 4; ++st)
                        qv[st] = *reinterpret_cast<const uint4*>(src + (st >> 1) * 64 + g4 * 16 + (st & 1) * 8);
                }
                mf_load(pol, pc, tile, TA, lookup(pc, tile), true);
                mf_load(pol, pc, min(tile + 1, pc.le - 1), TB, lookup(pc, min(tile + 1, pc.le - 1)), tile + 1 < pc.le);
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    qm[st] = __builtin_bit_cast(bf16x8_t, qj < n ? qv[st] : make_uint4(0u, 0u, 0u, 0u));
                mm = kMinusHuge;
                lm = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) om[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                // single bottom exit (zero-size loads past the piece's end): every path back to the
                // loop head issues TA's loads before TB's, so each wait leaves the other tile in flight
                for (;;) {
                    mf_compute(pc, tile, TA);
                    ++tile;
                    mf_load(pol, pc, min(tile + 1, pc.le - 1), TA, lookup(pc, min(tile + 1, pc.le - 1)), tile + 1 < pc.le);
                    if (tile < pc.le) mf_compute(pc, tile, TB);
                    ++tile;
                    mf_load(pol, pc, min(tile + 1, pc.le - 1), TB, lookup(pc, min(tile + 1, pc.le - 1)), tile + 1 < pc.le);
                    if (tile >= pc.le) break;
                }
                // partials of all 16 columns: whole units in their own slot, cut ones in the range's
                const float L = xor32_sum(xor16_sum(lm));
                const bool whole = pc.lt == 0 && pc.le == pr1 - pr0;
                const int64_t base = whole ? (static_cast<int64_t>(u) * wpg + wi) * 16
                                           : ((static_cast<int64_t>(w) * 2 + (pr0 <= u0 ? 0 : 1)) * wpg + wi) * 16;
                float* acc_b = whole ? p.punit_acc : p.psh_acc;
                float* ml_b = whole ? p.punit_ml : p.psh_ml;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    float* pa = acc_b + (base + 4 * g4 + rr) * HD + 8 * i16;
                    *reinterpret_cast<float4*>(pa) = make_float4(om[0][rr], om[1][rr], om[2][rr], om[3][rr]);
                    *reinterpret_cast<float4*>(pa + 4) = make_float4(om[4][rr], om[5][rr], om[6][rr], om[7][rr]);
                }
                if (g4 == 0) reinterpret_cast<float2*>(ml_b)[base + i16] = make_float2(mm, L);
            }
        }
    }
}

// Log-sum-exp merge of cut rows (reference: kernels/paged_attention.cu:361-393). One workgroup
// per row (token, kv-head group): it recomputes, from the prefix the decode kernel stored, which
// workgroups covered the row (wave-uniform scalar arithmetic) and exits if one did. One thread
// per (query head, 4 dims) of the row (wpg * rep * HD / 4 slices: 512 at GQA 2, 2048 at GQA 8,
// which loop twice over the workgroup's 1024 threads) folds the row's pieces online,
// w0, w0 + 2, ... into one accumulator and w0 + 1, w0 + 3, ... into another, and combines the two
// (small batches cut a row into up to 8 pieces; their loads go out four at a time).
// Shared-prefix inputs of the merge (null when the launch has no units).
struct MergeUnits {
    const int* unit_count;
    const int2* tok_unit;
    const float* ptok_acc;
    const float* ptok_ml;
    const float* punit_acc;
    const float* punit_ml;
    const float* psh_acc;
    const float* psh_ml;
};

template <int HD, int SM>
__global__ __launch_bounds__(1024) void paged_merge2_kernel(uint16_t* __restrict__ out, const float* __restrict__ part_acc,
                                                          const float* __restrict__ part_ml,
                                                          const int* __restrict__ prefix,
                                                          const float* __restrict__ v_scale, int num_tokens, int n_kv,
                                                          int rep, int wpg, int G, MergeUnits mu) {
    constexpr int TPH = HD / 4;                       // threads per query head
    const int row = blockIdx.x;
    const int hg_count = n_kv / wpg;
    const int heads_per_row = wpg * rep;             // query heads of one row group
    const int rows_real = num_tokens * hg_count;
    const int n_units = mu.tok_unit != nullptr ? *mu.unit_count : 0;
    const int64_t U = prefix[rows_real + n_units];
    const int64_t pr0 = prefix[row], pr1 = prefix[row + 1];
    const int t = row / hg_count, hgi = row % hg_count;
    // a member token of a shared-prefix unit: its own row (keys after the shared prefix) and its
    // unit's column are merged here even when one range held either whole
    const int2 tu = (mu.tok_unit != nullptr) ? mu.tok_unit[t] : make_int2(-1, 0);
    const bool member = tu.x >= 0;
    if (!member && pr1 == pr0) return;
    // workgroup holding tile u: the largest w with w*U/G <= u
    // workgroup holding tile u: the largest w with w*U/G <= u; 32-bit division whenever U * G fits
    // (the 64-bit one is a long scalar routine)
    const bool narrow = (U + 1) * G <= 0xffffffffll;
    auto owner = [&](int64_t u) {
        return narrow ? static_cast<int>((static_cast<uint32_t>(u + 1) * static_cast<uint32_t>(G) - 1u) / static_cast<uint32_t>(U))
                      : static_cast<int>(((u + 1) * G - 1) / U);
    };
    auto first_tile = [&](int w) -> int64_t {    // first tile of workgroup w's range
        return narrow ? static_cast<int64_t>(static_cast<uint32_t>(w) * static_cast<uint32_t>(U) / static_cast<uint32_t>(G))
                      : w * U / G;
    };
    const int w0 = pr1 > pr0 ? owner(pr0) : 0, w1 = pr1 > pr0 ? owner(pr1 - 1) : -1;
    if (!member && w0 == w1) return;
    const int64_t q0 = member ? prefix[rows_real + tu.x] : 0, q1 = member ? prefix[rows_real + tu.x + 1] : 0;
    const int v0 = member ? owner(q0) : 0, v1 = member ? owner(q1 - 1) : -1;
    const float vfin = (SM == CVH_SCALE_PER_TENSOR) ? v_scale[0] : 1.f;
    // every thread owns slices (head, 4 dims) of the row; the pieces are folded into two
    // accumulators, even and odd positions from the range's first piece, which are combined at the
    // end. The loads of four consecutive pieces are issued together (indices of absent pieces
    // clamped to the first one, their folds skipped), so a row's piece loads are not one dependent
    // chain.
    struct Acc {
        float M, L;
        float4 A;
    };
    auto fold = [](Acc& c, float2 ml, float4 a) {
        const float Mn = fmaxf(c.M, ml.x);
        const float co = exp2f(c.M - Mn), cn = exp2f(ml.x - Mn);
        c.L = c.L * co + ml.y * cn;
        c.A.x = c.A.x * co + a.x * cn;
        c.A.y = c.A.y * co + a.y * cn;
        c.A.z = c.A.z * co + a.z * cn;
        c.A.w = c.A.w * co + a.w * cn;
        c.M = Mn;
    };
    // pieces of workgroups wb..we (slot 0 if the workgroup's range starts inside the row at r0,
    // else slot 1); idx(w, slot) is the piece's index into ml / acc
    auto fold_range = [&](Acc& c0, Acc& c1, int wb, int we, int64_t r0, const float* ml_b, const float* acc_b,
                          auto idx, int d0) {
        const int64_t i_first = idx(wb, r0 <= first_tile(wb) ? 0 : 1);
        for (int w = wb; w <= we; w += 4) {
            float2 ml[4];
            float4 a[4];
            bool ok[4];
            int64_t ft[5];
#pragma unroll
            for (int k = 0; k < 5; ++k) ft[k] = first_tile(w + k);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int ww = w + k;
                // (a workgroup whose range is empty — possible when G > U — wrote nothing)
                ok[k] = ww <= we && ft[k] != ft[k + 1];
                const int64_t i = ok[k] ? idx(ww, r0 <= ft[k] ? 0 : 1) : i_first;
                ml[k] = reinterpret_cast<const float2*>(ml_b)[i];
                a[k] = *reinterpret_cast<const float4*>(acc_b + i * HD + d0);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (ok[k]) fold((k & 1) ? c1 : c0, ml[k], a[k]);
        }
    };
    const int slices = heads_per_row * TPH;
    for (int sl = static_cast<int>(threadIdx.x); sl < slices; sl += static_cast<int>(blockDim.x)) {
        const int hh = sl / TPH;
        const int d0 = (sl % TPH) * 4;
        Acc c0{kMinusHuge, 0.f, make_float4(0.f, 0.f, 0.f, 0.f)}, c1 = c0;
        const int h = hgi * heads_per_row + hh;      // query head index within the token
        if (member && w0 == w1) {                    // the row's own keys, held whole by one range
            const int64_t i = (int64_t)t * n_kv * rep + h;
            fold(c0, reinterpret_cast<const float2*>(mu.ptok_ml)[i], *reinterpret_cast<const float4*>(mu.ptok_acc + i * HD + d0));
        } else {
            fold_range(c0, c1, w0, w1, pr0, part_ml, part_acc,
                       [&](int w, int slot) { return (static_cast<int64_t>(w) * 2 + slot) * heads_per_row + hh; }, d0);
        }
        if (member) {                                // the unit's column of this head
            const int wv = hh / rep, col = rep * tu.y + hh % rep;
            if (v0 == v1) {
                const int64_t i = (static_cast<int64_t>(tu.x) * wpg + wv) * 16 + col;
                fold(c0, reinterpret_cast<const float2*>(mu.punit_ml)[i], *reinterpret_cast<const float4*>(mu.punit_acc + i * HD + d0));
            } else {
                fold_range(c0, c1, v0, v1, q0, mu.psh_ml, mu.psh_acc,
                           [&](int w, int slot) { return ((static_cast<int64_t>(w) * 2 + slot) * wpg + wv) * 16 + col; }, d0);
            }
        }
        const float Mn = fmaxf(c0.M, c1.M);
        const float e0 = exp2f(c0.M - Mn), e1 = exp2f(c1.M - Mn);
        const float L = c0.L * e0 + c1.L * e1;
        float4 A;
        A.x = c0.A.x * e0 + c1.A.x * e1;
        A.y = c0.A.y * e0 + c1.A.y * e1;
        A.z = c0.A.z * e0 + c1.A.z * e1;
        A.w = c0.A.w * e0 + c1.A.w * e1;
        const float f = vfin / L;
        uint16_t* o = out + ((int64_t)t * n_kv * rep + h) * HD + d0;
        const uint32_t lo = f32_to_bf16_bits(A.x * f) | (uint32_t(f32_to_bf16_bits(A.y * f)) << 16);
        const uint32_t hi = f32_to_bf16_bits(A.z * f) | (uint32_t(f32_to_bf16_bits(A.w * f)) << 16);
        *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
    }
}

// Plan of a batch layout, built once and shared by every launch over the same block tables,
// token_seq, token_kv_len and partition count (the 28 layers of a decode step): the row
// prefix and token metadata the decode workgroups would derive, and each workgroup's first
// piece with the physical blocks of its first two tiles. One workgroup; the same first-row
// search and piece rules as the decode kernel.
__global__ __launch_bounds__(1024) void paged_plan_kernel(Params p, PlanRec* plan, int G, int one_block) {
    extern __shared__ int prefix[];
    const int hg_count = p.n_kv / p.wpg;
    const int rows_real = p.num_tokens * hg_count;
    // the token table sits after the largest prefix this launch may build (real rows + units)
    int2* tok = reinterpret_cast<int2*>(reinterpret_cast<char*>(prefix) + lds_tok_offset(rows_real + p.max_units));
    int rows = rows_real;
    if (p.units != nullptr) {       // shared-prefix units: group first, then the prefix over rows + units
        fill_tokens(p, tok);
        const int nu = build_units(p, tok);
        if (threadIdx.x == 0) *p.unit_count = nu;
        rows = rows_real + nu;
        const UnitRec* units = p.units;
        scan_rows(rows, [&](int r) {
            return r < rows_real ? (tok[r / hg_count].x + kTileKeys - 1) / kTileKeys
                                 : (units[r - rows_real].keys + kTileKeys - 1) / kTileKeys;
        }, prefix);
    } else {
        build_row_prefix(p, rows, hg_count, prefix, tok);
        for (int t = threadIdx.x; t < p.num_tokens; t += blockDim.x) p.shared_tok[t] = 0;
    }
    for (int i = threadIdx.x; i <= rows; i += blockDim.x) p.prefix_out[i] = prefix[i];
    for (int t = threadIdx.x; t < p.num_tokens; t += blockDim.x) p.plan_tok[t] = tok[t];
    __syncthreads();
    const int64_t U = prefix[rows];
    const int log2_bs = p.log2_bs;
    auto pf = [&](int i) { return prefix[i]; };
    for (int w = threadIdx.x; w < G; w += blockDim.x) {
        const int64_t u0 = w * U / G, u1 = (w + 1) * U / G;
        const int r_s = first_row(pf, rows, u0);
        const int rlim = min(rows_real, r_s + p.qrows);
        PlanRec rec = {};
        rec.row = -1;
        rec.r_s = r_s;
        rec.r_e = end_row(pf, rows, u0, u1, r_s);
        rec.U = static_cast<int>(U);
        // the empty-row pass of the last workgroup may walk trailing empty rows up to `rows`; the
        // ranges packed into one workgroup share the choice (the other path has a barrier)
        rec.win = 1;
        for (int v = w - w % p.pack; v < w - w % p.pack + p.pack; ++v) {
            const int64_t v0 = v * U / G, v1 = (v + 1) * U / G;
            const int vs = first_row(pf, rows, v0);
            if (!(end_row(pf, rows, v0, v1, vs) - vs <= kPlanWin - 1 && (v != G - 1 || rows - vs <= kPlanWin - 1)))
                rec.win = 0;
        }
        for (int i = 0; i <= kPlanWin; ++i) rec.pre[i] = prefix[min(r_s + i, rows)];
        const int t_s = r_s / hg_count;
        for (int j = 0; j < kPlanWin; ++j) {
            const int t = min(t_s + j, p.num_tokens - 1);
            rec.tkl[j] = tok[t].x;
            rec.tsq[j] = tok[t].y;
        }
        for (int r = r_s; r < rlim; ++r) {
            const int64_t pr0 = prefix[r], pr1 = prefix[r + 1];
            if (pr0 >= u1) break;
            if (pr1 == pr0) continue;
            const int t = r / hg_count;
            rec.row = r;
            rec.lt = static_cast<int>(max(u0, pr0) - pr0);
            rec.le = static_cast<int>(min(u1, pr1) - pr0);
            rec.kv_len = tok[t].x;
            rec.seq = tok[t].y;
            break;
        }
        if (rec.row >= 0) {
            const int64_t* table = p.block_tables + static_cast<int64_t>(rec.seq) * p.table_width;
            const int off = p.shared_tok[rec.row / hg_count];     // a member row starts after its shared keys
            auto phys = [&](int tile, int64_t& lo, int64_t& hi) {
                const int p0 = tile * kTileKeys;
                lo = max(table[(off + p0) >> log2_bs], int64_t{0});
                hi = one_block ? lo
                               : max(table[(off + min(p0 + kTileKeys / 2, rec.kv_len - 1)) >> log2_bs], int64_t{0});
            };
            phys(rec.lt, rec.a_lo, rec.a_hi);
            rec.b_ok = rec.lt + 1 < rec.le;
            if (rec.b_ok) phys(rec.lt + 1, rec.b_lo, rec.b_hi);
        }
        plan[w] = rec;
    }
}

// ---- host side ------------------------------------------------------------------------------------
int ilog2_pow2(int64_t v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int l = 0;
    while ((int64_t{1} << l) < v) ++l;
    return l;
}

// One wave per kv head of a row group. Eight kv heads share a workgroup when they can: a tile is
// then whole 1 KiB slot rows (all heads of 32 keys), contiguous in HBM.
int waves_per_group(int n_kv) { return (n_kv % 8 == 0) ? 8 : (n_kv % 4 == 0) ? 4 : (n_kv % 2 == 0) ? 2 : 1; }

// Upper bound of the tile count U, from what the host knows (widths, not lengths).
int64_t tile_bound(int64_t T, int n_kv, int64_t table_width, int block_size) {
    const int64_t per_row = (table_width * block_size + kTileKeys - 1) / kTileKeys;
    return T * (n_kv / waves_per_group(n_kv)) * per_row;
}

constexpr int kMaxAutoPartitions = 1024;
constexpr int64_t kMaxPiecesPerRow = 8;
int auto_partitions(int64_t T, int n_kv, int64_t table_width, int block_size) {
    // one partition per resident workgroup slot, but never less than 2 tiles per partition and
    // at most kMaxAutoPartitions workgroups: with one kv head (one-wave workgroups, a tp = 8
    // share of config 3) 2048 partitions ran 21.3 us + a 30.6 us op, 1024 ran 18.9 / 24.9 us
    // and at most kMaxPiecesPerRow partitions per row: a small batch cut finer only lengthens the
    // merge of each row (16 sequences: 256 partitions op 30.5 us, 128 partitions 26.6 us)
    const int64_t b = (tile_bound(T, n_kv, table_width, block_size) + 1) / 2;
    const int64_t rows = T * (n_kv / waves_per_group(n_kv));
    const int64_t slots = std::min({static_cast<int64_t>(kResidentWaves / waves_per_group(n_kv)),
                                    static_cast<int64_t>(kMaxAutoPartitions), kMaxPiecesPerRow * rows});
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(slots, b)));
}

// Workspace: prefix int32 [rows + 1] | part_acc float [G][2][WPG][REP][HD] | part_ml float2 [...]
// | plan: token metadata int2 [T], shared-prefix keys int32 [T], workgroup records PlanRec [G]
struct Workspace {
    size_t prefix_off, acc_off, ml_off, tok_off, shared_off, plan_off, total;
    // shared-prefix units (layouts sized for shared launches only)
    size_t units_off, ucount_off, tok_unit_off, ptok_acc_off, ptok_ml_off, punit_acc_off, punit_ml_off, psh_acc_off,
            psh_ml_off;
    int max_units;
};
size_t align256(size_t v) { return (v + 255) & ~size_t{255}; }
// groups have two or more tokens and units up to 16 / rep of them: at most T / 2 units (2 T / 3 at
// two tokens per unit)
int max_units_for(int64_t T, int rep) { return static_cast<int>(rep >= 8 ? (2 * T + 2) / 3 : (T + 1) / 2); }
Workspace ws_layout(int64_t T, int n_heads, int n_kv, int HD, int G, bool shared = false) {
    const int64_t hg = n_kv / waves_per_group(n_kv);
    const int64_t rows = T * hg + (shared ? max_units_for(T, n_heads / n_kv) : 0);
    const int64_t slots = static_cast<int64_t>(G) * 2 * (n_heads / hg);   // [G][2][WPG*REP]
    Workspace w;
    w.prefix_off = 0;
    w.acc_off = align256(static_cast<size_t>(rows + 1) * sizeof(int));
    w.ml_off = w.acc_off + align256(static_cast<size_t>(slots) * HD * sizeof(float));
    w.tok_off = w.ml_off + align256(static_cast<size_t>(slots) * 2 * sizeof(float));
    w.shared_off = w.tok_off + align256(static_cast<size_t>(T) * sizeof(int2));
    w.plan_off = w.shared_off + align256(static_cast<size_t>(T) * sizeof(int));
    w.total = w.plan_off + align256(static_cast<size_t>(G) * sizeof(PlanRec));
    w.max_units = shared ? max_units_for(T, n_heads / n_kv) : 0;
    w.units_off = w.ucount_off = w.tok_unit_off = w.ptok_acc_off = w.ptok_ml_off = w.punit_acc_off = w.punit_ml_off =
            w.psh_acc_off = w.psh_ml_off = w.total;
    if (shared) {
        const size_t wpg = static_cast<size_t>(waves_per_group(n_kv));
        const size_t mu = static_cast<size_t>(w.max_units);
        w.units_off = w.total;
        w.ucount_off = w.units_off + align256(mu * sizeof(UnitRec));
        w.tok_unit_off = w.ucount_off + 256;
        w.ptok_acc_off = w.tok_unit_off + align256(static_cast<size_t>(T) * sizeof(int2));
        w.ptok_ml_off = w.ptok_acc_off + align256(static_cast<size_t>(T) * n_heads * HD * sizeof(float));
        w.punit_acc_off = w.ptok_ml_off + align256(static_cast<size_t>(T) * n_heads * 2 * sizeof(float));
        w.punit_ml_off = w.punit_acc_off + align256(mu * wpg * 16 * HD * sizeof(float));
        w.psh_acc_off = w.punit_ml_off + align256(mu * wpg * 16 * 2 * sizeof(float));
        w.psh_ml_off = w.psh_acc_off + align256(static_cast<size_t>(G) * 2 * wpg * 16 * HD * sizeof(float));
        w.total = w.psh_ml_off + align256(static_cast<size_t>(G) * 2 * wpg * 16 * 2 * sizeof(float));
    }
    return w;
}

// kPhasePlanned: the decode phase reads the plan kPhasePlan left in the workspace
// kPhaseShared (with kPhasePlanned): the shared-prefix layout: units and member rows of the plan
enum Phase { kPhaseDecode = 1, kPhaseMerge = 2, kPhaseBoth = 3, kPhasePlanned = 4, kPhasePlan = 8, kPhaseShared = 16 };

template <typename K>
void launch_with_lds(K kernel, int G, int threads, size_t lds, hipStream_t s, const Params& p) {
    if (lds > 65536)   // large token counts: opt in to more than 64 KiB of dynamic LDS
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(lds));
    kernel<<<dim3(G), threads, lds, s>>>(p);
}

// planned: 0 = derive the layout, 1 = read the plan, 2 = read the plan and its shared-prefix keys
template <int HD, int REP, int SM, bool PLANNED, bool SHARED>
void launch_decode_p(int G, int threads, size_t lds, hipStream_t s, const Params& p, bool one_block) {
    if constexpr (REP >= 4) {
        if (p.wpg == 8 && p.pack == 1) {      // full row groups: hold the first cut piece (DEFER)
            if (one_block)
                launch_with_lds(paged_decode_kernel<HD, REP, SM, true, PLANNED, SHARED, true>, G, threads, lds, s, p);
            else
                launch_with_lds(paged_decode_kernel<HD, REP, SM, false, PLANNED, SHARED, true>, G, threads, lds, s, p);
            return;
        }
    }
    if (one_block)
        launch_with_lds(paged_decode_kernel<HD, REP, SM, true, PLANNED, SHARED>, G, threads, lds, s, p);
    else
        launch_with_lds(paged_decode_kernel<HD, REP, SM, false, PLANNED, SHARED>, G, threads, lds, s, p);
}
template <int HD, int REP, int SM>
void launch_decode(int G, int threads, size_t lds, hipStream_t s, const Params& p, bool one_block, int planned) {
    if (planned == 2)
        launch_decode_p<HD, REP, SM, true, true>(G, threads, lds, s, p, one_block);
    else if (planned == 1)
        launch_decode_p<HD, REP, SM, true, false>(G, threads, lds, s, p, one_block);
    else
        launch_decode_p<HD, REP, SM, false, false>(G, threads, lds, s, p, one_block);
}

template <int HD, int SM>
bool launch_decode_rep(int rep, int G, int threads, size_t lds, hipStream_t s, const Params& p, bool one_block,
                       int planned) {
    switch (rep) {
        case 1: launch_decode<HD, 1, SM>(G, threads, lds, s, p, one_block, planned); return true;
        case 2: launch_decode<HD, 2, SM>(G, threads, lds, s, p, one_block, planned); return true;
        case 4:
            if constexpr (HD == 128) { launch_decode<HD, 4, SM>(G, threads, lds, s, p, one_block, planned); return true; }
            return false;
        case 8:
            if constexpr (HD == 128) { launch_decode<HD, 8, SM>(G, threads, lds, s, p, one_block, planned); return true; }
            return false;
        default: return false;
    }
}

int paged_attention(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache, const float* k_scale,
                    const float* v_scale, const int64_t* block_tables, int64_t table_width, const int64_t* token_seq,
                    const int64_t* token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                    int block_size, int scale_mode, double scale, int partitions, void* workspace,
                    size_t workspace_bytes, cvh_stream_t stream, int phase, const int32_t* shared_blocks = nullptr) {
    if (num_tokens < 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width < 0 || partitions < 0)
        return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!block_tables || !token_seq || !token_kv_len) return CVH_ERR_INVALID_ARG;
    if ((phase & (kPhaseDecode | kPhaseMerge)) && (!out || !q || !k_cache || !v_cache || !k_scale || !v_scale))
        return CVH_ERR_INVALID_ARG;
    if (table_width == 0) return CVH_ERR_INVALID_ARG;
    if (n_heads % n_kv_heads != 0) return CVH_ERR_UNSUPPORTED;
    const int rep = n_heads / n_kv_heads;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return CVH_ERR_UNSUPPORTED;
    // GQA 4 and 8: each kv head is presented to the kernel as rep/2 virtual kv heads of 2 query heads
    // that read the same K/V (consecutive, so in one workgroup, reading each tile together: the
    // second read hits the cache). One wave then holds two query heads' accumulators, as at GQA 2,
    // instead of spilling 4 or 8 heads' worth of registers.
    const int kv_split = virtual_kv_split(rep, head_dim);
    const int kv_shift = kv_split == 4 ? 2 : kv_split == 2 ? 1 : 0;
    n_kv_heads *= kv_split;
    const int rep_v = rep / kv_split;
    const int lg = ilog2_pow2(block_size);
    if (lg < 4 || lg > 12) return CVH_ERR_UNSUPPORTED;
    if (head_dim != 64 && head_dim != 128) return CVH_ERR_UNSUPPORTED;
    if (scale_mode != CVH_SCALE_PER_TOKEN_HEAD && scale_mode != CVH_SCALE_PER_TENSOR) return CVH_ERR_UNSUPPORTED;
    if (table_width > (int64_t{0x7fffffff} >> lg)) return CVH_ERR_UNSUPPORTED;   // contexts < 2^31 keys
    const int wpg = waves_per_group(n_kv_heads);
    const int64_t rows = num_tokens * (n_kv_heads / wpg);
    if (rows > kMaxRows) return CVH_ERR_UNSUPPORTED;
    if (tile_bound(num_tokens, n_kv_heads, table_width, block_size) >= (int64_t{1} << 31) / 2)
        return CVH_ERR_UNSUPPORTED;
    const int G = partitions ? partitions : auto_partitions(num_tokens, n_kv_heads, table_width, block_size);
    // shared-prefix launches (plan_shared and the _shared launches) use the larger layout; units run
    // where the MFMA unit path exists (head_dim 128, one row group per token)
    const bool shared = (phase & kPhaseShared) || shared_blocks != nullptr;
    // (the plan's grouping compares token pairs: up to 2048 query tokens, far above a decode batch)
    const bool units_on = shared && head_dim == 128 && n_kv_heads == wpg && num_tokens <= 2048;
    const Workspace wl = ws_layout(num_tokens, n_heads, n_kv_heads, head_dim, G, shared);
    if (workspace == nullptr || workspace_bytes < wl.total) return CVH_ERR_WORKSPACE;
    char* wsb = static_cast<char*>(workspace);

    Params p{};
    p.out = static_cast<uint16_t*>(out);
    p.max_units = wl.max_units;
    p.unit_tokens = 16 / rep_v;
    if (units_on) {
        p.units = reinterpret_cast<UnitRec*>(wsb + wl.units_off);
        p.unit_count = reinterpret_cast<int*>(wsb + wl.ucount_off);
        p.tok_unit = reinterpret_cast<int2*>(wsb + wl.tok_unit_off);
        p.ptok_acc = reinterpret_cast<float*>(wsb + wl.ptok_acc_off);
        p.ptok_ml = reinterpret_cast<float*>(wsb + wl.ptok_ml_off);
        p.punit_acc = reinterpret_cast<float*>(wsb + wl.punit_acc_off);
        p.punit_ml = reinterpret_cast<float*>(wsb + wl.punit_ml_off);
        p.psh_acc = reinterpret_cast<float*>(wsb + wl.psh_acc_off);
        p.psh_ml = reinterpret_cast<float*>(wsb + wl.psh_ml_off);
    }
    p.prefix_out = reinterpret_cast<int*>(wsb + wl.prefix_off);
    PlanRec* plan = reinterpret_cast<PlanRec*>(wsb + wl.plan_off);
    p.plan = plan;
    p.plan_tok = reinterpret_cast<int2*>(wsb + wl.tok_off);
    p.shared_tok = reinterpret_cast<int*>(wsb + wl.shared_off);
    p.shared_blocks = shared_blocks;
    p.part_acc = reinterpret_cast<float*>(wsb + wl.acc_off);
    p.part_ml = reinterpret_cast<float*>(wsb + wl.ml_off);
    p.q = static_cast<const uint16_t*>(q);
    p.k_cache = k_cache;
    p.v_cache = v_cache;
    p.k_scale = k_scale;
    p.v_scale = v_scale;
    p.block_tables = block_tables;
    p.table_width = table_width;
    p.token_seq = token_seq;
    p.token_kv_len = token_kv_len;
    p.num_tokens = static_cast<int>(num_tokens);
    p.n_kv = n_kv_heads;
    p.kv_shift = kv_shift;
    p.wpg = wpg;
    p.G = G;
    // ranges per workgroup: one-wave row groups run 4 (or 2) to a workgroup, as long as that still
    // leaves a workgroup for every CU (tp = 8 share of config 3: op 27.7 -> 23.3 us per layer;
    // two-wave row groups measured 3% slower packed and stay one range per workgroup)
    p.pack = 1;
    for (int k = wpg == 1 ? 4 : 1; k > 1; k >>= 1)
        if (G % k == 0 && G / k >= kResidentWaves / 8) {
            p.pack = k;
            break;
        }
    // the per-wave K transpose areas of the full-row-group MFMA launches (launch_decode_p's DEFER
    // instantiation: GQA 4/8 at head_dim 128, 8 kv heads per workgroup)
    const size_t kt_area = (rep_v >= 4 && head_dim == 128 && wpg == 8 && p.pack == 1)
                                   ? static_cast<size_t>(wpg) * kKtWaveBytes : 0;
    {
        // q staging rows: as many as the LDS left by the row prefix and token table allows
        const size_t fixed = lds_q_offset(static_cast<int>(rows) + p.max_units, static_cast<int>(num_tokens)) + kt_area;
        const size_t per_row = static_cast<size_t>(wpg) * p.pack * rep_v * head_dim * 2;
        const int fit = fixed < kLdsBytes ? static_cast<int>((kLdsBytes - fixed) / per_row) : 0;
        if (fit < 1) return CVH_ERR_UNSUPPORTED;
        p.qrows = std::min(q_stage_rows(wpg * p.pack, rep_v, head_dim), fit);
    }
    p.log2_bs = lg;
    // The softmax scale is folded into q with log2(e) (base-2 softmax); a per-tensor K scale is a
    // device float, so the kernel folds it into q after reading it.
    p.q_scale = static_cast<float>(scale) * kLog2e;

    auto s = reinterpret_cast<hipStream_t>(stream);
    if (phase & kPhasePlan) {
        const size_t lds = lds_q_offset(static_cast<int>(rows) + p.max_units, static_cast<int>(num_tokens));
        const bool one_block = (1 << lg) >= kTileKeys;
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(paged_plan_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        paged_plan_kernel<<<1, 1024, lds, s>>>(p, plan, G, one_block ? 1 : 0);
        if (hipGetLastError() != hipSuccess) return CVH_ERR_LAUNCH;
    }
    if (phase & kPhaseDecode) {
        const int planned = (phase & kPhasePlanned) ? ((phase & kPhaseShared) ? 2 : 1) : 0;
        const size_t lds = lds_q_offset(static_cast<int>(rows) + p.max_units, static_cast<int>(num_tokens)) +
                           static_cast<size_t>(p.qrows) * wpg * p.pack * rep_v * head_dim * 2 + kt_area;
        const int WG = G / p.pack, nth = 64 * wpg * p.pack;
        const bool one_block = (1 << lg) >= kTileKeys;
        bool ok;
        if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
            ok = head_dim == 128
                         ? launch_decode_rep<128, CVH_SCALE_PER_TOKEN_HEAD>(rep_v, WG, nth, lds, s, p, one_block, planned)
                         : launch_decode_rep<64, CVH_SCALE_PER_TOKEN_HEAD>(rep_v, WG, nth, lds, s, p, one_block, planned);
        else
            ok = head_dim == 128 ? launch_decode_rep<128, CVH_SCALE_PER_TENSOR>(rep_v, WG, nth, lds, s, p, one_block, planned)
                                 : launch_decode_rep<64, CVH_SCALE_PER_TENSOR>(rep_v, WG, nth, lds, s, p, one_block, planned);
        if (!ok) return CVH_ERR_UNSUPPORTED;
        if (hipGetLastError() != hipSuccess) return CVH_ERR_LAUNCH;
    }
    MergeUnits mu{};
    if (units_on)
        mu = MergeUnits{p.unit_count, p.tok_unit, p.ptok_acc, p.ptok_ml, p.punit_acc, p.punit_ml, p.psh_acc, p.psh_ml};
    if ((phase & kPhaseMerge) && (G > 1 || units_on)) {
        const dim3 mgrid(static_cast<unsigned>(rows));
        const int nt = static_cast<int>(num_tokens);
        // one thread per (head, 4 dims) slice, at most 1024 (GQA 8's 2048 slices loop twice)
        const int m2 = std::min(1024, wpg * rep_v * head_dim / 4);
        if (head_dim == 128) {
            if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
                paged_merge2_kernel<128, CVH_SCALE_PER_TOKEN_HEAD><<<mgrid, m2, 0, s>>>(
                        p.out, p.part_acc, p.part_ml, p.prefix_out, v_scale, nt, n_kv_heads, rep_v, wpg, G, mu);
            else
                paged_merge2_kernel<128, CVH_SCALE_PER_TENSOR><<<mgrid, m2, 0, s>>>(
                        p.out, p.part_acc, p.part_ml, p.prefix_out, v_scale, nt, n_kv_heads, rep_v, wpg, G, mu);
        } else {
            if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
                paged_merge2_kernel<64, CVH_SCALE_PER_TOKEN_HEAD><<<mgrid, m2, 0, s>>>(
                        p.out, p.part_acc, p.part_ml, p.prefix_out, v_scale, nt, n_kv_heads, rep_v, wpg, G, mu);
            else
                paged_merge2_kernel<64, CVH_SCALE_PER_TENSOR><<<mgrid, m2, 0, s>>>(
                        p.out, p.part_acc, p.part_ml, p.prefix_out, v_scale, nt, n_kv_heads, rep_v, wpg, G, mu);
        }
        if (hipGetLastError() != hipSuccess) return CVH_ERR_LAUNCH;
    }
    return CVH_OK;
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_paged_attention_partitions(int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                              int64_t table_width, int block_size) {
    if (num_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width <= 0 || block_size <= 0 ||
        n_heads % n_kv_heads != 0)
        return 1;
    const int rep = n_heads / n_kv_heads;
    const int n_kv = n_kv_heads * cvh::virtual_kv_split(rep, head_dim);   // the kernel's kv heads, as in the launch
    return cvh::auto_partitions(num_tokens, n_kv, table_width, block_size);
}

extern "C" size_t cvh_paged_attention_workspace_bytes(int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                                      int64_t table_width, int block_size, int partitions) {
    if (num_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width <= 0 || block_size <= 0 ||
        partitions < 0 || n_heads % n_kv_heads != 0)
        return 0;
    const int rep = n_heads / n_kv_heads;
    const int n_kv = n_kv_heads * cvh::virtual_kv_split(rep, head_dim);   // the kernel's kv heads, as in the launch
    const int G = partitions ? partitions : cvh::auto_partitions(num_tokens, n_kv, table_width, block_size);
    return cvh::ws_layout(num_tokens, n_heads, n_kv, head_dim, G).total;
}

extern "C" size_t cvh_paged_attention_workspace_bytes_shared(int64_t num_tokens, int n_heads, int n_kv_heads,
                                                             int head_dim, int64_t table_width, int block_size,
                                                             int partitions) {
    if (num_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width <= 0 || block_size <= 0 ||
        partitions < 0 || n_heads % n_kv_heads != 0)
        return 0;
    const int rep = n_heads / n_kv_heads;
    const int n_kv = n_kv_heads * cvh::virtual_kv_split(rep, head_dim);
    const int G = partitions ? partitions : cvh::auto_partitions(num_tokens, n_kv, table_width, block_size);
    return cvh::ws_layout(num_tokens, n_heads, n_kv, head_dim, G, true).total;
}

#define CVH_PA_ARGS                                                                                                  \
    out, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq, token_kv_len, num_tokens,     \
            n_heads, n_kv_heads, head_dim, block_size, scale_mode, scale, partitions, workspace, workspace_bytes,    \
            stream
#define CVH_PA_PARAMS                                                                                                \
    void *out, const void *q, const uint8_t *k_cache, const uint8_t *v_cache, const float *k_scale,                \
            const float *v_scale, const int64_t *block_tables, int64_t table_width, const int64_t *token_seq,       \
            const int64_t *token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,             \
            int block_size, int scale_mode, double scale, int partitions, void *workspace, size_t workspace_bytes,  \
            cvh_stream_t stream

extern "C" int cvh_paged_attention_fp8_ex(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseBoth);
}
extern "C" int cvh_paged_attention_fp8_split_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseDecode);
}
extern "C" int cvh_paged_attention_fp8_merge_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseMerge);
}
extern "C" int cvh_paged_attention_fp8_planned(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseBoth | cvh::kPhasePlanned);
}
extern "C" int cvh_paged_attention_fp8_planned_split_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseDecode | cvh::kPhasePlanned);
}
extern "C" int cvh_paged_attention_fp8_planned_shared(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseBoth | cvh::kPhasePlanned | cvh::kPhaseShared);
}
extern "C" int cvh_paged_attention_fp8_planned_shared_split_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseDecode | cvh::kPhasePlanned | cvh::kPhaseShared);
}
extern "C" int cvh_paged_attention_fp8_planned_shared_merge_phase(CVH_PA_PARAMS) {
    return cvh::paged_attention(CVH_PA_ARGS, cvh::kPhaseMerge | cvh::kPhasePlanned | cvh::kPhaseShared);
}
extern "C" int cvh_paged_attention_plan(const int64_t* block_tables, int64_t table_width, const int64_t* token_seq,
                                        const int64_t* token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads,
                                        int head_dim, int block_size, int partitions, void* workspace,
                                        size_t workspace_bytes, cvh_stream_t stream) {
    return cvh::paged_attention(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, block_tables, table_width,
                                token_seq, token_kv_len, num_tokens, n_heads, n_kv_heads, head_dim, block_size,
                                CVH_SCALE_PER_TOKEN_HEAD, 1.0, partitions, workspace, workspace_bytes, stream,
                                cvh::kPhasePlan);
}

extern "C" int cvh_paged_attention_plan_shared(const int64_t* block_tables, int64_t table_width,
                                               const int64_t* token_seq, const int64_t* token_kv_len,
                                               const int32_t* shared_blocks, int64_t num_tokens, int n_heads,
                                               int n_kv_heads, int head_dim, int block_size, int partitions,
                                               void* workspace, size_t workspace_bytes, cvh_stream_t stream) {
    if (shared_blocks == nullptr) return CVH_ERR_INVALID_ARG;
    return cvh::paged_attention(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, block_tables, table_width,
                                token_seq, token_kv_len, num_tokens, n_heads, n_kv_heads, head_dim, block_size,
                                CVH_SCALE_PER_TOKEN_HEAD, 1.0, partitions, workspace, workspace_bytes, stream,
                                cvh::kPhasePlan, shared_blocks);
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

// ---- no-allocation entry point ------------------------------------------------------------------
// The split workspace of cvh_paged_attention_fp8 lives here instead of in a caller buffer: a
// file-scope device array, one copy per GPU, alive until the process ends. Host code must not use
// the array's name as an address (it is a host-side stand-in); the device address is looked up
// once per device with hipGetSymbolAddress and cached. Nothing in the workspace needs to start at
// zero (every launch writes what it later reads), so calls clear nothing; calls that overlap on
// one GPU (two streams, or two host threads) share the array and race.
namespace cvh {
namespace {
// 24 MiB. With automatic partitions every supported launch fits: partials are at most
// G * 2 * (heads per row group) = G * 2 * wpg * REP <= 2048 * 2 * 8 = 32768 slots of HD floats
// (16 MiB at HD 128, GQA 8; G * wpg never exceeds the 2048 resident waves), plus their (max, sum)
// pairs (256 KiB) and the prefix, token and plan records of at most 8192 rows (< 0.5 MiB).
// Explicit partition counts beyond that are rejected.
constexpr size_t kScratchBytes = size_t{24} << 20;
constexpr int kMaxDevices = 64;
}  // namespace
}  // namespace cvh

static __device__ __align__(256) unsigned char scratch[cvh::kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[cvh::kMaxDevices] = {};

// Device address of this GPU's scratch array (looked up on the first call on each device, with
// that device current), or nullptr if the lookup failed.
void* device_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= cvh::kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

extern "C" size_t cvh_paged_attention_noalloc_max_workspace(void) { return cvh::kScratchBytes; }

extern "C" int cvh_paged_attention_fp8_noalloc(void* out, const void* q, const uint8_t* k_cache,
                                               const uint8_t* v_cache, const float* k_scale, const float* v_scale,
                                               const int64_t* block_tables, int64_t table_width,
                                               const int64_t* token_seq, const int64_t* token_kv_len,
                                               int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                               int block_size, int scale_mode, double scale, int partitions,
                                               cvh_stream_t stream) {
    if (num_tokens == 0) return CVH_OK;
    if (num_tokens < 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width <= 0 || block_size <= 0 || partitions < 0)
        return CVH_ERR_INVALID_ARG;
    const size_t need = cvh_paged_attention_workspace_bytes(num_tokens, n_heads, n_kv_heads, head_dim, table_width,
                                                            block_size, partitions);
    if (need == 0) return CVH_ERR_INVALID_ARG;
    if (need > cvh::kScratchBytes) return CVH_ERR_WORKSPACE;   // beyond the fixed array: use cvh_paged_attention_fp8_ex
    void* ws = device_scratch();
    if (ws == nullptr) return CVH_ERR_LAUNCH;
    return cvh::paged_attention(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq,
                                token_kv_len, num_tokens, n_heads, n_kv_heads, head_dim, block_size, scale_mode, scale,
                                partitions, ws, cvh::kScratchBytes, stream, cvh::kPhaseBoth);
}
