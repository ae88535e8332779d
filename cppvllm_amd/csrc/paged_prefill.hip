// FP8-e4m3 paged attention for multi-token query rows (chunked prefill / prompt continuation)
// on gfx950 matrix cores.
//
// Reference semantics: kernels/paged_attention.cu:89-359 with T > S — every query token t attends
// causally to keys [0, token_kv_len[t]) of sequence token_seq[t] through its block table, GQA
// query heads share the kv head, K/V dequantised with per-(token, kv head) (or per-tensor)
// scales, softmax in fp32. The decode kernel walks one query token per row; here 16 consecutive
// query tokens of a sequence share every K/V tile, so the score and PV products are real dense
// contractions and run on MFMA (v_mfma_f32_16x16x32_bf16 for scores, _f16 for PV):
//
//   S^T[key][row] = K . Q^T   A = K   (16 keys x 32 d, e4m3 -> bf16 exact),  B = Q^T (bf16)
//   O^T[d][row]  += V^T . P^T A = V^T (16 d x 32 keys, fp16 via LDS),        B = P^T (fp16, v scale folded)
//
// Both products put one query row per lane column (lane % 16), so the row's softmax state, its
// causal mask and its output accumulators live in the same lanes with no cross-lane shuffles
// except the 4-way max/sum over lane groups. The contraction index order inside an MFMA is
// free as long as A and B agree: lane group g = lane / 16 supplies d in
// {c*64 + g*16 + h*8 + 0..7} for step s = 2c + h, and the 8 contiguous keys {8g + 0..7} of a
// 32-key PV step (the score MFMAs take their K rows in the matching order, so these are the keys
// the lane's S^T outputs hold and its V^T fragment is one 16-byte LDS read).
//
// Work: a workgroup = (64 consecutive query tokens, one kv head), 4 waves of 16 tokens each
// (REP query heads per token), walking the keys of the tokens' sequence in 64-key tiles (staged
// as two 32-key load groups). The 256 threads load each tile once for all four waves: K is converted to bf16 and V transposed to fp16
// (each thread loads a 4 key x 4 d byte block with dword loads, transposes it with v_perm_b32 and
// converts it) into a double-buffered LDS tile, so one tile is multiplied while the next sits in
// registers and the one after is in flight. Tokens of different sequences inside the 64 run as
// separate passes (rows outside the pass are masked), so any ragged batch is valid input.
#include <hip/hip_runtime.h>

#include <math.h>

#include "cvh_device.h"

namespace cvh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_p __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kHD = 128;
constexpr int kQTok = 16;          // query tokens per wave
constexpr int kTile = 64;          // keys per tile (multiplied between two synchronisations)
constexpr int kSub = 32;           // keys per load group (a tile is staged as two)
// LDS row strides chosen against bank conflicts (64 banks of 4 bytes):
//  * V^T rows are 36 dwords (64 keys + 8 pad fp16), 16-byte aligned, so a lane's 16 fragment
//    reads are ds_read_b128 at immediate offsets from one address (rows j*16 + i16 lie
//    j * 2304 bytes apart); the 16 rows read by a quarter-wave land 4 banks apart;
//  * K rows are 136 bf16 (272 bytes): the 16 rows read by one 16-byte load land 4 banks apart.
constexpr int kVtStride = 72;      // fp16 per LDS row of V^T
constexpr float kLog2eP = 1.4426950408889634f;
constexpr float kNegHuge = -1e30f;
constexpr float kRescaleLog2 = 8.0f;   // tolerated staleness of the running max (log2 units)

// K/V and scale tiles are read with raw buffer loads: a scalar descriptor per wave and tile (the
// block's first key of the tile as base, the valid keys as size) and per-thread offsets fixed for
// the whole launch, so addressing costs no vector instructions and keys past the context (or in
// a block whose table entry is negative) read as zeros without a branch.
constexpr int kBufWord3 = 0x00020000;      // raw buffer, 32-bit data format
constexpr int kNt = 2;                     // non-temporal: each K/V byte is read once per workgroup
typedef unsigned int u32x4_p __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufWord3);
}

template <bool HI> __device__ __forceinline__ uint32_t pk_bf16(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_p));
}

// The PV product runs in fp16: V e4m3 -> fp16 is exact (like bf16), and p (times the V scale,
// <= 2^8 x the scale) keeps 11 significant bits instead of bf16's 8, so a row dominated by a few
// 20x-outlier values stays within an output ulp of the fp32 restatement.
typedef _Float16 f16x2_p __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
template <bool HI> __device__ __forceinline__ uint32_t pk_f16(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_p));
}

// max / sum over the 4 lane groups (lanes l, l^16, l^32, l^48), xor 16 then xor 32, with the
// gfx950 permlane swaps (with both operands = v, the returned pair holds, per lane, its own value
// and its partner's) instead of LDS-routed ds_bpermute
__device__ __forceinline__ float max_groups(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_groups(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int kWgTok = 4 * kQTok;  // query tokens per workgroup: 16 per wave
constexpr int kKRow = kHD + 8;      // bf16 per LDS row of K (272 bytes: 16 rows of a read hit distinct banks)

// A double-buffered K/V tile in LDS: K as bf16 rows, V transposed (V^T rows = d), scales.
struct PrefillLds {
    uint16_t k[2][kTile][kKRow];
    uint16_t vt[2][kHD * kVtStride];
    float ks[2][kTile], vs[2][kTile];
    int64_t tseq[kWgTok];
    int tkvl[kWgTok];
};

// The workgroup's share of one 32-key load group as loaded by thread tid (raw e4m3 and f32
// scales): K: key tid/8, bytes (tid%8)*16 .. +16;  V: keys 4*(tid/32) + e, bytes 4*(tid%32) .. +4;
// scales: key tid/8. Every wave's keys lie in one half of the group (wave w: keys 8w .. 8w+7),
// so with 16-key blocks each wave still reads from a single block.
struct TileRegs {
    uint4 k;
    uint32_t v[4];
    float ks, vs;
};

// KSPLIT: 8 waves; waves 4..7 take the second half of every run's key tiles for the same 64
// tokens, with their own LDS tiles, and hand their (m, l, O) to waves 0..3 through LDS at the end.
template <int REP, int SCALE_MODE, bool KSPLIT>
__global__ __launch_bounds__(KSPLIT ? 512 : 256, KSPLIT ? 1 : 2) void paged_prefill_kernel(
        uint16_t* __restrict__ out, const uint16_t* __restrict__ q, const uint8_t* __restrict__ kc,
        const uint8_t* __restrict__ vc, const float* __restrict__ ksc, const float* __restrict__ vsc,
        const int64_t* __restrict__ tables, int64_t W, const int64_t* __restrict__ token_seq,
        const int64_t* __restrict__ token_kv_len, int T, int H, int KV, int lg_bs, float scale_log2,
        const int* __restrict__ order) {
    constexpr int NH = KSPLIT ? 2 : 1;
    __shared__ __align__(16) PrefillLds smv[NH];
    __shared__ int half_sync[2];
    const int tid = threadIdx.x & 255, lane = tid & 63;
    const int half = KSPLIT ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 8) : 0;
    PrefillLds& sm = smv[half];
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // item = (64-token group, kv head), kv heads fastest along the 1-D grid. With a plan the groups
    // come from order[] (descending key-tile count); without one they run last group first: a
    // prompt's later groups attend over more keys, so this starts the long items of each prompt
    // early (4096-token step of config-5 prompts: 46.1 -> 41.8 us against first group first)
    const int item_group = order ? order[blockIdx.x / KV]
                                 : static_cast<int>(gridDim.x) / KV - 1 - static_cast<int>(blockIdx.x) / KV;
    const int kvh = static_cast<int>(blockIdx.x) % KV;
    const int t0 = item_group * kWgTok;
    const int g = lane >> 4, i16 = lane & 15;
    const int BS = 1 << lg_bs, bs_mask = BS - 1;
    const int64_t row_bytes = static_cast<int64_t>(KV) * kHD;      // one slot row, all kv heads

    if (threadIdx.x < 2) half_sync[threadIdx.x] = 0;
    // token metadata of the 64 tokens -> LDS (clamped like the decode kernel)
    if (half == 0 && tid < kWgTok) {
        const int t = t0 + tid;
        int64_t sq = -1, kv = 0;
        if (t < T) {
            sq = token_seq[t];
            kv = token_kv_len[t];
            if (sq < 0 || kv < 0) kv = 0;
            if (kv > (W << lg_bs)) kv = W << lg_bs;
        }
        smv[0].tseq[tid] = sq;
        smv[0].tkvl[tid] = static_cast<int>(kv);
    }
    // this wave's 16 query rows (token t0 + 16w + i16, heads kvh*REP + rb) as MFMA B operands:
    // step s = 2c + h covers d = c*64 + g*16 + h*8 + 0..7
    const int tq = t0 + 16 * w + i16;
    bf16x8_t qop[REP][4];
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        const uint16_t* qr = q + (static_cast<int64_t>(tq < T ? tq : 0) * H + kvh * REP + rb) * kHD;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (tq < T) v = *reinterpret_cast<const uint4*>(qr + (st >> 1) * 64 + g * 16 + (st & 1) * 8);
            qop[rb][st] = __builtin_bit_cast(bf16x8_t, v);
        }
    }
    __syncthreads();

    f32x4_t o[REP][8];
    float m[REP], lsum[REP];
    // Power-of-two range of the fp16 PV weights, wave-uniform: w = exp2(s - m - e) * vs with
    // vs * 2^-e <= 2^7 for the largest V scale of the tile, so w <= 2^15 whatever the magnitude of
    // V (per-(token, head) or per-tensor scales from 1e-11 to 1e38) and the tile's largest weights
    // stay normal fp16 numbers. e acts as an offset of the running max: l and O carry the same
    // 2^-e, a change of e rescales both like a move of the max, and O / l is unchanged.
    float ew = 0.f;
    float win_hi = 128.f, win_lo = 1.0f / 64.f;     // [2^(e-6), 2^(e+7)): the tile max needs no new e
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        m[rb] = kNegHuge;
        lsum[rb] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[rb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    const float ks_tensor = SCALE_MODE == CVH_SCALE_PER_TENSOR ? ksc[0] : 0.f;
    const float vs_tensor = SCALE_MODE == CVH_SCALE_PER_TENSOR ? vsc[0] : 0.f;

    // every wave sees all 64 tokens (lane l <-> token l) so the run loop is uniform across waves
    const int64_t all_seq = smv[0].tseq[lane];
    const int all_kvl = smv[0].tkvl[lane];
    const int64_t my_seq = smv[0].tseq[16 * w + i16];
    const int my_kvl = smv[0].tkvl[16 * w + i16];
    // this wave's keys: [8w, 8w + 8) of every tile; with 16-key blocks waves 2, 3 read the second block
    const int khalf = (BS < kSub && w >= 2) ? 16 : 0;
    const int khalf_span = BS < kSub ? 16 : kSub;
    const uint32_t row_bytes32 = static_cast<uint32_t>(row_bytes);
    const uint32_t k_off = static_cast<uint32_t>((tid >> 3) - khalf) * row_bytes32 + kvh * kHD + (tid & 7) * 16;
    // V: this thread's 4-key group (vkg) and 4-byte d block (vdc); a wave covers 16 keys (one block
    // at 16-key blocks) x 64 d, a half-wave 4 key groups x 8 d blocks, so the V^T stores of a
    // half-wave cover 32 rows (2-way bank conflicts at most)
    const int vkg = (lane & 3) + 4 * (w >> 1), vdc = (lane >> 2) + 16 * (w & 1);
    const uint32_t v_off = static_cast<uint32_t>(4 * vkg - khalf) * row_bytes32 + kvh * kHD + vdc * 4;
    // K row position in LDS: key 32a + 8q + 4b + r of a tile sits at row 16(2a + b) + 4q + r, so the
    // score rows of block kb (lane group g, element r) are keys 32(kb/2) + 8g + 4(kb%2) + r and each
    // lane group's eight PV keys of a 32-key step are contiguous in V^T
    const int kk = tid >> 3;
    const int k_pos = 16 * ((kk >> 2) & 1) + 4 * (kk >> 3) + (kk & 3);
    const uint32_t s_off = static_cast<uint32_t>((tid >> 3) - khalf) * 4u;
    // The 4 waves sharing a tile buffer synchronise per tile. With two halves this is a counter in
    // LDS per half instead of the workgroup barrier, so the halves run their own tile counts and
    // drift apart: the two waves of a SIMD then tend to be in different phases (one issuing MFMA,
    // the other softmax VALU). The wait is bounded (a lost wave cannot hang the launch).
    int passed = 0;
    auto tile_barrier = [&]() {
        if constexpr (!KSPLIT) {
            __syncthreads();
        } else {
            ++passed;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_fetch_add(&half_sync[half], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            for (int spin = 0; spin < (1 << 22); ++spin) {
                const int c = __builtin_amdgcn_readfirstlane(
                        __hip_atomic_load(&half_sync[half], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
                if (c >= 4 * passed) break;
                __builtin_amdgcn_s_sleep(1);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
    };
    uint64_t todo = __builtin_amdgcn_ballot_w64(all_kvl > 0);
    while (todo) {
        const int leader = __builtin_ctzll(todo);
        const int64_t rseq =
                static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(all_seq), leader))) |
                (static_cast<int64_t>(__builtin_amdgcn_readlane(static_cast<int>(all_seq >> 32), leader)) << 32);
        const bool in_run = all_seq == rseq && all_kvl > 0;
        todo &= ~__builtin_amdgcn_ballot_w64(in_run);
        int kmax_l = in_run ? all_kvl : 0;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) kmax_l = max(kmax_l, __shfl_xor(kmax_l, d, 64));
        const int kmax = __builtin_amdgcn_readfirstlane(kmax_l);
        // this half's key range: tiles [0, n0) or [n0, ntiles)
        const int ntiles = (kmax + kTile - 1) / kTile;
        const int n0 = KSPLIT ? (ntiles + 1) >> 1 : ntiles;
        const int n_iter = half ? ntiles - n0 : n0;
        const int kbeg = half ? n0 * kTile : 0;
        const int kend = half ? kmax : min(kmax, n0 * kTile);
        const int64_t* trow = tables + rseq * W;
        const int row_kvl = (my_seq == rseq) ? my_kvl : 0;
        // keys this wave's rows need in the run: tiles past it are staged for the other waves only
        int wk = row_kvl;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) wk = max(wk, __shfl_xor(wk, d, 64));
        const int wave_kmax = __builtin_amdgcn_readfirstlane(wk);
        // tiles below every row's length need no causal mask (rows outside the run have length 0)
        int wn = row_kvl;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) wn = min(wn, __shfl_xor(wn, d, 64));
        const int wave_kmin = __builtin_amdgcn_readfirstlane(wn);

        // cooperative load of tile kb0 into registers (keys >= kend and negative table entries
        // read as zeros; a negative entry inside a context is invalid input)
        auto load_tile = [&](int kb0, TileRegs& r) {
            const int kfirst = kb0 + khalf;                       // first key of this wave's block range
            const int span = min(max(kend - kfirst, 0), khalf_span);
            const int64_t blk = span > 0 ? trow[kfirst >> lg_bs] : -1;
            const int valid = blk >= 0 ? span : 0;
            const int64_t slot0 = (blk << lg_bs) + (kfirst & bs_mask);
            const uint32_t vb = static_cast<uint32_t>(valid) * static_cast<uint32_t>(row_bytes);
            const auto rk = rsrc(kc + slot0 * row_bytes, vb);
            const auto rv = rsrc(vc + slot0 * row_bytes, vb);
            const u32x4_p kw = __builtin_amdgcn_raw_buffer_load_b128(rk, k_off, 0, kNt);
            r.k = make_uint4(kw[0], kw[1], kw[2], kw[3]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                r.v[e] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rv, v_off + e * row_bytes32, 0, kNt));
            if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
                const int64_t si = ((((blk < 0 ? 0 : blk) * KV + kvh)) << lg_bs) + (kfirst & bs_mask);
                r.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(ksc + si, valid * 4u), s_off, 0, kNt));
                r.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(vsc + si, valid * 4u), s_off, 0, kNt));
            } else {
                const bool ok = s_off < valid * 4u;
                r.ks = ok ? ks_tensor : 0.f;
                r.vs = ok ? vs_tensor : 0.f;
            }
        };
        // registers -> LDS buffer: K converted to bf16, V transposed to fp16 (4x4 byte blocks with
        // v_perm_b32) and converted, scales
        auto store_tile = [&](int buf, int sub, const TileRegs& r) {
            {
                const int key = 2 * 16 * sub + k_pos, cc = tid & 7;
                const uint4 lo = make_uint4(pk_bf16<false>(r.k.x), pk_bf16<true>(r.k.x), pk_bf16<false>(r.k.y),
                                            pk_bf16<true>(r.k.y));
                const uint4 hi = make_uint4(pk_bf16<false>(r.k.z), pk_bf16<true>(r.k.z), pk_bf16<false>(r.k.w),
                                            pk_bf16<true>(r.k.w));
                *reinterpret_cast<uint4*>(&sm.k[buf][key][cc * 16]) = lo;
                *reinterpret_cast<uint4*>(&sm.k[buf][key][cc * 16 + 8]) = hi;
            }
            {
                const int kg = vkg, c = vdc;
                const uint32_t w0 = r.v[0], w1 = r.v[1], w2 = r.v[2], w3 = r.v[3];
                const uint32_t a = __builtin_amdgcn_perm(w1, w0, 0x05010400u);   // w0b0 w1b0 w0b1 w1b1
                const uint32_t b = __builtin_amdgcn_perm(w1, w0, 0x07030602u);   // w0b2 w1b2 w0b3 w1b3
                const uint32_t cc = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
                const uint32_t dd = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
                const uint32_t tr[4] = {__builtin_amdgcn_perm(cc, a, 0x05040100u),
                                        __builtin_amdgcn_perm(cc, a, 0x07060302u),
                                        __builtin_amdgcn_perm(dd, b, 0x05040100u),
                                        __builtin_amdgcn_perm(dd, b, 0x07060302u)};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    uint32_t* dst = reinterpret_cast<uint32_t*>(&sm.vt[buf][(c * 4 + e) * kVtStride + sub * kSub + 4 * kg]);
                    dst[0] = pk_f16<false>(tr[e]);
                    dst[1] = pk_f16<true>(tr[e]);
                }
            }
            if ((tid & 7) == 0) {
                sm.ks[buf][2 * 16 * sub + k_pos] = r.ks * scale_log2;
                sm.vs[buf][2 * 16 * sub + k_pos] = r.vs;
            }
        };
        // kb = 16-key row block of the tile (4), PV step h = keys 32h .. 32h + 31 (2)
        auto compute = [&](int buf, int kb0, bool masked) {
            f32x4_t sc[4][REP];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                bf16x8_t ka[4];
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    ka[st] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                                                  &sm.k[buf][kb * 16 + i16][(st >> 1) * 64 + g * 16 + (st & 1) * 8]));
#pragma unroll
                for (int rb = 0; rb < REP; ++rb) {
                    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int st = 0; st < 4; ++st)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[st], qop[rb][st], acc, 0, 0, 0);
                    sc[kb][rb] = acc;
                }
            }
            float ksr[4][4], vsr[4][4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const float4 a = *reinterpret_cast<const float4*>(&sm.ks[buf][kb * 16 + g * 4]);
                const float4 b = *reinterpret_cast<const float4*>(&sm.vs[buf][kb * 16 + g * 4]);
                ksr[kb][0] = a.x; ksr[kb][1] = a.y; ksr[kb][2] = a.z; ksr[kb][3] = a.w;
                vsr[kb][0] = b.x; vsr[kb][1] = b.y; vsr[kb][2] = b.z; vsr[kb][3] = b.w;
            }
            // the tile's largest V scale (scales are >= 0; keys past a context read 0); a new
            // range exponent only when it leaves [2^-6, 2^7) x 2^e
            // (each lane tests its own 16 keys; only when some lane is above the window, or none
            // reaches it, does the wave reduce the maximum and move e, kept within [-100, 120] so
            // that p' = exp2(s - m - e) <= 2^108 stays a finite fp32)
            const float e_old = ew;
            {
                float vm = 0.f;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    vm = fmaxf(vm, fmaxf(fmaxf(vsr[kb][0], vsr[kb][1]), fmaxf(vsr[kb][2], vsr[kb][3])));
                const uint64_t above = __builtin_amdgcn_ballot_w64(vm >= win_hi);
                const uint64_t inside = __builtin_amdgcn_ballot_w64(vm >= win_lo);
                if (above != 0 || inside == 0) {
                    vm = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(max_groups(vm))));
                    if (vm > 0.f) {
                        const int vexp = ((__float_as_int(vm) >> 23) & 0xff) - 127;   // floor(log2 vm), vm normal
                        const int en = min(max(vexp - 6, -100), 120);
                        ew = static_cast<float>(en);
                        win_hi = __builtin_ldexpf(1.0f, en + 7);
                        win_lo = __builtin_ldexpf(1.0f, en - 6);
                    }
                }
            }
            uint32_t pp[REP][2][4];
#pragma unroll
            for (int rb = 0; rb < REP; ++rb) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sc[kb][rb][r] *= ksr[kb][r];
                if (masked) {              // wave-uniform: only tiles reaching past a row's length
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (kb0 + (kb >> 1) * 32 + g * 8 + (kb & 1) * 4 + r >= row_kvl) sc[kb][rb][r] = -INFINITY;
                }
                float mt = kNegHuge;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) mt = fmaxf(mt, sc[kb][rb][r]);
                mt = max_groups(mt);
                // the running max only moves when the tile's max exceeds it by more than 2^8 (a
                // stale max leaves p <= 2^8: exact in fp32, the same relative bf16 rounding), so
                // most tiles skip the rescale of O
                const float mn0 = mt > m[rb] + kRescaleLog2 ? mt : m[rb];
                const float alpha = __builtin_amdgcn_exp2f((m[rb] + e_old) - (mn0 + ew));
                m[rb] = mn0;
                const float mn = mn0 + ew;                                   // offset max of this tile's p
                float ps = 0.f;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; r += 2) {
                        const float p0 = __builtin_amdgcn_exp2f(sc[kb][rb][r] - mn);
                        const float p1 = __builtin_amdgcn_exp2f(sc[kb][rb][r + 1] - mn);
                        ps += p0 + p1;
                        pp[rb][kb >> 1][(kb & 1) * 2 + r / 2] = pack_f16x2(p0 * vsr[kb][r], p1 * vsr[kb][r + 1]);
                    }
                lsum[rb] = lsum[rb] * alpha + ps;
                if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {     // wave-uniform: the max moved
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[rb][j] *= alpha;
                }
            }
            // PV, one 32-key step at a time: its V^T fragments serve every head
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint4 va = *reinterpret_cast<const uint4*>(&sm.vt[buf][(j * 16 + i16) * kVtStride + h * kSub + g * 8]);
#pragma unroll
                    for (int rb = 0; rb < REP; ++rb)
                        o[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, va),
                                                                          __builtin_bit_cast(f16x8_t, pp[rb][h]),
                                                                          o[rb][j], 0, 0, 0);
                }
            }
        };

        // two-stage pipeline: tile i is multiplied from LDS while tile i+1 sits in registers (two
        // load groups, stored to the other buffer after the multiply) and tile i+2's loads are in
        // flight
        TileRegs ra, rb2;
        load_tile(kbeg, ra);
        load_tile(kbeg + kSub, rb2);
        store_tile(0, 0, ra);
        store_tile(0, 1, rb2);
        load_tile(kbeg + kTile, ra);
        load_tile(kbeg + kTile + kSub, rb2);
        tile_barrier();
        for (int i = 0, kb0 = kbeg; i < n_iter; ++i, kb0 += kTile) {
            const int buf = i & 1;
            if (kb0 < kend && kb0 < wave_kmax) compute(buf, kb0, kb0 + kTile > wave_kmin);
            if (kb0 + kTile < kend) {
                store_tile(buf ^ 1, 0, ra);
                store_tile(buf ^ 1, 1, rb2);
                load_tile(kb0 + 2 * kTile, ra);
                load_tile(kb0 + 2 * kTile + kSub, rb2);
            }
            tile_barrier();
        }
    }

    if constexpr (KSPLIT) {
        // waves 4..7 -> LDS (the tiles are no longer read): per (rb, value) a row of 256 lanes
        constexpr int kVals = 2 + 32;
        static_assert(sizeof(smv) >= REP * kVals * 256 * sizeof(float), "combine buffer");
        float* xs = reinterpret_cast<float*>(smv);
        __syncthreads();                 // both halves are done with their tiles
        if (half) {
#pragma unroll
            for (int rb = 0; rb < REP; ++rb) {
                float* d = xs + rb * kVals * 256 + tid;
                d[0] = m[rb] + ew;                  // l and O of this half carry 2^-ew
                d[256] = sum_groups(lsum[rb]);
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) d[(2 + 4 * j + e) * 256] = o[rb][j][e];
            }
        }
        __syncthreads();
        if (half) return;
        if (tq >= T) return;
#pragma unroll
        for (int rb = 0; rb < REP; ++rb) {
            const float* d = xs + rb * kVals * 256 + tid;
            const float m0 = m[rb] + ew, m1 = d[0], l1 = d[256];
            const float mn = fmaxf(m0, m1);
            const float a0 = __builtin_amdgcn_exp2f(m0 - mn), a1 = __builtin_amdgcn_exp2f(m1 - mn);
            const float l = sum_groups(lsum[rb]) * a0 + l1 * a1;
            const float inv = l > 0.f ? 1.0f / l : 0.f;
            uint16_t* orow = out + (static_cast<int64_t>(tq) * H + kvh * REP + rb) * kHD;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = (o[rb][j][e] * a0 + d[(2 + 4 * j + e) * 256] * a1) * inv;
                *reinterpret_cast<uint2*>(orow + j * 16 + g * 4) =
                        make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            }
        }
        return;
    }

    if (tq >= T) return;
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        const float l = sum_groups(lsum[rb]);
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        uint16_t* orow = out + (static_cast<int64_t>(tq) * H + kvh * REP + rb) * kHD;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint2 v = make_uint2(pack_bf16x2(o[rb][j][0] * inv, o[rb][j][1] * inv),
                                       pack_bf16x2(o[rb][j][2] * inv, o[rb][j][3] * inv));
            *reinterpret_cast<uint2*>(orow + j * 16 + g * 4) = v;
        }
    }
}

int ilog2_exact(int v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

template <int REP, int SM>
int launch_rep(uint16_t* out, const uint16_t* q, const uint8_t* kc, const uint8_t* vc, const float* ks,
               const float* vs, const int64_t* tables, int64_t W, const int64_t* tseq, const int64_t* tkvl, int T,
               int H, int KV, int lg, float sl2, const int* order, hipStream_t s) {
    const unsigned gx = static_cast<unsigned>((T + kWgTok - 1) / kWgTok);
    if (order) {
        // longest items first, each split over two 4-wave halves: the dispatcher starts the long
        // items at once and the short ones fill the slots they leave
        paged_prefill_kernel<REP, SM, true><<<dim3(gx * KV), 512, 0, s>>>(out, q, kc, vc, ks, vs, tables, W, tseq,
                                                                           tkvl, T, H, KV, lg, sl2, order);
    } else {
        paged_prefill_kernel<REP, SM, false><<<dim3(gx * KV), 256, 0, s>>>(out, q, kc, vc, ks, vs, tables, W, tseq,
                                                                           tkvl, T, H, KV, lg, sl2, nullptr);
    }
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

// ---- plan: 64-token groups by descending key-tile count -------------------------------------
// One 1024-thread workgroup: the cost of a group is its largest clamped token_kv_len in 32-key
// tiles (buckets capped at kCostBuckets - 1); a counting sort writes the groups in descending
// cost order (ties in any order: the order only steers the dispatcher, results do not depend on
// it). Workspace: cost[groups] then order[groups] (int32).
constexpr int kCostBuckets = 1024;
constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(const int64_t* __restrict__ token_seq,
                                                                    const int64_t* __restrict__ token_kv_len, int T,
                                                                    int64_t max_keys, int* __restrict__ cost,
                                                                    int* __restrict__ order) {
    __shared__ int hist[kCostBuckets];
    __shared__ int scan[kCostBuckets];
    const int tid = threadIdx.x;
    const int groups = (T + kWgTok - 1) / kWgTok;
    for (int i = tid; i < kCostBuckets; i += kPlanThreads) hist[i] = 0;
    __syncthreads();
    // 16 lanes per group, 4 tokens per lane (coalesced), max over the 16 lanes
    for (int gb = 0; gb < groups; gb += kPlanThreads / 16) {
        const int gi = gb + (tid >> 4);
        int64_t kmax = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = gi * kWgTok + (tid & 15) * 4 + j;
            if (gi < groups && t < T) {
                const int64_t kv = token_kv_len[t];
                if (token_seq[t] >= 0 && kv > kmax) kmax = kv;
            }
        }
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const int64_t o = __shfl_xor(kmax, d, 64);
            kmax = o > kmax ? o : kmax;
        }
        if (gi < groups && (tid & 15) == 0) {
            kmax = min(kmax, max_keys);
            const int c = static_cast<int>(min<int64_t>((kmax + kSub - 1) / kSub, kCostBuckets - 1));
            cost[gi] = c;
            atomicAdd(&hist[c], 1);
        }
    }
    __syncthreads();
    // exclusive scan in descending cost: start[c] = number of groups with cost > c
    const int rb = kCostBuckets - 1 - tid;           // bucket of this thread, reversed
    int v = tid < kCostBuckets ? hist[rb] : 0;
    scan[tid] = v;
    __syncthreads();
    for (int d = 1; d < kCostBuckets; d <<= 1) {
        const int add = tid >= d ? scan[tid - d] : 0;
        __syncthreads();
        scan[tid] += add;
        __syncthreads();
    }
    if (tid < kCostBuckets) hist[rb] = scan[tid] - v;   // exclusive
    __syncthreads();
    for (int gi = tid; gi < groups; gi += kPlanThreads) order[atomicAdd(&hist[cost[gi]], 1)] = gi;
}

size_t plan_bytes(int64_t num_tokens) {
    const int64_t groups = (num_tokens + kWgTok - 1) / kWgTok;
    return static_cast<size_t>(2 * groups) * sizeof(int);
}

}  // namespace
}  // namespace cvh

namespace cvh {
namespace {
int prefill_entry(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache, const float* k_scale,
                  const float* v_scale, const int64_t* block_tables, int64_t table_width, const int64_t* token_seq,
                  const int64_t* token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                  int block_size, int scale_mode, double scale, const int* order, cvh_stream_t stream) {
    if (num_tokens < 0 || n_heads <= 0 || n_kv_heads <= 0 || table_width < 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (table_width == 0) return CVH_ERR_INVALID_ARG;
    if (!out || !q || !k_cache || !v_cache || !k_scale || !v_scale || !block_tables || !token_seq || !token_kv_len)
        return CVH_ERR_INVALID_ARG;
    if (n_heads % n_kv_heads != 0) return CVH_ERR_INVALID_ARG;
    const int rep = n_heads / n_kv_heads;
    const int lg = ilog2_exact(block_size);
    if (head_dim != kHD || lg < 4 || lg > 12 || (rep != 1 && rep != 2)) return CVH_ERR_UNSUPPORTED;
    if (scale_mode != CVH_SCALE_PER_TOKEN_HEAD && scale_mode != CVH_SCALE_PER_TENSOR) return CVH_ERR_UNSUPPORTED;
    if (num_tokens > (int64_t{1} << 30)) return CVH_ERR_UNSUPPORTED;
    if (table_width > (int64_t{0x7fffffff} >> lg)) return CVH_ERR_UNSUPPORTED;    // contexts < 2^31 keys
    if ((num_tokens + kWgTok - 1) / kWgTok * n_kv_heads > 0x7fffffff) return CVH_ERR_UNSUPPORTED;   // 1-D grid
    auto s = reinterpret_cast<hipStream_t>(stream);
    const float sl2 = static_cast<float>(scale) * kLog2eP;
    auto* o = static_cast<uint16_t*>(out);
    auto* qq = static_cast<const uint16_t*>(q);
    const int T = static_cast<int>(num_tokens);
#define CVH_PF(R, SM)                                                                                             \
    launch_rep<R, SM>(o, qq, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq, token_kv_len, \
                      T, n_heads, n_kv_heads, lg, sl2, order, s)
    if (rep == 1)
        return scale_mode == CVH_SCALE_PER_TOKEN_HEAD ? CVH_PF(1, CVH_SCALE_PER_TOKEN_HEAD)
                                                      : CVH_PF(1, CVH_SCALE_PER_TENSOR);
    return scale_mode == CVH_SCALE_PER_TOKEN_HEAD ? CVH_PF(2, CVH_SCALE_PER_TOKEN_HEAD) : CVH_PF(2, CVH_SCALE_PER_TENSOR);
#undef CVH_PF
}
}  // namespace
}  // namespace cvh

extern "C" int cvh_paged_attention_fp8_prefill(void* out, const void* q, const uint8_t* k_cache,
                                               const uint8_t* v_cache, const float* k_scale, const float* v_scale,
                                               const int64_t* block_tables, int64_t table_width,
                                               const int64_t* token_seq, const int64_t* token_kv_len,
                                               int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                               int block_size, int scale_mode, double scale, cvh_stream_t stream) {
    return cvh::prefill_entry(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq,
                              token_kv_len, num_tokens, n_heads, n_kv_heads, head_dim, block_size, scale_mode, scale,
                              nullptr, stream);
}

extern "C" size_t cvh_paged_attention_prefill_workspace_bytes(int64_t num_tokens) {
    return num_tokens <= 0 ? 0 : cvh::plan_bytes(num_tokens);
}

extern "C" int cvh_paged_attention_prefill_plan(const int64_t* token_seq, const int64_t* token_kv_len,
                                                int64_t num_tokens, int64_t table_width, int block_size,
                                                void* workspace, size_t workspace_bytes, cvh_stream_t stream) {
    using namespace cvh;
    if (num_tokens < 0 || table_width < 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!token_seq || !token_kv_len || !workspace) return CVH_ERR_INVALID_ARG;
    if (num_tokens > (int64_t{1} << 30)) return CVH_ERR_UNSUPPORTED;
    const int lg = ilog2_exact(block_size);
    if (lg < 4 || lg > 12) return CVH_ERR_UNSUPPORTED;
    if (workspace_bytes < plan_bytes(num_tokens)) return CVH_ERR_WORKSPACE;
    const int64_t groups = (num_tokens + kWgTok - 1) / kWgTok;
    int* cost = static_cast<int*>(workspace);
    prefill_plan_kernel<<<1, kPlanThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            token_seq, token_kv_len, static_cast<int>(num_tokens), table_width << lg, cost, cost + groups);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

extern "C" int cvh_paged_attention_fp8_prefill_planned(void* out, const void* q, const uint8_t* k_cache,
                                                       const uint8_t* v_cache, const float* k_scale,
                                                       const float* v_scale, const int64_t* block_tables,
                                                       int64_t table_width, const int64_t* token_seq,
                                                       const int64_t* token_kv_len, int64_t num_tokens, int n_heads,
                                                       int n_kv_heads, int head_dim, int block_size, int scale_mode,
                                                       double scale, const void* workspace, size_t workspace_bytes,
                                                       cvh_stream_t stream) {
    using namespace cvh;
    if (num_tokens > 0 && (!workspace || workspace_bytes < plan_bytes(num_tokens))) return CVH_ERR_WORKSPACE;
    const int* order = num_tokens > 0 ? static_cast<const int*>(workspace) + (num_tokens + kWgTok - 1) / kWgTok
                                      : nullptr;
    return prefill_entry(out, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_width, token_seq,
                         token_kv_len, num_tokens, n_heads, n_kv_heads, head_dim, block_size, scale_mode, scale, order,
                         stream);
}
