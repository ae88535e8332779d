// FP8-e4m3 paged attention for multi-token query rows (chunked prefill / prompt continuation)
// on gfx950 matrix cores.
//
// Reference semantics: kernels/paged_attention.cu:89-359 with T > S — every query token t attends
// causally to keys [0, token_kv_len[t]) of sequence token_seq[t] through its block table, GQA
// query heads share the kv head, K/V dequantised with per-(token, kv head) (or per-tensor)
// scales, softmax in fp32. The decode kernel walks one query token per row; here 16 consecutive
// query tokens of a sequence share every K/V tile, so the score and PV products are real dense
// contractions and run on MFMA (v_mfma_f32_16x16x32_bf16):
//
//   S^T[key][row] = K . Q^T   A = K   (16 keys x 32 d, e4m3 -> bf16 exact),  B = Q^T (bf16)
//   O^T[d][row]  += V^T . P^T A = V^T (16 d x 32 keys, bf16 via LDS),        B = P^T (bf16, v scale folded)
//
// Both products put one query row per lane column (lane % 16), so the row's softmax state, its
// causal mask and its output accumulators live in the same lanes with no cross-lane shuffles
// except the 4-way max/sum over lane groups. The contraction index order inside an MFMA is
// free as long as A and B agree: lane group g = lane / 16 supplies d in
// {c*64 + g*16 + h*8 + 0..7} for step s = 2c + h (so each lane reads 16 contiguous K bytes per
// chunk), and keys {g*4 + 0..3, 16 + g*4 + 0..3} for the PV step (the keys its S^T output holds).
//
// Work: a wave = (16 consecutive query tokens, one kv head); a workgroup = WPG waves on WPG kv
// heads of the same tokens, so the whole 1 KB slot row of a key is read by one workgroup. Tokens
// of different sequences inside one 16-token tile are processed as separate runs (rows outside
// the run are masked), so any ragged batch is valid input; tiles rarely straddle sequences.
// V tiles are transposed through a per-wave LDS region (32 keys x 128 d bf16): each lane loads
// a 4 key x 4 d byte block with 4 dword loads, transposes it with v_perm_b32, converts to bf16 and
// stores 4 keys of one d with ds_write_b64.
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
constexpr int kTile = 32;          // keys per tile
// LDS row strides chosen against bank conflicts (64 banks of 4 bytes):
//  * V^T rows are 17 dwords (32 keys + 2 pad bf16): the writers (lane c -> row 4c + e) land on
//    banks 4*17*c mod 64, 16 distinct 2-dword slots per 16 lanes; accessed as dword pairs
//    (ds_write2/ds_read2_b32), since odd rows are only 4-byte aligned;
//  * q rows are 136 bf16 (272 bytes): the 16 rows read by one 16-byte load land 4 banks apart.
constexpr int kVtStride = 34;      // bf16 per LDS row of V^T
constexpr int kQStride = kHD + 8;  // bf16 per LDS row of q
constexpr float kLog2eP = 1.4426950408889634f;
constexpr float kNegHuge = -1e30f;
constexpr int kSplits = 4;         // waves per workgroup, each walking every 4th key tile

template <bool HI> __device__ __forceinline__ uint32_t pk_bf16(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

// 8 e4m3 codes (two dwords) -> 8 bf16 (exact for finite codes)
__device__ __forceinline__ bf16x8_t fp8x8_to_bf16(uint32_t a, uint32_t b) {
    const uint32_t r[4] = {pk_bf16<false>(a), pk_bf16<true>(a), pk_bf16<false>(b), pk_bf16<true>(b)};
    return __builtin_bit_cast(bf16x8_t, r);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_p));
}

__device__ __forceinline__ float max_groups(float v) {   // max over the 4 lane groups (lanes l, l^16, l^32, l^48)
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float sum_groups(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// K/V/scales of one 32-key tile as loaded (raw e4m3 words and f32 scales), so the next tile's
// loads can be in flight while the current tile is computed.
struct TileRaw {
    uint4 k[2][2];        // [key block kb][chunk c]: 16 K bytes of key kb*16 + i16, d = c*64 + g*16
    uint32_t v[4][4];     // [it][e]: 4 V bytes (d = 4*(lane%32) + 0..3) of key it*8 + (lane/32)*4 + e
    float ks[2][4], vs[2][4];   // scales of keys kb*16 + g*4 + r
};

template <int REP, int SCALE_MODE, int NS>
__global__ __launch_bounds__(64 * NS, 2) void paged_prefill_kernel(
        uint16_t* __restrict__ out, const uint16_t* __restrict__ q, const uint8_t* __restrict__ kc,
        const uint8_t* __restrict__ vc, const float* __restrict__ ksc, const float* __restrict__ vsc,
        const int64_t* __restrict__ tables, int64_t W, const int64_t* __restrict__ token_seq,
        const int64_t* __restrict__ token_kv_len, int T, int H, int KV, int lg_bs, float scale_log2) {
    // LDS: per-wave V^T staging during the key loop; reused for the cross-wave combine afterwards
    constexpr int kVtBytes = kHD * kVtStride * 2;
    constexpr int kPartBytes = NS * 8 * 64 * 16;                 // one rb's O^T partials of all waves
    constexpr int kLoopBytes = NS * kVtBytes;
    __shared__ __align__(16) char lds[kLoopBytes > kPartBytes ? kLoopBytes : kPartBytes];
    __shared__ __align__(16) uint16_t q_lds[REP][kQTok][kQStride];    // the tile's q rows, shared by the waves
    __shared__ float ml_lds[NS][REP][2][kQTok];                  // per wave: running max and sum per row

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // key split of this wave
    uint16_t* vt = reinterpret_cast<uint16_t*>(lds + w * kVtBytes);
    const int kvh = blockIdx.y;
    const int t0 = blockIdx.x * kQTok;
    const int g = lane >> 4, i16 = lane & 15;
    const int BS = 1 << lg_bs, bs_mask = BS - 1;
    const int64_t row_bytes = static_cast<int64_t>(KV) * kHD;      // one slot row, all kv heads

    // this lane's query row (token t0 + i16; heads kvh*REP + rb)
    const int tq = t0 + i16;
    int64_t seq = -1, kvl = 0;
    if (tq < T) {
        seq = token_seq[tq];
        kvl = token_kv_len[tq];
        if (seq < 0 || kvl < 0) kvl = 0;
        if (kvl > (W << lg_bs)) kvl = W << lg_bs;        // contexts end at the table's last block
    }

    f32x4_t o[REP][8];
    float m[REP], lsum[REP];
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        m[rb] = kNegHuge;
        lsum[rb] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[rb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    const float ks_tensor = SCALE_MODE == CVH_SCALE_PER_TENSOR ? ksc[0] : 0.f;
    const float vs_tensor = SCALE_MODE == CVH_SCALE_PER_TENSOR ? vsc[0] : 0.f;

    // runs of equal sequence among the 16 tokens (lanes 0..15 carry the rows)
    bool q_staged = false;
    uint64_t todo = __builtin_amdgcn_ballot_w64(lane < kQTok && kvl > 0);
    while (todo) {
        const int leader = __builtin_ctzll(todo);
        const int64_t rseq =
                static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(seq), leader))) |
                (static_cast<int64_t>(__builtin_amdgcn_readlane(static_cast<int>(seq >> 32), leader)) << 32);
        const bool in_run = seq == rseq && kvl > 0;
        todo &= ~__builtin_amdgcn_ballot_w64(lane < kQTok && in_run);
        int kmax_l = in_run ? static_cast<int>(kvl) : 0;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) kmax_l = max(kmax_l, __shfl_xor(kmax_l, d, 64));
        const int kmax = __builtin_amdgcn_readfirstlane(kmax_l);
        const int64_t* trow = tables + rseq * W;
        const int row_kvl = in_run ? static_cast<int>(kvl) : 0;

        // load one tile's raw K/V/scales (keys >= kmax and negative table entries read as zeros;
        // a negative entry inside a context is invalid input)
        auto load_tile = [&](int kb0, TileRaw& r) {
            // the tile's keys are two runs of 16 consecutive slots (one block when BS >= 32), so
            // every address is a wave-uniform base plus a 32-bit lane offset
            const bool any = kb0 < kmax;
            const int64_t blk0 = any ? trow[kb0 >> lg_bs] : -1;
            const int64_t blk1 = BS < kTile ? (kb0 + 16 < kmax ? trow[(kb0 + 16) >> lg_bs] : -1) : blk0;
            const int64_t slot0 = (blk0 << lg_bs) + (kb0 & bs_mask);
            const int64_t slot1 = BS < kTile ? (blk1 << lg_bs) + ((kb0 + 16) & bs_mask) : slot0 + 16;
            const uint8_t* kb_ptr[2] = {kc + slot0 * row_bytes + kvh * kHD, kc + slot1 * row_bytes + kvh * kHD};
            const uint8_t* vb_ptr[2] = {vc + slot0 * row_bytes + kvh * kHD, vc + slot1 * row_bytes + kvh * kHD};
            const bool ok[2] = {blk0 >= 0, blk1 >= 0};
            const uint32_t rb32 = static_cast<uint32_t>(row_bytes);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                r.k[kb][0] = r.k[kb][1] = make_uint4(0, 0, 0, 0);
                if (ok[kb] && kb0 + kb * 16 + i16 < kmax) {
                    const uint8_t* kr = kb_ptr[kb] + (static_cast<uint32_t>(i16) * rb32 + static_cast<uint32_t>(g * 16));
                    r.k[kb][0] = *reinterpret_cast<const uint4*>(kr);
                    r.k[kb][1] = *reinterpret_cast<const uint4*>(kr + 64);
                }
            }
            const int c = lane & 31, kg = lane >> 5;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int h = it >> 1;                           // keys it*8 + ... are in half h
                const uint8_t* vr = vb_ptr[h] + (static_cast<uint32_t>((it & 1) * 8 + kg * 4) * rb32 +
                                                 static_cast<uint32_t>(c * 4));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int key = it * 8 + kg * 4 + e;
                    r.v[it][e] = (ok[h] && kb0 + key < kmax) ? *reinterpret_cast<const uint32_t*>(vr + e * rb32) : 0u;
                }
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int key = kb * 16 + g * 4;
                if constexpr (SCALE_MODE == CVH_SCALE_PER_TOKEN_HEAD) {
                    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
                    if (ok[kb] && kb0 + key < kmax) {
                        const int64_t blk = kb ? blk1 : blk0;
                        const int64_t sb = ((blk * KV + kvh) << lg_bs) + ((kb0 + kb * 16) & bs_mask);
                        a = *reinterpret_cast<const float4*>(ksc + sb + g * 4);
                        b = *reinterpret_cast<const float4*>(vsc + sb + g * 4);
                    }
                    r.ks[kb][0] = a.x; r.ks[kb][1] = a.y; r.ks[kb][2] = a.z; r.ks[kb][3] = a.w;
                    r.vs[kb][0] = b.x; r.vs[kb][1] = b.y; r.vs[kb][2] = b.z; r.vs[kb][3] = b.w;
                } else {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const bool lv = ok[kb] && kb0 + key + rr < kmax;
                        r.ks[kb][rr] = lv ? ks_tensor : 0.f;
                        r.vs[kb][rr] = lv ? vs_tensor : 0.f;
                    }
                }
            }
        };

        TileRaw cur, nxt;
        int kb0 = w * kTile;
        load_tile(kb0, cur);
        if (!q_staged) {
            // q of the 16 tokens x REP heads into LDS (16 bytes per thread per pass), issued after
            // the first tile's loads so the two round trips overlap. Runs are the same for every
            // wave of the workgroup, so this barrier is reached uniformly.
            for (int i = threadIdx.x; i < REP * kQTok * (kHD / 8); i += 64 * NS) {
                const int c8 = i % (kHD / 8), row = i / (kHD / 8);
                const int rb = row / kQTok, tk = row % kQTok;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (t0 + tk < T)
                    v = *reinterpret_cast<const uint4*>(q + (static_cast<int64_t>(t0 + tk) * H + kvh * REP + rb) * kHD +
                                                        c8 * 8);
                *reinterpret_cast<uint4*>(&q_lds[rb][tk][c8 * 8]) = v;
            }
            __syncthreads();
            q_staged = true;
        }
        for (; kb0 < kmax; kb0 += NS * kTile) {

            // ---- S^T = K . Q^T (K e4m3 -> bf16 per step; Q from LDS)
            f32x4_t s[2][REP];
#pragma unroll
            for (int rb = 0; rb < REP; ++rb) {
                bf16x8_t qb[4];
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    qb[st] = __builtin_bit_cast(
                            bf16x8_t, *reinterpret_cast<const uint4*>(&q_lds[rb][i16][(st >> 1) * 64 + g * 16 + (st & 1) * 8]));
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        const uint4 kw = cur.k[kb][st >> 1];
                        const bf16x8_t ka = (st & 1) ? fp8x8_to_bf16(kw.z, kw.w) : fp8x8_to_bf16(kw.x, kw.y);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[st], acc, 0, 0, 0);
                    }
                    s[kb][rb] = acc;
                }
            }

            // ---- V^T into this wave's LDS region (the previous tile's reads were issued before
            //      these writes; a wave's LDS operations complete in order)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            {
                const int c = lane & 31, kg = lane >> 5;
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const uint32_t w0 = cur.v[it][0], w1 = cur.v[it][1], w2 = cur.v[it][2], w3 = cur.v[it][3];
                    const uint32_t a = __builtin_amdgcn_perm(w1, w0, 0x05010400u);   // w0b0 w1b0 w0b1 w1b1
                    const uint32_t b = __builtin_amdgcn_perm(w1, w0, 0x07030602u);   // w0b2 w1b2 w0b3 w1b3
                    const uint32_t cc = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
                    const uint32_t dd = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
                    const uint32_t tr[4] = {__builtin_amdgcn_perm(cc, a, 0x05040100u),
                                            __builtin_amdgcn_perm(cc, a, 0x07060302u),
                                            __builtin_amdgcn_perm(dd, b, 0x05040100u),
                                            __builtin_amdgcn_perm(dd, b, 0x07060302u)};
                    const int key = it * 8 + kg * 4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        uint32_t* dst = reinterpret_cast<uint32_t*>(vt + (c * 4 + e) * kVtStride + key);
                        dst[0] = pk_bf16<false>(tr[e]);
                        dst[1] = pk_bf16<true>(tr[e]);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // this tile's K/V words are consumed: the next tile's loads go out now and stay in
            // flight through the softmax and PV products
            load_tile(kb0 + NS * kTile, nxt);

            // ---- scores, mask, online softmax (one query row per lane column)
#pragma unroll
            for (int rb = 0; rb < REP; ++rb) {
                float mt = kNegHuge;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = kb0 + kb * 16 + g * 4 + r;
                        float sv = s[kb][rb][r] * (cur.ks[kb][r] * scale_log2);
                        sv = key < row_kvl ? sv : -INFINITY;
                        s[kb][rb][r] = sv;
                        mt = fmaxf(mt, sv);
                    }
                mt = max_groups(mt);
                const float mn = fmaxf(m[rb], mt);
                const float alpha = __builtin_amdgcn_exp2f(m[rb] - mn);
                m[rb] = mn;
                float ps = 0.f;
                uint32_t pp[4];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; r += 2) {
                        const float p0 = __builtin_amdgcn_exp2f(s[kb][rb][r] - mn);
                        const float p1 = __builtin_amdgcn_exp2f(s[kb][rb][r + 1] - mn);
                        ps += p0 + p1;
                        pp[kb * 2 + r / 2] = pack_bf16x2(p0 * cur.vs[kb][r], p1 * cur.vs[kb][r + 1]);
                    }
                lsum[rb] = lsum[rb] * alpha + ps;
                if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {     // wave-uniform: the max moved
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[rb][j] *= alpha;
                }
                const bf16x8_t pop = __builtin_bit_cast(bf16x8_t, pp);
                // ---- O^T += V^T . P^T over the 8 d blocks
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint16_t* vr = vt + (j * 16 + i16) * kVtStride + g * 4;
                    const uint32_t* v32 = reinterpret_cast<const uint32_t*>(vr);
                    const uint32_t va[4] = {v32[0], v32[1], v32[8], v32[9]};
                    o[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, va), pop,
                                                                       o[rb][j], 0, 0, 0);
                }
            }
            cur = nxt;
        }
    }

    // ---- combine the NS key splits: row max and sum per wave, then O^T partials one rb at a time;
    //      wave w finishes d blocks [w*8/NS, (w+1)*8/NS) of every row
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        const float l = sum_groups(lsum[rb]);
        if (g == 0) {
            ml_lds[w][rb][0][i16] = m[rb];
            ml_lds[w][rb][1][i16] = l;
        }
    }
    __syncthreads();                         // every wave is past its key loop: V^T area is free
    float fs[REP][NS], inv[REP];
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        float mx = kNegHuge;
#pragma unroll
        for (int x = 0; x < NS; ++x) mx = fmaxf(mx, ml_lds[x][rb][0][i16]);
        float l = 0.f;
#pragma unroll
        for (int x = 0; x < NS; ++x) {
            fs[rb][x] = __builtin_amdgcn_exp2f(ml_lds[x][rb][0][i16] - mx);
            l += fs[rb][x] * ml_lds[x][rb][1][i16];
        }
        inv[rb] = l > 0.f ? 1.0f / l : 0.f;
    }
    f32x4_t* part = reinterpret_cast<f32x4_t*>(lds);     // [NS][8][64] per rb
    constexpr int kJPer = 8 / NS;
#pragma unroll
    for (int rb = 0; rb < REP; ++rb) {
        if (rb) __syncthreads();             // the previous rb's partials have been read
#pragma unroll
        for (int j = 0; j < 8; ++j) part[(w * 8 + j) * 64 + lane] = o[rb][j];
        __syncthreads();
        if (tq < T) {
            uint16_t* orow = out + (static_cast<int64_t>(tq) * H + kvh * REP + rb) * kHD;
#pragma unroll
            for (int jj = 0; jj < kJPer; ++jj) {
                const int j = w * kJPer + jj;
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int x = 0; x < NS; ++x) acc += part[(x * 8 + j) * 64 + lane] * fs[rb][x];
                acc *= inv[rb];
                const uint2 v = make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]));
                *reinterpret_cast<uint2*>(orow + j * 16 + g * 4) = v;
            }
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
               int H, int KV, int lg, float sl2, hipStream_t s) {
    const unsigned gx = static_cast<unsigned>((T + kQTok - 1) / kQTok);
    paged_prefill_kernel<REP, SM, kSplits><<<dim3(gx, KV), 64 * kSplits, 0, s>>>(out, q, kc, vc, ks, vs, tables, W,
                                                                                tseq, tkvl, T, H, KV, lg, sl2);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_paged_attention_fp8_prefill(void* out, const void* q, const uint8_t* k_cache,
                                               const uint8_t* v_cache, const float* k_scale, const float* v_scale,
                                               const int64_t* block_tables, int64_t table_width,
                                               const int64_t* token_seq, const int64_t* token_kv_len,
                                               int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                               int block_size, int scale_mode, double scale, cvh_stream_t stream) {
    using namespace cvh;
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
    auto s = reinterpret_cast<hipStream_t>(stream);
    const float sl2 = static_cast<float>(scale) * kLog2eP;
    auto* o = static_cast<uint16_t*>(out);
    auto* qq = static_cast<const uint16_t*>(q);
    const int T = static_cast<int>(num_tokens);
    if (rep == 1) {
        if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
            return launch_rep<1, CVH_SCALE_PER_TOKEN_HEAD>(o, qq, k_cache, v_cache, k_scale, v_scale, block_tables,
                                                           table_width, token_seq, token_kv_len, T, n_heads,
                                                           n_kv_heads, lg, sl2, s);
        return launch_rep<1, CVH_SCALE_PER_TENSOR>(o, qq, k_cache, v_cache, k_scale, v_scale, block_tables,
                                                   table_width, token_seq, token_kv_len, T, n_heads, n_kv_heads, lg,
                                                   sl2, s);
    }
    if (scale_mode == CVH_SCALE_PER_TOKEN_HEAD)
        return launch_rep<2, CVH_SCALE_PER_TOKEN_HEAD>(o, qq, k_cache, v_cache, k_scale, v_scale, block_tables,
                                                       table_width, token_seq, token_kv_len, T, n_heads, n_kv_heads,
                                                       lg, sl2, s);
    return launch_rep<2, CVH_SCALE_PER_TENSOR>(o, qq, k_cache, v_cache, k_scale, v_scale, block_tables, table_width,
                                               token_seq, token_kv_len, T, n_heads, n_kv_heads, lg, sl2, s);
}
