// bf16 GEMM for the decode-step projections on gfx950 matrix cores: Y[M][N] = X[M][K] . W[N][K]^T
// (torch's linear layout: both operands K-contiguous), fp32 accumulation, bf16 output rounded to
// nearest even. Replaces the at::linear calls of the reference's layer loop
// (model/model_architecture.cpp:155,178,182,185) and its lm_head (:224) for M <= a few hundred
// rows, where library GEMMs run latency-bound (one HBM round trip per K step of a few large
// tiles). Here every byte of W is read from HBM exactly once per call, by one wave, with all of
// that wave's K range in flight in a two-chunk register pipeline, and reused from registers for
// all M rows of the workgroup.
//
// MFMA v_mfma_f32_16x16x32_bf16 with A = W (16 output columns n, lane % 16 = n), B = X (16 rows m,
// lane % 16 = m); the product D[n][m] leaves lane (i16 = lane % 16, g = lane / 16) holding
// Y[m = i16][n = 4g .. 4g+3] — four consecutive outputs of one row, one 8-byte store. The
// standard operand layout applies: at MFMA step s of a 128-wide K chunk, lane group g supplies
// k in [32s + 8g, 32s + 8g + 8), so one 16-byte load instruction of a wave reads 64 contiguous
// bytes of each of 16 rows.
//
// Work decomposition (template <MF, NWN, XLDS>): a workgroup is 4 waves; NWN of them split the
// 16*NWN output columns of the workgroup's column tile, the other factor NWK = 4 / NWN splits K;
// each wave computes 16*MF rows x 16 columns over its K range. W always goes HBM -> registers
// (each byte read once, by one wave). X, which every column tile re-reads, either goes straight to
// registers (XLDS = 0) or, when NWN waves share it, through a double-buffered LDS chunk loaded
// once per workgroup (XLDS = 1). K-split partial sums are added through LDS in a fixed order
// (wave wk = 0, 1, ...), so results are deterministic for a configuration.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cvh_device.h"

namespace cvh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 128;        // K elements per pipeline chunk (4 MFMA steps of 32)
constexpr int kXRow = kChunk + 8;  // bf16 per LDS row of an X chunk (272 B: 16 rows of a read hit distinct banks)

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}


// W operand of one chunk for one wave: lane (i16, g) holds k = 32s + 8g .. +8 of row i16 at step s,
// so each load instruction reads 64 contiguous bytes of each of the wave's 16 rows.
struct WChunk {
    u32x4_t v[4];
};
__device__ __forceinline__ void load_w(WChunk& c, const uint16_t* wp, int k) {
#pragma unroll
    for (int s = 0; s < 4; ++s) c.v[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + k + 32 * s));
}

// X operand fragments of one chunk read straight from global memory (same k layout as W).
template <int MF>
struct XChunk {
    u32x4_t v[MF][4];
};
template <int MF>
__device__ __forceinline__ void load_x(XChunk<MF>& c, const uint16_t* const* xp, int k) {
#pragma unroll
    for (int f = 0; f < MF; ++f)
#pragma unroll
        for (int s = 0; s < 4; ++s) c.v[f][s] = *reinterpret_cast<const u32x4_t*>(xp[f] + k + 32 * s);
}

template <int MF>
__device__ __forceinline__ void mma_regs(f32x4_t* acc, const WChunk& w, const XChunk<MF>& x) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, w.v[s]);
#pragma unroll
        for (int f = 0; f < MF; ++f)
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, x.v[f][s]), acc[f], 0, 0, 0);
    }
}

// X fragments from an LDS chunk tile [rows][kXRow] (this wave's K part).
template <int MF>
__device__ __forceinline__ void mma_lds(f32x4_t* acc, const WChunk& w, const uint16_t* xs, int i16, int g) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, w.v[s]);
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xs + (f * 16 + i16) * kXRow + 32 * s + 8 * g);
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, xv), acc[f], 0, 0, 0);
        }
    }
}

// Cooperative X chunk of the workgroup: NWK parts (one per K split) x BM rows x 128 k, 16 bytes
// per thread per instruction; rows past M read row M-1 (never stored).
template <int MF, int NWK>
struct XStage {
    static constexpr int kPieces = NWK * MF * 16 * (kChunk / 8);   // 16-byte pieces per chunk
    static constexpr int kPer = kPieces / 256;
    u32x4_t v[kPer];
};
template <int MF, int NWK>
__device__ __forceinline__ void stage_load(XStage<MF, NWK>& st, const uint16_t* x, int M, int K, int m0, int kper,
                                           int kc) {
#pragma unroll
    for (int i = 0; i < XStage<MF, NWK>::kPer; ++i) {
        const int p = i * 256 + threadIdx.x;
        const int piece = p & 15, row = (p >> 4) % (MF * 16), part = (p >> 4) / (MF * 16);
        const int m = min(m0 + row, M - 1);
        st.v[i] = *reinterpret_cast<const u32x4_t*>(x + static_cast<size_t>(m) * K + part * kper + kc + piece * 8);
    }
}
template <int MF, int NWK>
__device__ __forceinline__ void stage_store(const XStage<MF, NWK>& st, uint16_t* xs) {
#pragma unroll
    for (int i = 0; i < XStage<MF, NWK>::kPer; ++i) {
        const int p = i * 256 + threadIdx.x;
        const int piece = p & 15, rr = p >> 4;     // rr = part * BM + row
        *reinterpret_cast<u32x4_t*>(xs + rr * kXRow + piece * 8) = st.v[i];
    }
}

template <int MF, int NWN, bool XLDS>
__global__ __launch_bounds__(256) void gemm_nt_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, int M, int N, int K) {
    constexpr int NWK = 4 / NWN;
    constexpr int BM = 16 * MF;
    constexpr int kRed = NWK > 1 ? 4 * MF * 64 : 1;
    constexpr int kXs = XLDS ? 2 * NWK * BM * kXRow : 1;
    __shared__ f32x4_t red[kRed];
    __shared__ __attribute__((aligned(16))) uint16_t xs[kXs];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int wn = wave % NWN, wk = wave / NWN;
    const int n0 = (blockIdx.x * NWN + wn) * 16;
    const int m0 = blockIdx.y * BM;
    const int kper = K / NWK;
    const int nc = kper / kChunk;

    const uint16_t* wp = w + static_cast<size_t>(n0 + i16) * K + wk * kper + 8 * g;
    f32x4_t acc[MF];
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    if constexpr (XLDS) {
        // X chunk c sits in LDS buffer c & 1 while chunk c + 1 is in registers; W chunks c + 1 and
        // c + 2 are in flight while chunk c is multiplied
        XStage<MF, NWK> st;
        WChunk wa, wb;
        stage_load<MF, NWK>(st, x, M, K, m0, kper, 0);
        load_w(wa, wp, 0);
        stage_store<MF, NWK>(st, xs);
        if (nc > 1) {
            stage_load<MF, NWK>(st, x, M, K, m0, kper, kChunk);
            load_w(wb, wp, kChunk);
        }
        __syncthreads();
        for (int c = 0; c < nc; c += 2) {
            mma_lds<MF>(acc, wa, xs + (wk * BM) * kXRow, i16, g);
            if (c + 1 < nc) stage_store<MF, NWK>(st, xs + NWK * BM * kXRow);
            if (c + 2 < nc) {
                stage_load<MF, NWK>(st, x, M, K, m0, kper, (c + 2) * kChunk);
                load_w(wa, wp, (c + 2) * kChunk);
            }
            __syncthreads();
            if (c + 1 >= nc) break;
            mma_lds<MF>(acc, wb, xs + (NWK * BM + wk * BM) * kXRow, i16, g);
            if (c + 2 < nc) stage_store<MF, NWK>(st, xs);
            if (c + 3 < nc) {
                stage_load<MF, NWK>(st, x, M, K, m0, kper, (c + 3) * kChunk);
                load_w(wb, wp, (c + 3) * kChunk);
            }
            __syncthreads();
        }
    } else {
        const uint16_t* xp[MF];
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int m = min(m0 + f * 16 + i16, M - 1);    // rows past M load row M-1; never stored
            xp[f] = x + static_cast<size_t>(m) * K + wk * kper + 8 * g;
        }
        WChunk wa, wb;
        XChunk<MF> xa, xb;
        load_w(wa, wp, 0);
        load_x<MF>(xa, xp, 0);
        int c = 0;
        for (; c + 2 <= nc; c += 2) {
            load_w(wb, wp, (c + 1) * kChunk);
            load_x<MF>(xb, xp, (c + 1) * kChunk);
            mma_regs<MF>(acc, wa, xa);
            if (c + 2 < nc) {
                load_w(wa, wp, (c + 2) * kChunk);
                load_x<MF>(xa, xp, (c + 2) * kChunk);
            }
            mma_regs<MF>(acc, wb, xb);
        }
        if (c < nc) mma_regs<MF>(acc, wa, xa);
    }

    if constexpr (NWK > 1) {
#pragma unroll
        for (int f = 0; f < MF; ++f) red[(wave * MF + f) * 64 + lane] = acc[f];
        __syncthreads();
        // wave (wn, wk) finishes the row fragments f with f % NWK == wk, summing wk' = 0.. in order
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            if (f % NWK != wk) continue;
            f32x4_t s = red[(wn * MF + f) * 64 + lane];
#pragma unroll
            for (int j = 1; j < NWK; ++j) s += red[((j * NWN + wn) * MF + f) * 64 + lane];
            acc[f] = s;
        }
    }
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        if (NWK > 1 && f % NWK != wk) continue;
        const int m = m0 + f * 16 + i16;
        if (m < M) {
            uint2 v;
            v.x = pack_bf16x2(acc[f][0], acc[f][1]);
            v.y = pack_bf16x2(acc[f][2], acc[f][3]);
            *reinterpret_cast<uint2*>(y + static_cast<size_t>(m) * N + n0 + 4 * g) = v;
        }
    }
}

// ---- one-shot variant: every load of the workgroup in flight at once ------------------------
// For the decode shapes a workgroup's whole problem is small (tens of KB of W, a few KB to 128 KB
// of X), so a K loop that waits one memory round trip per chunk is latency-bound. Here a
// workgroup issues its X tile (BM rows x all K) straight into LDS with global_load_lds_dwordx4 and
// each wave issues all NC chunks of its W rows into registers, then waits once and multiplies.
// X in LDS: [row][chunk of 128 k][16-byte slot], piece p of a row chunk stored at slot
// p ^ (row & 15) so the 16 rows one MFMA fragment read hits 16 distinct 4-bank groups.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glob_void_t;

template <int MF, int NWN, int NC>
__global__ __launch_bounds__(256) void gemm_oneshot_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w, int M, int N, int K) {
    constexpr int NWK = 4 / NWN;
    constexpr int BM = 16 * MF;
    constexpr int NCH = NWK * NC;                 // 128-k chunks per row (K / 128)
    constexpr int kSlots = BM * NCH * 16;         // 16-byte slots of the X tile
    static_assert(kSlots % 256 == 0, "X tile must be whole rounds of 256 slots");
    __shared__ __attribute__((aligned(16))) uint16_t xs[kSlots * 8];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int wn = wave % NWN, wk = wave / NWN;
    const int n0 = (blockIdx.x * NWN + wn) * 16;
    const int m0 = blockIdx.y * BM;

    // X tile -> LDS: wave instruction j writes the 64 consecutive slots (jj*4 + wave)*64 .. +64.
    // Every column tile reads the same X rows: the order is rotated by the column tile so the
    // workgroups of an XCD do not all ask the same L2 channel for the same lines at once.
    constexpr int kRounds = kSlots / 256;
#pragma unroll
    for (int j = 0; j < kRounds; ++j) {
        const int jj = (j + static_cast<int>(blockIdx.x)) % kRounds;
        const int base = (jj * 4 + wave) * 64;
        const int slot = base + lane;
        const int rq = slot >> 4, r = rq / NCH, q = rq - r * NCH;
        const int p = (slot & 15) ^ (r & 15);
        const int m = min(m0 + r, M - 1);         // rows past M read row M-1 (never stored)
        __builtin_amdgcn_global_load_lds(
            (glob_void_t*)(x + static_cast<size_t>(m) * K + q * kChunk + p * 8), (lds_void_t*)(xs + base * 8), 16, 0,
            0);
    }
    asm volatile("" ::: "memory");
    // all of this wave's W: NC chunks x 4 steps, lane (i16, g) holds k = c*128 + 32s + 8g .. +8
    const uint16_t* wp = w + static_cast<size_t>(n0 + i16) * K + wk * (NC * kChunk) + 8 * g;
    u32x4_t wr[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int s = 0; s < 4; ++s)
            wr[c][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + c * kChunk + 32 * s));
    __builtin_amdgcn_sched_barrier(0);
    // X slots have landed once at most the W loads are outstanding; a bare barrier (no fence), so
    // the W loads stay in flight into the multiply
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NC * 4 > 63 ? 63 : NC * 4) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    f32x4_t acc[MF];
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // software pipeline over the NC*4 MFMA steps: X fragments of step t + 2 are read from LDS
    // while step t multiplies (one wave per SIMD: nothing else hides the LDS latency)
    constexpr int kSteps = NC * 4;
    constexpr int kAhead = 2;
    u32x4_t xf[kAhead + 1][MF];
    auto read_step = [&](int t, u32x4_t* dst) {
        const int q = wk * NC + (t >> 2), sl = (4 * (t & 3) + g) ^ i16;
#pragma unroll
        for (int f = 0; f < MF; ++f)
            dst[f] = *reinterpret_cast<const u32x4_t*>(xs + (((f * 16 + i16) * NCH + q) * 16 + sl) * 8);
    };
#pragma unroll
    for (int t = 0; t < kAhead; ++t) read_step(t, xf[t]);
#pragma unroll
    for (int t = 0; t < kSteps; ++t) {
        if (t + kAhead < kSteps) read_step(t + kAhead, xf[(t + kAhead) % (kAhead + 1)]);
        __builtin_amdgcn_sched_barrier(0);        // keep the reads ahead of this step's multiplies
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, wr[t >> 2][t & 3]);
#pragma unroll
        for (int f = 0; f < MF; ++f)
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, xf[t % (kAhead + 1)][f]),
                                                             acc[f], 0, 0, 0);
    }

    if constexpr (NWK > 1) {
        __syncthreads();                          // X tile no longer read: reuse it for the partials
        f32x4_t* red = reinterpret_cast<f32x4_t*>(xs);
#pragma unroll
        for (int f = 0; f < MF; ++f) red[(wave * MF + f) * 64 + lane] = acc[f];
        __syncthreads();
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            if (f % NWK != wk) continue;
            f32x4_t t = red[(wn * MF + f) * 64 + lane];
#pragma unroll
            for (int j = 1; j < NWK; ++j) t += red[((j * NWN + wn) * MF + f) * 64 + lane];
            acc[f] = t;
        }
    }
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        if (NWK > 1 && f % NWK != wk) continue;
        const int m = m0 + f * 16 + i16;
        if (m < M) {
            uint2 v;
            v.x = pack_bf16x2(acc[f][0], acc[f][1]);
            v.y = pack_bf16x2(acc[f][2], acc[f][3]);
            *reinterpret_cast<uint2*>(y + static_cast<size_t>(m) * N + n0 + 4 * g) = v;
        }
    }
}

// ---- tiled variant: X and W both through a ring of LDS stages -------------------------------
// Measured on MI355X: loads whose 64 lanes cover 1 KB of contiguous bytes deliver 19-26 TB/s from
// L2 and 7.6 TB/s from HBM, while the MFMA register layout (16 rows x 64 B per instruction) gets
// 8.5 and 6.0. Here both operands move global -> LDS with global_load_lds_dwordx4 in the
// contiguous pattern and MFMA fragments are read from LDS. A wave computes MF x NF fragments of
// 16 x 16; the workgroup is WM x WN waves, a BM x BN = (16*MF*WM) x (16*NF*WN) output tile, and
// walks K in 128-wide chunks through S LDS stages.
// LDS chunk layout per operand: [row][16 slots of 16 B], piece p of a row stored at slot
// p ^ (row & 15): one DMA instruction fills 4 whole rows (4 runs of 256 contiguous global bytes)
// and the 16 rows of a fragment read hit 16 distinct 4-bank groups.
// The DMA is issued from inline assembly on purpose: the compiler cannot tell which LDS stage a
// global_load_lds writes and would wait for all of them (vmcnt(0)) before any LDS read, which
// serialises the ring. The kernel therefore counts vmcnt itself; it issues no other vector-memory
// loads, so the compiler's own counter bookkeeping is unaffected. M0 (the LDS destination) is
// saved and restored inside the statement: the compiler does not honour M0 as a clobber.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(gptr), "s"(lds_addr)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// Stages: as many 128-k chunks in flight as the LDS (160 KB) holds, up to 8, within the 63
// outstanding vector-memory operations a wave can count.
constexpr int stages_for(int stage_bytes, int dma_per_stage) {
    int st = (160 * 1024) / stage_bytes;
    if (st > 8) st = 8;
    while (st > 2 && dma_per_stage * (st - 2) > 63) --st;
    return st;
}
// wait until at most `ahead` later stages (dma_per_stage operations each) are still in flight
template <int D, int A>
__device__ __forceinline__ void wait_stages(int ahead) {
    if constexpr (A == 0) {
        wait_vmcnt<0>();
    } else {
        if (ahead >= A) wait_vmcnt<D * A>();
        else wait_stages<D, A - 1>(ahead);
    }
}

// Epilogues of the tiled kernels.
enum { kEpiStore = 0, kEpiSwiglu = 1 };

// One 128-k chunk of a wave's MF x NF fragments from LDS chunk tiles (rows of 256 B, 16-byte
// pieces stored at slot p ^ (row & 15)): xs points at the wave's first X row, ws at its first W row.
template <int MF, int NF>
__device__ __forceinline__ void chunk_mma(f32x4_t (&acc)[MF][NF], const uint8_t* xs, const uint8_t* ws, int i16,
                                          int g) {
    constexpr int kRowBytes = kChunk * 2;
#pragma unroll
    for (int s = 0; s < kChunk / 32; ++s) {
        const int sl = ((4 * s + g) ^ i16) * 16;
        u32x4_t a[NF], b[MF];
#pragma unroll
        for (int e = 0; e < NF; ++e) a[e] = *reinterpret_cast<const u32x4_t*>(ws + (e * 16 + i16) * kRowBytes + sl);
#pragma unroll
        for (int f = 0; f < MF; ++f) b[f] = *reinterpret_cast<const u32x4_t*>(xs + (f * 16 + i16) * kRowBytes + sl);
#pragma unroll
        for (int f = 0; f < MF; ++f)
#pragma unroll
            for (int e = 0; e < NF; ++e)
                acc[f][e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[e]),
                                                                    __builtin_bit_cast(bf16x8_t, b[f]), acc[f][e], 0, 0,
                                                                    0);
    }
}

// Stores a wave's fragments: kEpiStore writes y [M][N] in bf16; kEpiSwiglu reads fragment pairs
// (e, e+1) as gate and up of the same outputs (W rows interleaved in blocks of 16) and writes
// act = y [M][N/2] with the SwiGLU kernel's arithmetic, the products rounded to bf16 first as the
// reference's gate_up tensor is.
template <int MF, int NF, int WN, int EPI>
__device__ __forceinline__ void tile_epilogue(const f32x4_t (&acc)[MF][NF], uint16_t* __restrict__ y, int M, int N,
                                              int m0, int n0, int wm, int wn, int i16, int g) {
    if constexpr (EPI == kEpiStore) {
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int m = m0 + (wm * MF + f) * 16 + i16;
            if (m >= M) continue;
#pragma unroll
            for (int e = 0; e < NF; ++e) {
                uint2 v;
                v.x = pack_bf16x2(acc[f][e][0], acc[f][e][1]);
                v.y = pack_bf16x2(acc[f][e][2], acc[f][e][3]);
                *reinterpret_cast<uint2*>(y + static_cast<size_t>(m) * N + n0 + (wn * NF + e) * 16 + 4 * g) = v;
            }
        }
    } else {
        // W rows interleaved in blocks of 16 (gate j..j+15, then up j..j+15): fragment pair
        // (e, e+1) of a lane holds gate and up of the same 4 outputs. y is act [M][N/2]; the
        // products are rounded to bf16 first, as the reference's gate_up tensor is.
        static_assert(NF % 2 == 0, "gate/up fragment pairs");
        const int I = N >> 1;
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int m = m0 + (wm * MF + f) * 16 + i16;
            if (m >= M) continue;
#pragma unroll
            for (int e = 0; e < NF; e += 2) {
                const int j = ((n0 + (wn * NF + e) * 16) >> 1) + 4 * g;
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    o[r] = silu_mul<CVH_DTYPE_BF16>(round_bf16(acc[f][e][r]), round_bf16(acc[f][e + 1][r]));
                uint2 v;
                v.x = pack_bf16x2(o[0], o[1]);
                v.y = pack_bf16x2(o[2], o[3]);
                *reinterpret_cast<uint2*>(y + static_cast<size_t>(m) * I + j) = v;
            }
        }
    }
}


// Shape constants of a tiled configuration.
template <int MF, int NF, int WM, int WN, int S>
struct Tiled {
    static_assert(WM * WN == 4, "four waves");
    static constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN;
    static constexpr int kRowBytes = kChunk * 2;                       // 256 B per row chunk
    static constexpr int kStageBytes = (BM + BN) * kRowBytes;
    static constexpr int kDma = (BM + BN) * 16 / 256;                  // 16-byte DMA slots per thread per stage
    static_assert((BM + BN) * 16 % 256 == 0, "whole DMA rounds");
    static constexpr int kStages = S > 0 ? S : stages_for(kStageBytes, kDma);   // S = 0: as deep as fits
    static_assert(kStages >= 2 && kDma * (kStages - 2) <= 63 && kStages * kStageBytes <= 160 * 1024, "stages");
    static constexpr int kLdsBytes = kStages * kStageBytes;
};

// The K loop of a tiled workgroup: the BM x BN output tile at (m0, n0) accumulated in acc (wave
// (wm, wn) holds MF x NF fragments). lds holds Tiled::kLdsBytes.
struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

// hook() runs once, after the first chunk has landed (inputs requested before the loop have
// arrived by then): an epilogue issues its dependent loads there so they land under the loop.
template <int MF, int NF, int WM, int WN, int S, typename Hook = NoHook>
__device__ __forceinline__ void tiled_mainloop(f32x4_t (&acc)[MF][NF], uint8_t* lds, const uint16_t* __restrict__ x,
                                               const uint16_t* __restrict__ w, int M, int K, int m0, int n0,
                                               Hook hook = Hook{}) {
    using C = Tiled<MF, NF, WM, WN, S>;
    constexpr int BM = C::BM, kRowBytes = C::kRowBytes, kStageBytes = C::kStageBytes, kDma = C::kDma;
    constexpr int kStages = C::kStages;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;
    const uint32_t lds0 = lds_addr(lds);

    // this thread's DMA sources: slot L = (j*4 + wave)*64 + lane of a stage; rows [0, BM) are X,
    // rows [BM, BM+BN) are W; only the K offset changes from chunk to chunk
    const uint16_t* src[kDma];
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
        const int L = (j * 4 + wave) * 64 + lane;
        const int r = L >> 4, p = (L & 15) ^ (r & 15);
        const uint16_t* row = r < BM ? x + static_cast<size_t>(min(m0 + r, M - 1)) * K
                                     : w + static_cast<size_t>(n0 + r - BM) * K;
        src[j] = row + p * 8;
    }
    auto issue = [&](int c, int stage) {
        const uint32_t base = lds0 + stage * kStageBytes;
#pragma unroll
        for (int j = 0; j < kDma; ++j)
            dma16(src[j] + c * kChunk, __builtin_amdgcn_readfirstlane(base + (j * 4 + wave) * 1024));
    };

#pragma unroll
    for (int f = 0; f < MF; ++f)
#pragma unroll
        for (int e = 0; e < NF; ++e) acc[f][e] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int nc = K / kChunk;
#pragma unroll
    for (int i = 0; i < kStages - 1; ++i)
        if (i < nc) issue(i, i);
    for (int c = 0; c < nc; ++c) {
        wait_stages<kDma, kStages - 2>(nc - 1 - c);   // chunks c+1 .. c+kStages-2 may stay in flight
        __builtin_amdgcn_s_barrier();               // chunk c landed for every wave; stage of c-1 free
        asm volatile("" ::: "memory");
        if (c + kStages - 1 < nc) issue(c + kStages - 1, (c + kStages - 1) % kStages);
        if (c == 0) hook();
        const uint8_t* st = lds + (c % kStages) * kStageBytes;
        chunk_mma<MF, NF>(acc, st + (wm * MF * 16) * kRowBytes, st + (BM + wn * NF * 16) * kRowBytes, i16, g);
    }
}

template <int MF, int NF, int WM, int WN, int S, int EPI = kEpiStore>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w, int M, int N, int K) {
    using C = Tiled<MF, NF, WM, WN, S>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[C::kLdsBytes];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int m0 = blockIdx.y * C::BM, n0 = blockIdx.x * C::BN;
    f32x4_t acc[MF][NF];
    tiled_mainloop<MF, NF, WM, WN, S>(acc, lds, x, w, M, K, m0, n0);
    tile_epilogue<MF, NF, WN, EPI>(acc, y, M, N, m0, n0, wave / WN, wave % WN, lane & 15, lane >> 4);
}

// ---- tiled kernel with fused epilogues (the decode step's layer boundaries) ------------------
// kEpiResid (o_proj, down_proj): resid <- rnd(resid + rnd(x.w^T)), the residual add of
//   add_rms_norm (kernels/fused_ops.cu:70-73), and row_ss[m][n/16] <- the sum of squares of the
//   new residual over the 16 columns n .. n+15 (in column order, then lanes 4g combined by xor 16,
//   32), so the norm's sum over a row is the in-order sum of N/16 partials, whatever the tiling.
// RS (qkv, gate/up after such a producer): x rows are the raw residual v; the row's RMS factor
//   inv = 1 / sqrt(sum(row_ss) / K + eps) multiplies the accumulator before the epilogue's first
//   rounding, and the norm gain is pre-multiplied into the weight columns, so y = rnd(inv * v.w'^T)
//   with w' = rnd(w * gain) stands for rnd(rnd(rnd(v * inv) * gain) . w^T).
// kEpiQkv (qkv projection): the bf16 tile goes to LDS and every (row, head) of it runs the QK-norm
//   / RoPE / FP8 K/V write task (qkv_task_*) of the standalone kernel; BN is a whole number of
//   128-wide heads, so a tile holds complete heads.
enum { kEpiResid = 2, kEpiQkv = 3 };

struct FusedArgs {
    uint16_t* y;                 // kEpiStore: y [M][N]; kEpiSwiglu: act [M][N/2]; kEpiResid: resid [M][N]
    float* ss_out;               // kEpiResid: [M][N/16]
    const float* ss_in;          // RS: [M][K/16]
    float eps_in;                // RS: the row norm's eps
    const int64_t* positions;    // kEpiQkv
    const int64_t* slots;        // kEpiQkv
    QkvDst qkv;                  // kEpiQkv
};

constexpr int kMaxRsQuads = 4;   // RS: K / 256 float4 partial loads per lane (K <= 1024)

template <int MF, int NF, int WM, int WN, int S, int EPI, bool RS, int SM>
__global__ __launch_bounds__(256) void gemm_fused_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w, int M, int N, int K,
                                                         FusedArgs a) {
    using C = Tiled<MF, NF, WM, WN, S>;
    constexpr int BM = C::BM, BN = C::BN;
    constexpr int kTs = BN + 8;                                   // bf16 per LDS row of the kEpiQkv tile
    constexpr int kEpiLds = EPI == kEpiQkv ? BM * kTs * 2 : 0;
    constexpr int kLds = C::kLdsBytes > kEpiLds ? C::kLdsBytes : kEpiLds;
    constexpr int kHeads = BN / 128;                              // kEpiQkv: heads per tile
    constexpr int kTasks = BM * kHeads;
    constexpr int kIter = (kTasks + 15) / 16;                     // tasks per 16-lane group
    static_assert(EPI != kEpiQkv || BN % 128 == 0, "whole heads per tile");
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    // Everything the epilogue reads from global memory is requested before the K loop's DMA (the
    // loop's own vmcnt waits then cover it too).
    float4 rsq[RS ? MF : 1][RS ? kMaxRsQuads : 1];
    if constexpr (RS) {
        const int nq = K >> 8;                                    // float4 per lane per row
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int m = min(m0 + (wm * MF + f) * 16 + i16, M - 1);
            const float4* p = reinterpret_cast<const float4*>(a.ss_in + static_cast<size_t>(m) * (K >> 4)) + g * nq;
#pragma unroll
            for (int q = 0; q < kMaxRsQuads; ++q) rsq[f][q] = q < nq ? p[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    uint2 hres[EPI == kEpiResid ? MF : 1][EPI == kEpiResid ? NF : 1];
    if constexpr (EPI == kEpiResid) {
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int m = min(m0 + (wm * MF + f) * 16 + i16, M - 1);
#pragma unroll
            for (int e = 0; e < NF; ++e)
                hres[f][e] = *reinterpret_cast<const uint2*>(a.y + static_cast<size_t>(m) * N + n0 +
                                                             (wn * NF + e) * 16 + 4 * g);
        }
    }
    int64_t tpos[EPI == kEpiQkv ? kIter : 1], tslot[EPI == kEpiQkv ? kIter : 1];
    if constexpr (EPI == kEpiQkv) {
#pragma unroll
        for (int it = 0; it < kIter; ++it) {
            const int r = (it * 16 + (static_cast<int>(threadIdx.x) >> 4)) / kHeads;
            const int m = min(m0 + min(r, BM - 1), M - 1);
            tpos[it] = a.positions[m];
            tslot[it] = a.slots[m];
        }
    }

    // kEpiQkv: the Q/K tasks' norm gains and cos/sin (which need the positions) are requested
    // inside the K loop
    QkvTaskIn<128> in[EPI == kEpiQkv ? kIter : 1];
    const int gl = threadIdx.x & 15, grp = threadIdx.x >> 4;
    auto hook = [&]() {
        if constexpr (EPI == kEpiQkv) {
#pragma unroll
            for (int it = 0; it < kIter; ++it)
                qkv_task_load_consts<128>(in[it], n0 / 128 + (it * 16 + grp) % kHeads, tpos[it], a.qkv, gl);
        }
    };
    f32x4_t acc[MF][NF];
    tiled_mainloop<MF, NF, WM, WN, S>(acc, lds, x, w, M, K, m0, n0, hook);

    if constexpr (RS) {
        const int nq = K >> 8;
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            float sum = 0.f;
#pragma unroll
            for (int q = 0; q < kMaxRsQuads; ++q) {
                if (q < nq) {
                    sum = sum + rsq[f][q].x;
                    sum = sum + rsq[f][q].y;
                    sum = sum + rsq[f][q].z;
                    sum = sum + rsq[f][q].w;
                }
            }
            sum = sum + shfl_xor(sum, 16);
            sum = sum + shfl_xor(sum, 32);
            const float inv = 1.0f / __builtin_sqrtf(sum / static_cast<float>(K) + a.eps_in);
#pragma unroll
            for (int e = 0; e < NF; ++e) acc[f][e] *= inv;
        }
    }

    if constexpr (EPI == kEpiStore || EPI == kEpiSwiglu) {
        tile_epilogue<MF, NF, WN, EPI>(acc, a.y, M, N, m0, n0, wm, wn, i16, g);
    } else if constexpr (EPI == kEpiResid) {
        const int nss = N >> 4;
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int m = m0 + (wm * MF + f) * 16 + i16;
#pragma unroll
            for (int e = 0; e < NF; ++e) {
                const uint32_t y01 = pack_bf16x2(acc[f][e][0], acc[f][e][1]);
                const uint32_t y23 = pack_bf16x2(acc[f][e][2], acc[f][e][3]);
                const float yv[4] = {bf16_bits_to_f32(y01 & 0xffffu), bf16_bits_to_f32(y01 >> 16),
                                     bf16_bits_to_f32(y23 & 0xffffu), bf16_bits_to_f32(y23 >> 16)};
                const float hv[4] = {bf16_bits_to_f32(hres[f][e].x & 0xffffu), bf16_bits_to_f32(hres[f][e].x >> 16),
                                     bf16_bits_to_f32(hres[f][e].y & 0xffffu), bf16_bits_to_f32(hres[f][e].y >> 16)};
                uint32_t vb[4];
                float ss = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    vb[r] = f32_to_bf16_bits(hv[r] + yv[r]);
                    const float v = bf16_bits_to_f32(vb[r]);
                    ss = ss + v * v;
                }
                ss = ss + shfl_xor(ss, 16);
                ss = ss + shfl_xor(ss, 32);
                if (m < M) {
                    const int n = n0 + (wn * NF + e) * 16;
                    *reinterpret_cast<uint2*>(a.y + static_cast<size_t>(m) * N + n + 4 * g) =
                            make_uint2(vb[0] | (vb[1] << 16), vb[2] | (vb[3] << 16));
                    if (g == 0) a.ss_out[static_cast<size_t>(m) * nss + (n >> 4)] = ss;
                }
            }
        }
    } else {
        // kEpiQkv: bf16 tile [BM][kTs] in LDS (the stages are free once every wave has left the loop)
        __syncthreads();
        uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int r = (wm * MF + f) * 16 + i16;
#pragma unroll
            for (int e = 0; e < NF; ++e) {
                uint2 v;
                v.x = pack_bf16x2(acc[f][e][0], acc[f][e][1]);
                v.y = pack_bf16x2(acc[f][e][2], acc[f][e][3]);
                *reinterpret_cast<uint2*>(tile + r * kTs + (wn * NF + e) * 16 + 4 * g) = v;
            }
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < kIter; ++it) {
            const int idx = it * 16 + grp;
            qkv_task_load_x<128>(in[it], tile + min(idx / kHeads, BM - 1) * kTs + (idx % kHeads) * 128, gl);
        }
#pragma unroll
        for (int it = 0; it < kIter; ++it) {
            const int idx = it * 16 + grp;
            const int m = m0 + idx / kHeads;
            if (idx < kTasks && m < M) qkv_task_run<128, SM>(in[it], m, n0 / 128 + idx % kHeads, tslot[it], a.qkv, gl);
        }
    }
}

typedef void (*GemmFn)(uint16_t*, const uint16_t*, const uint16_t*, int, int, int);

struct GemmCfg {
    int mf, nwn, xlds, nc;         // nc > 0: one-shot kernel with exactly nc chunks per wave
    GemmFn fn;
    int nf = 0, wm = 0, st = 0;    // nf > 0: tiled kernel, MF x NF fragments per wave, WM x nwn waves,
                                   // st LDS stages (0: as many as fit)
    int code() const {
        if (nf) return 100000 * (st ? st : 9) + 20000 + 1000 * mf + 100 * nf + 10 * wm + nwn;
        return nc ? 10000 + 100 * nc + 10 * mf + nwn : 100 * xlds + 10 * mf + nwn;
    }
    int bm() const { return nf ? 16 * mf * wm : 16 * mf; }
    int bn() const { return nf ? 16 * nf * nwn : 16 * nwn; }
};

#define CVH_GEMM_CFG(MF, NWN, X) GemmCfg{MF, NWN, X, 0, gemm_nt_kernel<MF, NWN, X>}
#define CVH_GEMM_ONE(MF, NWN, NC) GemmCfg{MF, NWN, 1, NC, gemm_oneshot_kernel<MF, NWN, NC>}
#define CVH_GEMM_TILE(MF, NF, WM, WN, S) GemmCfg{MF, WN, 1, 0, gemm_tiled_kernel<MF, NF, WM, WN, S>, NF, WM, S}
const GemmCfg kCfgs[] = {
    CVH_GEMM_CFG(1, 1, 0), CVH_GEMM_CFG(1, 2, 0), CVH_GEMM_CFG(1, 4, 0),
    CVH_GEMM_CFG(2, 1, 0), CVH_GEMM_CFG(2, 2, 0), CVH_GEMM_CFG(2, 4, 0),
    CVH_GEMM_CFG(4, 1, 0), CVH_GEMM_CFG(4, 2, 0), CVH_GEMM_CFG(4, 4, 0),
    CVH_GEMM_CFG(1, 2, 1), CVH_GEMM_CFG(1, 4, 1),
    CVH_GEMM_CFG(2, 2, 1), CVH_GEMM_CFG(2, 4, 1),
    CVH_GEMM_CFG(4, 2, 1), CVH_GEMM_CFG(4, 4, 1),
    CVH_GEMM_CFG(8, 4, 1),
    // K = 1024
    CVH_GEMM_ONE(1, 4, 8), CVH_GEMM_ONE(2, 4, 8), CVH_GEMM_ONE(4, 4, 8),
    CVH_GEMM_ONE(1, 2, 4), CVH_GEMM_ONE(2, 2, 4), CVH_GEMM_ONE(4, 2, 4),
    CVH_GEMM_ONE(1, 1, 2), CVH_GEMM_ONE(2, 1, 2), CVH_GEMM_ONE(4, 1, 2),
    // K = 2048
    CVH_GEMM_ONE(1, 2, 8), CVH_GEMM_ONE(2, 2, 8),
    CVH_GEMM_ONE(1, 1, 4), CVH_GEMM_ONE(2, 1, 4),
    // K = 3072
    CVH_GEMM_ONE(1, 1, 6), CVH_GEMM_ONE(1, 2, 12),
    // tiled, any K % 128 == 0
    CVH_GEMM_TILE(1, 1, 4, 1, 3), CVH_GEMM_TILE(1, 1, 2, 2, 3), CVH_GEMM_TILE(1, 1, 1, 4, 3),
    CVH_GEMM_TILE(2, 1, 2, 2, 3), CVH_GEMM_TILE(1, 2, 2, 2, 3), CVH_GEMM_TILE(2, 2, 2, 2, 3),
    CVH_GEMM_TILE(2, 1, 4, 1, 3), CVH_GEMM_TILE(1, 2, 1, 4, 3), CVH_GEMM_TILE(4, 1, 1, 4, 3),
    CVH_GEMM_TILE(2, 4, 2, 2, 3), CVH_GEMM_TILE(4, 2, 2, 2, 3), CVH_GEMM_TILE(1, 2, 4, 1, 3),
    CVH_GEMM_TILE(2, 1, 1, 4, 3), CVH_GEMM_TILE(2, 2, 1, 4, 3),
    CVH_GEMM_TILE(1, 1, 2, 2, 0), CVH_GEMM_TILE(1, 1, 4, 1, 0), CVH_GEMM_TILE(2, 1, 2, 2, 0),
};
#undef CVH_GEMM_CFG
#undef CVH_GEMM_ONE
#undef CVH_GEMM_TILE

// Tiled configurations with the SwiGLU epilogue (an even number of column fragments per wave).
#define CVH_GEMM_SWIGLU(MF, NF, WM, WN, S) \
    GemmCfg{MF, WN, 1, 0, gemm_tiled_kernel<MF, NF, WM, WN, S, kEpiSwiglu>, NF, WM, S}
const GemmCfg kSwigluCfgs[] = {
    CVH_GEMM_SWIGLU(1, 2, 2, 2, 3), CVH_GEMM_SWIGLU(2, 2, 2, 2, 3), CVH_GEMM_SWIGLU(2, 4, 2, 2, 3),
    CVH_GEMM_SWIGLU(1, 2, 1, 4, 3), CVH_GEMM_SWIGLU(1, 2, 4, 1, 3), CVH_GEMM_SWIGLU(4, 2, 2, 2, 3),
    CVH_GEMM_SWIGLU(2, 2, 1, 4, 3),
};
#undef CVH_GEMM_SWIGLU

const GemmCfg* find_swiglu_cfg(int code) {
    for (const GemmCfg& c : kSwigluCfgs)
        if (c.code() == code) return &c;
    return nullptr;
}

const GemmCfg* find_cfg(int code) {
    for (const GemmCfg& c : kCfgs)
        if (c.code() == code) return &c;
    return nullptr;
}

// Automatic choice. For the Qwen3-0.6B decode projections the configuration is the fastest one
// measured on MI355X (HIP-graph replay, weights cold in the last-level cache) for the largest
// row count of each bucket; other shapes take the generic rule below.
struct ShapeRule {
    int n, k;
    int max_m[8];
    int code[8];
};
const ShapeRule kRules[] = {
    {4096, 1024, {8, 16, 32, 96, 128, 1 << 30}, {11, 10211, 10221, 321122, 322122, 322222}},      // qkv
    {1024, 2048, {8, 64, 1 << 30}, {11, 10411, 321122}},                                          // o_proj
    {6144, 1024, {1, 16, 32, 64, 128, 1 << 30}, {11, 112, 321122, 322122, 322222, 322422}},       // gate_up
    {1024, 3072, {8, 64, 96, 1 << 30}, {11, 10611, 921141, 921122}},                              // down
    {151936, 1024, {8, 16, 32, 64, 1 << 30}, {321122, 321114, 321222, 322422, 324222}},           // lm_head
};

const GemmCfg* auto_cfg(int64_t M, int N, int K) {
    for (const ShapeRule& r : kRules) {
        if (r.n != N || r.k != K) continue;
        for (int b = 0; b < 8; ++b)
            if (M <= r.max_m[b]) return find_cfg(r.code[b]);
    }
    if (M <= 16 && K % (4 * kChunk) == 0) return find_cfg(11);      // weight streaming, K split over 4 waves
    if (N % 32 == 0) return find_cfg(321122);                       // 32 x 32 tiles through LDS
    return find_cfg(321141);                                        // 64 x 16 tiles
}

}  // namespace
}  // namespace cvh

extern "C" int cvh_gemm_bf16_nt(void* y, const void* x, const void* w, int64_t M, int N, int K, int config,
                                cvh_stream_t stream) {
    using namespace cvh;
    if (M < 0 || N <= 0 || K <= 0) return CVH_ERR_INVALID_ARG;
    if (M == 0) return CVH_OK;
    if (!y || !x || !w) return CVH_ERR_INVALID_ARG;
    if (M > (1 << 20) || N % 16 || K % kChunk) return CVH_ERR_UNSUPPORTED;
    const GemmCfg* cfg = config > 0 ? find_cfg(config) : auto_cfg(M, N, K);
    if (!cfg || N % cfg->bn()) return CVH_ERR_UNSUPPORTED;
    if (!cfg->nf && K % ((4 / cfg->nwn) * kChunk)) return CVH_ERR_UNSUPPORTED;
    if (cfg->nc && K != (4 / cfg->nwn) * cfg->nc * kChunk) return CVH_ERR_UNSUPPORTED;
    const dim3 grid(N / cfg->bn(), static_cast<unsigned>((M + cfg->bm() - 1) / cfg->bm()));
    hipLaunchKernelGGL(cfg->fn, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                       static_cast<int>(M), N, K);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

namespace cvh {
namespace {
// Measured fastest SwiGLU-epilogue configuration for the Qwen3-0.6B gate/up shape (I = 3072,
// K = 1024) per row-count bucket (64 x 32 tiles up to 64 rows, 32 x 64 up to 128, 64 x 128 above);
// other shapes take 32 x 64 tiles.
const GemmCfg* auto_swiglu_cfg(int64_t M, int I, int K) {
    if (I == 3072 && K == 1024) return find_swiglu_cfg(M <= 64 ? 321241 : M <= 128 ? 321222 : 322422);
    return find_swiglu_cfg(321222);
}
}  // namespace
}  // namespace cvh

extern "C" int cvh_gemm_bf16_nt_swiglu(void* act, const void* x, const void* w, int64_t M, int I, int K, int config,
                                       cvh_stream_t stream) {
    using namespace cvh;
    if (M < 0 || I <= 0 || K <= 0) return CVH_ERR_INVALID_ARG;
    if (M == 0) return CVH_OK;
    if (!act || !x || !w) return CVH_ERR_INVALID_ARG;
    if (M > (1 << 20) || I % 16 || K % kChunk || I > (1 << 29)) return CVH_ERR_UNSUPPORTED;
    const int N = 2 * I;
    const GemmCfg* cfg = config > 0 ? find_swiglu_cfg(config) : auto_swiglu_cfg(M, I, K);
    if (!cfg || N % cfg->bn()) return CVH_ERR_UNSUPPORTED;
    const dim3 grid(N / cfg->bn(), static_cast<unsigned>((M + cfg->bm() - 1) / cfg->bm()));
    hipLaunchKernelGGL(cfg->fn, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<uint16_t*>(act), static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                       static_cast<int>(M), N, K);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

extern "C" int cvh_gemm_bf16_nt_swiglu_config(int64_t M, int I, int K) {
    const cvh::GemmCfg* c = cvh::auto_swiglu_cfg(M, I, K);
    return c ? c->code() : 0;
}

extern "C" int cvh_gemm_bf16_nt_swiglu_configs(int* codes, int capacity) {
    int n = 0;
    for (const cvh::GemmCfg& c : cvh::kSwigluCfgs) {
        if (codes && n < capacity) codes[n] = c.code();
        ++n;
    }
    return n;
}

extern "C" int cvh_gemm_bf16_nt_configs(int* codes, int capacity) {
    int n = 0;
    for (const cvh::GemmCfg& c : cvh::kCfgs) {
        if (codes && n < capacity) codes[n] = c.code();
        ++n;
    }
    return n;
}

extern "C" int cvh_gemm_bf16_nt_config(int64_t M, int N, int K) {
    const cvh::GemmCfg* c = cvh::auto_cfg(M, N, K);
    return c ? c->code() : 0;
}

// ---- fused-epilogue entry points -------------------------------------------------------------
namespace cvh {
namespace {

typedef void (*FusedFn)(const uint16_t*, const uint16_t*, int, int, int, FusedArgs);
struct FusedCfg {
    int code, bm, bn;
    FusedFn fn;
};
constexpr int tiled_code(int mf, int nf, int wm, int wn, int st) {
    return 100000 * (st ? st : 9) + 20000 + 1000 * mf + 100 * nf + 10 * wm + wn;
}
#define CVH_FUSED(MF, NF, WM, WN, S, EPI, RS, SM) \
    FusedCfg{tiled_code(MF, NF, WM, WN, S), 16 * MF * WM, 16 * NF * WN, gemm_fused_kernel<MF, NF, WM, WN, S, EPI, RS, SM>}
const FusedCfg kResidCfgs[] = {
    CVH_FUSED(1, 1, 2, 2, 3, kEpiResid, false, 0), CVH_FUSED(1, 1, 2, 2, 0, kEpiResid, false, 0),
    CVH_FUSED(1, 1, 4, 1, 3, kEpiResid, false, 0), CVH_FUSED(1, 1, 4, 1, 0, kEpiResid, false, 0),
    CVH_FUSED(2, 1, 2, 2, 3, kEpiResid, false, 0), CVH_FUSED(1, 2, 2, 2, 3, kEpiResid, false, 0),
    CVH_FUSED(2, 1, 4, 1, 3, kEpiResid, false, 0), CVH_FUSED(1, 1, 1, 4, 3, kEpiResid, false, 0),
};
const FusedCfg kSwigluRsCfgs[] = {
    CVH_FUSED(1, 2, 4, 1, 3, kEpiSwiglu, true, 0), CVH_FUSED(1, 2, 2, 2, 3, kEpiSwiglu, true, 0),
    CVH_FUSED(2, 2, 2, 2, 3, kEpiSwiglu, true, 0), CVH_FUSED(2, 4, 2, 2, 3, kEpiSwiglu, true, 0),
    CVH_FUSED(1, 2, 1, 4, 3, kEpiSwiglu, true, 0),
};
#define CVH_QKV_CFGS(RS, SM)                                                                                 \
    CVH_FUSED(1, 2, 1, 4, 3, kEpiQkv, RS, SM), CVH_FUSED(2, 2, 1, 4, 3, kEpiQkv, RS, SM),                    \
    CVH_FUSED(1, 4, 2, 2, 3, kEpiQkv, RS, SM), CVH_FUSED(2, 4, 2, 2, 3, kEpiQkv, RS, SM)
const FusedCfg kQkvCfgs[2][2][4] = {
    {{CVH_QKV_CFGS(false, CVH_SCALE_PER_TOKEN_HEAD)}, {CVH_QKV_CFGS(false, CVH_SCALE_PER_TENSOR)}},
    {{CVH_QKV_CFGS(true, CVH_SCALE_PER_TOKEN_HEAD)}, {CVH_QKV_CFGS(true, CVH_SCALE_PER_TENSOR)}},
};
#undef CVH_QKV_CFGS
#undef CVH_FUSED

enum { kFusedResidual = 0, kFusedSwigluRownorm = 1, kFusedQkv = 2 };

template <size_t NC>
const FusedCfg* find_fused(const FusedCfg (&t)[NC], int code) {
    for (const FusedCfg& c : t)
        if (c.code == code) return &c;
    return nullptr;
}

// Automatic tile per row count (measured on MI355X for the Qwen3-0.6B decode shapes).
int auto_fused_code(int kind, int64_t M) {
    switch (kind) {
        case kFusedResidual: return tiled_code(1, 1, 2, 2, 0);
        case kFusedSwigluRownorm:
            return M <= 64 ? tiled_code(1, 2, 4, 1, 3) : M <= 128 ? tiled_code(1, 2, 2, 2, 3) : tiled_code(2, 4, 2, 2, 3);
        default: return M <= 128 ? tiled_code(1, 2, 1, 4, 3) : tiled_code(1, 4, 2, 2, 3);
    }
}

const FusedCfg* fused_cfg(int kind, int code, bool rs, int sm) {
    switch (kind) {
        case kFusedResidual: return find_fused(kResidCfgs, code);
        case kFusedSwigluRownorm: return find_fused(kSwigluRsCfgs, code);
        case kFusedQkv: return find_fused(kQkvCfgs[rs ? 1 : 0][sm == CVH_SCALE_PER_TENSOR ? 1 : 0], code);
        default: return nullptr;
    }
}

int launch_fused(const FusedCfg* c, const void* x, const void* w, int64_t M, int N, int K, const FusedArgs& a,
                 cvh_stream_t stream) {
    if (!c || N % c->bn) return CVH_ERR_UNSUPPORTED;
    const dim3 grid(N / c->bn, static_cast<unsigned>((M + c->bm - 1) / c->bm));
    hipLaunchKernelGGL(c->fn, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<int>(M), N, K, a);
    return hipGetLastError() == hipSuccess ? CVH_OK : CVH_ERR_LAUNCH;
}

bool rs_shape_ok(int K) { return K % 256 == 0 && K / 256 <= kMaxRsQuads; }

}  // namespace
}  // namespace cvh

extern "C" int cvh_gemm_bf16_nt_residual(void* resid, float* row_ss, const void* x, const void* w, int64_t M, int N,
                                         int K, int config, cvh_stream_t stream) {
    using namespace cvh;
    if (M < 0 || N <= 0 || K <= 0) return CVH_ERR_INVALID_ARG;
    if (M == 0) return CVH_OK;
    if (!resid || !row_ss || !x || !w) return CVH_ERR_INVALID_ARG;
    if (M > (1 << 20) || N % 16 || K % kChunk || N > (1 << 20)) return CVH_ERR_UNSUPPORTED;
    FusedArgs a{};
    a.y = static_cast<uint16_t*>(resid);
    a.ss_out = row_ss;
    const int code = config > 0 ? config : auto_fused_code(kFusedResidual, M);
    return launch_fused(fused_cfg(kFusedResidual, code, false, 0), x, w, M, N, K, a, stream);
}

extern "C" int cvh_gemm_bf16_nt_swiglu_rownorm(void* act, const void* x, const float* row_ss, double eps,
                                               const void* w, int64_t M, int I, int K, int config,
                                               cvh_stream_t stream) {
    using namespace cvh;
    if (M < 0 || I <= 0 || K <= 0) return CVH_ERR_INVALID_ARG;
    if (M == 0) return CVH_OK;
    if (!act || !x || !row_ss || !w) return CVH_ERR_INVALID_ARG;
    if (M > (1 << 20) || I % 16 || K % kChunk || I > (1 << 19) || !rs_shape_ok(K)) return CVH_ERR_UNSUPPORTED;
    FusedArgs a{};
    a.y = static_cast<uint16_t*>(act);
    a.ss_in = row_ss;
    a.eps_in = static_cast<float>(eps);
    const int code = config > 0 ? config : auto_fused_code(kFusedSwigluRownorm, M);
    return launch_fused(fused_cfg(kFusedSwigluRownorm, code, true, 0), x, w, M, 2 * I, K, a, stream);
}

extern "C" int cvh_gemm_qkv_norm_rope_kv_write_fp8(
        void* q_out, const void* x, const float* row_ss, double x_eps, const void* w_qkv, const void* q_norm,
        const void* k_norm, const float* cos_t, const float* sin_t, const int64_t* positions, const int64_t* slots,
        uint8_t* k_cache, uint8_t* v_cache, float* k_scale, float* v_scale, int64_t num_tokens, int dim, int n_heads,
        int n_kv_heads, int head_dim, int block_size, int scale_mode, double eps, int config, cvh_stream_t stream) {
    using namespace cvh;
    if (num_tokens < 0 || dim <= 0 || n_heads <= 0 || n_kv_heads <= 0) return CVH_ERR_INVALID_ARG;
    if (num_tokens == 0) return CVH_OK;
    if (!q_out || !x || !w_qkv || !q_norm || !k_norm || !cos_t || !sin_t || !positions || !slots || !k_cache ||
        !v_cache || !k_scale || !v_scale)
        return CVH_ERR_INVALID_ARG;
    if (head_dim != 128 || num_tokens > (1 << 20) || dim % kChunk || (row_ss && !rs_shape_ok(dim)))
        return CVH_ERR_UNSUPPORTED;
    if (scale_mode != CVH_SCALE_PER_TOKEN_HEAD && scale_mode != CVH_SCALE_PER_TENSOR) return CVH_ERR_UNSUPPORTED;
    int lg = 0;
    while ((1 << lg) < block_size) ++lg;
    if ((1 << lg) != block_size || lg < 4 || lg > 12) return CVH_ERR_UNSUPPORTED;
    const int N = (n_heads + 2 * n_kv_heads) * head_dim;
    FusedArgs a{};
    a.ss_in = row_ss;
    a.eps_in = static_cast<float>(x_eps);
    a.positions = positions;
    a.slots = slots;
    a.qkv = QkvDst{static_cast<uint16_t*>(q_out), static_cast<const uint16_t*>(q_norm),
                   static_cast<const uint16_t*>(k_norm), cos_t, sin_t, k_cache, v_cache, k_scale, v_scale, nullptr,
                   nullptr, n_heads, n_kv_heads, lg, static_cast<float>(eps)};
    const int code = config > 0 ? config : auto_fused_code(kFusedQkv, num_tokens);
    return launch_fused(fused_cfg(kFusedQkv, code, row_ss != nullptr, scale_mode), x, w_qkv, num_tokens, N, dim, a,
                        stream);
}

extern "C" int cvh_gemm_fused_configs(int kind, int* codes, int capacity) {
    using namespace cvh;
    const FusedCfg* t = nullptr;
    int n = 0;
    switch (kind) {
        case kFusedResidual: t = kResidCfgs; n = static_cast<int>(sizeof(kResidCfgs) / sizeof(FusedCfg)); break;
        case kFusedSwigluRownorm:
            t = kSwigluRsCfgs;
            n = static_cast<int>(sizeof(kSwigluRsCfgs) / sizeof(FusedCfg));
            break;
        case kFusedQkv: t = kQkvCfgs[0][0]; n = 4; break;
        default: return 0;
    }
    for (int i = 0; i < n && codes && i < capacity; ++i) codes[i] = t[i].code;
    return n;
}

extern "C" int cvh_gemm_fused_config(int kind, int64_t M) {
    return kind >= 0 && kind <= 2 ? cvh::auto_fused_code(kind, M) : 0;
}
