// Decode-step runner: staging, the layer loop through the C ABI, and HIP-graph capture / replay.
//
// Reference: engine/model_runner.cpp:169-212 (launch / collect), :327-357 (graph rows: idle rows on
// the scratch block at kv_len 1), :371-428 (capture one graph per batch size, replay the smallest
// size >= the row count); model/model_architecture.cpp:130-191 (the backbone the graph holds).
// Everything here is host code over the library's extern "C" entry points and the HIP runtime; the
// only allocations are in cvh_runner_create / cvh_runner_capture.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <set>
#include <utility>
#include <vector>

#include "../../include/cppvllm_runner.h"

namespace {

#define CVR_CHECK(call)                        \
    do {                                       \
        const int rc_ = (call);                \
        if (rc_ != CVH_OK) return rc_;         \
    } while (0)

int hip_ok(hipError_t e) {
    if (e == hipSuccess) return CVH_OK;
    (void)hipGetLastError();
    return CVH_ERR_LAUNCH;
}

}  // namespace

struct cvh_runner;
namespace {
// Live runners: every entry point checks its handle here first, so a stale or foreign pointer is
// rejected with CVH_ERR_INVALID_ARG instead of being dereferenced.
std::mutex g_live_mu;
std::set<const cvh_runner*> g_live;
bool live(const cvh_runner* r) {
    std::lock_guard<std::mutex> lock(g_live_mu);
    return r != nullptr && g_live.count(r) != 0;
}
}  // namespace

struct cvh_runner {
    cvh_runner_desc d{};
    std::vector<cvh_runner_layer> layers;
    int64_t qkv_n = 0;                // (H + 2 KV) * HD
    int ss_slots = 0;                 // D / 16 row sums of squares
    // device input arena (int64): tok | pos | cu | feed | shared (int32 pairs) | tables (B x W)
    int64_t off[6] = {};
    int64_t arena_len = 0;
    int64_t* arena = nullptr;
    int64_t* h_arena[2] = {nullptr, nullptr};   // pinned staging, one per launch slot
    // per-token metadata and activations for max_batch rows
    int64_t *seq = nullptr, *slot = nullptr, *kvl = nullptr;
    void *h = nullptr, *x = nullptr, *q = nullptr, *att = nullptr, *act = nullptr, *qkv = nullptr, *o = nullptr;
    float* ss = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    hipStream_t capture_stream = nullptr;
    std::map<std::pair<int, int>, std::pair<hipGraph_t, hipGraphExec_t>> graphs;

    int64_t* tok() const { return arena + off[0]; }
    int64_t* pos() const { return arena + off[1]; }
    int64_t* cu() const { return arena + off[2]; }
    int64_t* feed() const { return arena + off[3]; }
    int32_t* shared() const { return reinterpret_cast<int32_t*>(arena + off[4]); }
    int64_t* tables() const { return arena + off[5]; }

    ~cvh_runner() {
        for (auto& g : graphs) {
            (void)hipGraphExecDestroy(g.second.second);
            (void)hipGraphDestroy(g.second.first);
        }
        for (void* p : {static_cast<void*>(arena), static_cast<void*>(seq), static_cast<void*>(slot),
                        static_cast<void*>(kvl), h, x, q, att, act, qkv, o, static_cast<void*>(ss), ws})
            if (p) (void)hipFree(p);
        for (int64_t* p : h_arena)
            if (p) (void)hipHostFree(p);
        if (capture_stream) (void)hipStreamDestroy(capture_stream);
    }

    bool fused(int B) const { return d.fused_min_rows <= B && B <= d.fused_max_rows; }

    // The backbone over the staged rows [0, B) (model_architecture.cpp:149-188, with the planned
    // attention of this library), then the final norm into desc.hidden.
    int forward(int B, bool sh, hipStream_t s) {
        const cvh_runner_desc& c = d;
        const int D = c.dim, H = c.n_heads, KV = c.n_kv_heads, HD = c.head_dim, I = c.intermediate;
        const int64_t W = c.table_width;
        const double eps = c.norm_eps;
        CVR_CHECK(cvh_build_token_metadata(cu(), B, pos(), B, tables(), W, c.block_size, seq, slot, kvl, s));
        CVR_CHECK(cvh_embedding(h, c.embed, tok(), B, D, c.vocab, s));
        if (sh)
            CVR_CHECK(cvh_paged_attention_plan_shared(tables(), W, seq, kvl, shared(), B, H, KV, HD, c.block_size, 0,
                                                      ws, ws_bytes, s));
        else
            CVR_CHECK(cvh_paged_attention_plan(tables(), W, seq, kvl, B, H, KV, HD, c.block_size, 0, ws, ws_bytes, s));
        auto attention = [&](const cvh_runner_layer& L) {
            auto fn = sh ? cvh_paged_attention_fp8_planned_shared : cvh_paged_attention_fp8_planned;
            return fn(att, q, L.k_cache, L.v_cache, L.k_scale, L.v_scale, tables(), W, seq, kvl, B, H, KV, HD,
                      c.block_size, c.scale_mode, c.attn_scale, 0, ws, ws_bytes, s);
        };
        if (fused(B)) {
            // layer boundaries in the projections' epilogues; layer 0's input normed with a unit gain
            CVR_CHECK(cvh_rms_norm(x, h, c.unit_gain, B, D, eps, CVH_DTYPE_BF16, s));
            for (int li = 0; li < c.n_layers; ++li) {
                const cvh_runner_layer& L = layers[li];
                CVR_CHECK(cvh_gemm_qkv_norm_rope_kv_write_fp8(
                        q, li == 0 ? x : h, li == 0 ? nullptr : ss, eps, L.w_qkv_folded, L.q_norm, L.k_norm,
                        c.rope_cos, c.rope_sin, pos(), slot, L.k_cache, L.v_cache, L.k_scale, L.v_scale, B, D, H, KV,
                        HD, c.block_size, c.scale_mode, eps, 0, s));
                CVR_CHECK(attention(L));
                CVR_CHECK(cvh_gemm_bf16_nt_residual(h, ss, att, L.w_o, B, D, H * HD, 0, s));
                CVR_CHECK(cvh_gemm_bf16_nt_swiglu_rownorm(act, h, ss, eps, L.w_gate_up_folded, B, I, D, 0, s));
                CVR_CHECK(cvh_gemm_bf16_nt_residual(h, ss, act, L.w_down, B, D, I, 0, s));
            }
            return cvh_rms_norm(c.hidden, h, c.final_norm, B, D, eps, CVH_DTYPE_BF16, s);
        }
        CVR_CHECK(cvh_rms_norm(x, h, layers[0].attn_norm, B, D, eps, CVH_DTYPE_BF16, s));
        for (int li = 0; li < c.n_layers; ++li) {
            const cvh_runner_layer& L = layers[li];
            CVR_CHECK(cvh_gemm_bf16_nt(qkv, x, L.w_qkv, B, static_cast<int>(qkv_n), D, 0, s));
            CVR_CHECK(cvh_qk_norm_rope_kv_write_fp8(q, qkv, L.q_norm, L.k_norm, c.rope_cos, c.rope_sin, pos(), slot,
                                                    L.k_cache, L.v_cache, L.k_scale, L.v_scale, nullptr, nullptr, B,
                                                    H, KV, HD, c.block_size, c.scale_mode, eps, s));
            CVR_CHECK(attention(L));
            CVR_CHECK(cvh_gemm_bf16_nt(o, att, L.w_o, B, D, H * HD, 0, s));
            CVR_CHECK(cvh_add_rms_norm(h, o, L.ffn_norm, x, B, D, eps, CVH_DTYPE_BF16, s));
            CVR_CHECK(cvh_gemm_bf16_nt_swiglu(act, x, L.w_gate_up, B, I, D, 0, s));
            CVR_CHECK(cvh_gemm_bf16_nt(o, act, L.w_down, B, D, I, 0, s));
            const bool last = li + 1 == c.n_layers;
            CVR_CHECK(cvh_add_rms_norm(h, o, last ? c.final_norm : layers[li + 1].attn_norm, last ? c.hidden : x, B,
                                       D, eps, CVH_DTYPE_BF16, s));
        }
        return CVH_OK;
    }
};

extern "C" int cvh_runner_create(const cvh_runner_desc* desc, cvh_runner** out) {
    if (out == nullptr) return CVH_ERR_INVALID_ARG;
    *out = nullptr;
    if (desc == nullptr || desc->layers == nullptr || desc->n_layers <= 0 || desc->dim <= 0 || desc->dim % 256 != 0 ||
        desc->n_heads <= 0 || desc->n_kv_heads <= 0 || desc->n_heads % desc->n_kv_heads != 0 ||
        desc->head_dim <= 0 || desc->intermediate <= 0 || desc->vocab <= 0 || desc->max_batch <= 0 ||
        desc->max_batch > 256 || desc->table_width <= 0 || desc->block_size <= 0 || desc->scratch_block < 0 ||
        desc->embed == nullptr || desc->final_norm == nullptr || desc->unit_gain == nullptr ||
        desc->rope_cos == nullptr || desc->rope_sin == nullptr || desc->hidden == nullptr)
        return CVH_ERR_INVALID_ARG;
    // the decode projections run on cvh_gemm_* (N % 16 == 0, K % 128 == 0; gate/up interleaved by 16)
    const int64_t qkv_n = static_cast<int64_t>(desc->n_heads + 2 * desc->n_kv_heads) * desc->head_dim;
    if (desc->dim % 128 != 0 || (desc->n_heads * desc->head_dim) % 128 != 0 || desc->intermediate % 128 != 0 ||
        (2 * desc->intermediate) % 32 != 0 || qkv_n % 16 != 0)
        return CVH_ERR_UNSUPPORTED;
    // the fused-epilogue projections: 128-wide heads, rows of at most 1024 (the row-norm partials a
    // lane sums), 256-column tiles over the hidden size, 128-column gate/up tiles
    if (desc->fused_min_rows <= desc->fused_max_rows &&
        (desc->head_dim != 128 || desc->dim > 1024 || (2 * desc->intermediate) % 128 != 0 || desc->fused_min_rows < 1))
        return CVH_ERR_UNSUPPORTED;
    for (int i = 0; i < desc->n_layers; ++i) {
        const cvh_runner_layer& L = desc->layers[i];
        if (!L.w_qkv || !L.w_o || !L.w_gate_up || !L.w_down || !L.attn_norm || !L.ffn_norm || !L.q_norm || !L.k_norm ||
            !L.k_cache || !L.v_cache || !L.k_scale || !L.v_scale)
            return CVH_ERR_INVALID_ARG;
        if (desc->fused_min_rows <= desc->fused_max_rows && (!L.w_qkv_folded || !L.w_gate_up_folded))
            return CVH_ERR_INVALID_ARG;
    }
    cvh_runner* r = new (std::nothrow) cvh_runner();
    if (r == nullptr) return CVH_ERR_LAUNCH;
    r->d = *desc;
    r->layers.assign(desc->layers, desc->layers + desc->n_layers);
    r->d.layers = nullptr;
    r->qkv_n = qkv_n;
    r->ss_slots = desc->dim / 16;
    const int64_t Bm = desc->max_batch, W = desc->table_width;
    const int64_t lens[6] = {Bm, Bm, Bm + 1, Bm, (Bm + 1) / 2, Bm * W};
    for (int i = 0; i < 6; ++i) r->off[i] = (i ? r->off[i - 1] + lens[i - 1] : 0);
    r->arena_len = r->off[5] + lens[5];
    const int D = desc->dim, HD = desc->head_dim, H = desc->n_heads;
    // the shared-prefix layout: the shared graphs plan prefix-sharing units in the same workspace
    r->ws_bytes = cvh_paged_attention_workspace_bytes_shared(Bm, H, desc->n_kv_heads, HD, W, desc->block_size, 0);
    int rc = CVH_OK;
    auto dmalloc = [&](auto** p, size_t bytes) {
        if (rc == CVH_OK && hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(bytes, 256)) != hipSuccess) {
            (void)hipGetLastError();
            *p = nullptr;
            rc = CVH_ERR_LAUNCH;
        }
    };
    dmalloc(&r->arena, r->arena_len * 8);
    dmalloc(&r->seq, Bm * 8);
    dmalloc(&r->slot, Bm * 8);
    dmalloc(&r->kvl, Bm * 8);
    dmalloc(&r->h, Bm * D * 2);
    dmalloc(&r->x, Bm * D * 2);
    dmalloc(&r->q, Bm * H * HD * 2);
    dmalloc(&r->att, Bm * H * HD * 2);
    dmalloc(&r->act, Bm * desc->intermediate * 2);
    dmalloc(&r->qkv, Bm * qkv_n * 2);
    dmalloc(&r->o, Bm * D * 2);
    dmalloc(&r->ss, Bm * r->ss_slots * 4);
    dmalloc(&r->ws, r->ws_bytes);
    for (auto& p : r->h_arena)
        if (rc == CVH_OK && hipHostMalloc(reinterpret_cast<void**>(&p), r->arena_len * 8, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            rc = CVH_ERR_LAUNCH;
        }
    if (rc == CVH_OK && hipStreamCreateWithFlags(&r->capture_stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        r->capture_stream = nullptr;
        rc = CVH_ERR_LAUNCH;
    }
    if (rc == CVH_OK) {
        // a defined arena before the first stage (capture reads its pointers, not its contents)
        std::memset(r->h_arena[0], 0, r->arena_len * 8);
        rc = hip_ok(hipMemcpy(r->arena, r->h_arena[0], r->arena_len * 8, hipMemcpyHostToDevice));
    }
    if (rc != CVH_OK) {
        delete r;
        return rc;
    }
    {
        std::lock_guard<std::mutex> lock(g_live_mu);
        g_live.insert(r);
    }
    *out = r;
    return CVH_OK;
}

extern "C" int cvh_runner_destroy(cvh_runner* r) {
    {
        std::lock_guard<std::mutex> lock(g_live_mu);
        if (r == nullptr || g_live.erase(r) == 0) return CVH_ERR_INVALID_ARG;
    }
    delete r;
    return CVH_OK;
}

extern "C" int cvh_runner_stage(cvh_runner* r, int slot, int64_t rows, int batch, const int64_t* tokens,
                                const int64_t* positions, const int64_t* tables, int64_t tables_width,
                                const int64_t* feed, const int32_t* shared_blocks, const int64_t* prev_sampled,
                                cvh_stream_t stream) {
    if (!live(r) || slot < 0 || slot > 1 || rows < 0 || batch <= 0 || batch > r->d.max_batch || rows > batch ||
        (rows > 0 && (tokens == nullptr || positions == nullptr || tables == nullptr || tables_width <= 0)))
        return CVH_ERR_INVALID_ARG;
    // a position past the runner's table width would be clamped by the kernels, not attended
    const int64_t max_pos = r->d.table_width * r->d.block_size;
    for (int64_t i = 0; i < rows; ++i)
        if (positions[i] < 0 || positions[i] >= max_pos) return CVH_ERR_INVALID_ARG;
    bool need_feed = false;
    if (feed != nullptr)
        for (int64_t i = 0; i < rows && !need_feed; ++i) need_feed = feed[i] >= 0;
    if (need_feed && prev_sampled == nullptr) return CVH_ERR_INVALID_ARG;
    int64_t* hst = r->h_arena[slot];
    const int64_t* o = r->off;
    const int64_t W = r->d.table_width, B = batch;
    for (int64_t i = 0; i < B; ++i) {
        hst[o[0] + i] = i < rows ? tokens[i] : 0;
        hst[o[1] + i] = i < rows ? positions[i] : 0;
        hst[o[3] + i] = (need_feed && i < rows) ? feed[i] : -1;
    }
    for (int64_t i = 0; i <= B; ++i) hst[o[2] + i] = i;
    int32_t* sh = reinterpret_cast<int32_t*>(hst + o[4]);
    for (int64_t i = 0; i < B; ++i) sh[i] = (shared_blocks != nullptr && i < rows) ? shared_blocks[i] : 0;
    int64_t* tab = hst + o[5];
    const int64_t w = std::min(W, tables_width);
    for (int64_t i = 0; i < B; ++i) {
        int64_t* row = tab + i * W;
        std::fill(row, row + W, int64_t{-1});
        if (i < rows) std::memcpy(row, tables + i * tables_width, w * sizeof(int64_t));
        else row[0] = r->d.scratch_block;    // idle rows: one key of the scratch block
    }
    const int64_t n = o[5] + B * W;
    CVR_CHECK(hip_ok(hipMemcpyAsync(r->arena, hst, n * sizeof(int64_t), hipMemcpyHostToDevice, stream)));
    if (need_feed) CVR_CHECK(cvh_feed_tokens(r->tok(), r->feed(), prev_sampled, rows, stream));
    return CVH_OK;
}

extern "C" int cvh_runner_forward(cvh_runner* r, int batch, int shared, cvh_stream_t stream) {
    if (!live(r) || batch <= 0 || batch > r->d.max_batch) return CVH_ERR_INVALID_ARG;
    return r->forward(batch, shared != 0, stream);
}

extern "C" int cvh_runner_capture(cvh_runner* r, int batch, int shared) {
    if (!live(r) || batch <= 0 || batch > r->d.max_batch) return CVH_ERR_INVALID_ARG;
    hipStream_t s = r->capture_stream;
    // the runner's stream does not wait on the caller's: let a preceding stage (on any stream) land
    CVR_CHECK(hip_ok(hipDeviceSynchronize()));
    // one eager run first: kernels that opt in to large LDS set their attributes outside the capture
    CVR_CHECK(r->forward(batch, shared != 0, s));
    CVR_CHECK(hip_ok(hipStreamSynchronize(s)));
    CVR_CHECK(hip_ok(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal)));
    const int rc = r->forward(batch, shared != 0, s);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != CVH_OK || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        return rc != CVH_OK ? rc : CVH_ERR_LAUNCH;
    }
    hipGraphExec_t ex = nullptr;
    if (hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess) {
        (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        return CVH_ERR_LAUNCH;
    }
    auto key = std::make_pair(batch, shared != 0 ? 1 : 0);
    auto it = r->graphs.find(key);
    if (it != r->graphs.end()) {
        (void)hipGraphExecDestroy(it->second.second);
        (void)hipGraphDestroy(it->second.first);
    }
    r->graphs[key] = {g, ex};
    return CVH_OK;
}

extern "C" int cvh_runner_replay(cvh_runner* r, int batch, int shared, cvh_stream_t stream) {
    if (!live(r)) return CVH_ERR_INVALID_ARG;
    auto it = r->graphs.find(std::make_pair(batch, shared != 0 ? 1 : 0));
    if (it == r->graphs.end()) return CVH_ERR_INVALID_ARG;
    return hip_ok(hipGraphLaunch(it->second.second, stream));
}
