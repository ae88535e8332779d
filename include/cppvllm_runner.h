/*
 * cppvllm_runner.h — decode-step runner of a Qwen3-shaped model on the gfx950 kernels.
 *
 * Replaces the decode half of the reference's ModelRunner (engine/model_runner.cpp:169-212 launch /
 * collect, :327-357 graph-row staging, :371-428 CUDA-graph capture and replay) and the layer loop
 * of Qwen3::forward_backbone it replays (model/model_architecture.cpp:130-191): the step's rows are
 * staged from host arrays through pinned memory, and the 28-layer forward runs through the C ABI of
 * cppvllm_hip.h, eagerly or as a HIP graph captured and replayed with the HIP runtime. No libtorch
 * here: weights, the KV cache, the RoPE tables and the output rows are device pointers the caller
 * owns; the runner allocates its own inputs, activations, attention workspace, pinned staging and
 * graphs in cvh_runner_create (the only calls that allocate) and frees them in cvh_runner_destroy.
 *
 * The forward is the one of the reference with this library's kernels:
 *   token metadata (slots, kv_len) -> embedding -> per layer:
 *     rows < fused_min_rows or > fused_max_rows (reference rounding points):
 *       qkv = x W_qkv^T; QK-RMSNorm + RoPE + FP8 K/V write; planned paged attention;
 *       o = att W_o^T; add_rms_norm(h, o, ffn_norm) -> x; act = swiglu(x W_gu^T); m = act W_down^T;
 *       add_rms_norm(h, m, next norm) -> x
 *     rows in [fused_min_rows, fused_max_rows] (the projections' fused epilogues):
 *       QKV projection with the row RMS factor and QK-norm/RoPE/K/V write in its epilogue;
 *       planned attention; o_proj adds into h and leaves the row sums of squares; gate/up with the
 *       row RMS factor and SwiGLU; down adds into h; the final norm -> hidden.
 * Idle rows [rows, batch) attend over one key of the scratch block (kv_len 1) and write their K/V
 * there (engine/model_runner.cpp:346).
 * Return values are the CVH_* codes of cppvllm_hip.h.
 */
#ifndef CPPVLLM_RUNNER_H
#define CPPVLLM_RUNNER_H

#include "cppvllm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One decoder layer's device pointers (bf16 weights in torch's linear layout, [out][in]). */
typedef struct cvh_runner_layer {
    const void* w_qkv;            /* [(H + 2 KV) * HD][D] */
    const void* w_qkv_folded;     /* w_qkv with attn_norm's gain folded into its columns (fused path) */
    const void* w_o;              /* [D][H * HD] */
    const void* w_gate_up;        /* [2 I][D], gate / up rows interleaved in blocks of 16 */
    const void* w_gate_up_folded; /* w_gate_up with ffn_norm's gain folded in (fused path) */
    const void* w_down;           /* [D][I] */
    const void* attn_norm;        /* [D] */
    const void* ffn_norm;         /* [D] */
    const void* q_norm;           /* [HD] */
    const void* k_norm;           /* [HD] */
    uint8_t* k_cache;             /* this layer's paged cache (layout of cppvllm_hip.h) */
    uint8_t* v_cache;
    float* k_scale;
    float* v_scale;
} cvh_runner_layer;

typedef struct cvh_runner_desc {
    int n_layers, dim, n_heads, n_kv_heads, head_dim, intermediate;
    int64_t vocab;
    double norm_eps;              /* RMSNorm eps (config.h:19) */
    double attn_scale;            /* softmax scale, 1/sqrt(head_dim) */
    int block_size, scale_mode;   /* KV cache block size and CVH_SCALE_* */
    int max_batch;                /* largest decode batch (rows of a graph) */
    int64_t table_width;          /* block-table width of the staged rows */
    int64_t scratch_block;        /* physical block the idle rows of a batch use */
    int fused_min_rows, fused_max_rows;   /* fused-epilogue window; max < min: never fused */
    const void* embed;            /* [vocab][D] (tied lm_head) */
    const void* final_norm;       /* [D] */
    const void* unit_gain;        /* [D] of ones (the layer-0 input norm of the fused path) */
    const float* rope_cos;        /* [max_position][HD / 2] */
    const float* rope_sin;
    void* hidden;                 /* output: bf16 [max_batch][D], final-normed rows of the last step */
    const cvh_runner_layer* layers;   /* n_layers entries (copied by cvh_runner_create) */
} cvh_runner_desc;

typedef struct cvh_runner cvh_runner;

/* Allocate the runner for this model (inputs, activations, workspace, pinned staging). */
int cvh_runner_create(const cvh_runner_desc* desc, cvh_runner** out);
/* Free everything cvh_runner_create and cvh_runner_capture allocated. */
int cvh_runner_destroy(cvh_runner* r);
/* Stage `rows` decode rows padded to `batch` (rows <= batch <= max_batch) through pinned slot
 * `slot` (0 or 1: a slot is rewritten only after the step that used it has completed): host
 * tokens [rows], positions [rows], tables [rows][tables_width] (-1 padded; columns beyond the
 * runner's table_width are dropped; a position outside [0, table_width * block_size) is
 * rejected with CVH_ERR_INVALID_ARG), optional feed [rows] (>= 0: take the token from
 * prev_sampled[feed[i]], the device samples of the previous step; cvh_feed_tokens), optional
 * shared_blocks [rows] (leading blocks each row shares with other rows; used by shared forwards).
 * One host-to-device copy on `stream`. */
int cvh_runner_stage(cvh_runner* r, int slot, int64_t rows, int batch, const int64_t* tokens,
                     const int64_t* positions, const int64_t* tables, int64_t tables_width, const int64_t* feed,
                     const int32_t* shared_blocks, const int64_t* prev_sampled, cvh_stream_t stream);
/* The decode forward of the staged batch, launched eagerly on `stream`; writes desc.hidden. shared:
 * the attention plan marks each row's shared blocks (cvh_paged_attention_plan_shared). */
int cvh_runner_forward(cvh_runner* r, int batch, int shared, cvh_stream_t stream);
/* Capture the same forward into a HIP graph for (batch, shared) (replaces an earlier capture). It
 * first waits for all device work, then runs the forward once eagerly on the runner's own stream
 * (like cvh_runner_forward it writes the staged rows' K/V slots and desc.hidden): stage idle rows
 * (rows = 0, which point at the scratch block) before capturing. Not for use during serving. */
int cvh_runner_capture(cvh_runner* r, int batch, int shared);
/* Replay the captured graph of (batch, shared) on `stream`; CVH_ERR_INVALID_ARG if none. */
int cvh_runner_replay(cvh_runner* r, int batch, int shared, cvh_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* CPPVLLM_RUNNER_H */
