/*
 * cppvllm_hip.h — C ABI of the MI355X (gfx950) FP8 paged-decode hot path.
 *
 * Drop-in boundary for the kernel layer of cppvllm. Each entry point replaces one
 * at::Tensor-taking free function of the reference kernel layer; tensors become plain
 * device pointers plus the shapes the reference reads from tensor metadata, and the
 * current c10 stream becomes an explicit hipStream_t. No libtorch types cross this ABI.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers unless stated otherwise; the caller owns every buffer.
 *   - No entry point allocates device memory or synchronises the stream (capture-safe).
 *   - Return value: CVH_OK (0) or a CVH_ERR_* code. Nothing throws across this ABI.
 *   - num_tokens == 0 is a successful no-op (the reference returns early,
 *     kernels/paged_attention.cu:462, kernels/fused_ops.cu:227,237,252).
 *
 * KV-cache layout (one layer), identical to the reference (engine/model_runner.cpp:104-113):
 *   k_cache, v_cache : uint8 OCP e4m3fn, [num_blocks][block_size][n_kv_heads][head_dim]
 *   k_scale, v_scale : float32,
 *       CVH_SCALE_PER_TOKEN_HEAD: memory order [num_blocks][n_kv_heads][block_size]
 *                                 (kernels/fused_ops.cu:136,185; paged_attention.cu:224)
 *       CVH_SCALE_PER_TENSOR    : one float each (k_scale[0], v_scale[0]); read-only inputs.
 *   slot s addresses token (s / block_size, s % block_size) of the pool.
 */
#ifndef CPPVLLM_HIP_H
#define CPPVLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* cvh_stream_t; /* == hipStream_t; NULL = default stream */

enum {
    CVH_OK = 0,
    CVH_ERR_INVALID_ARG = 1,   /* null pointer where one is required, negative size, ... */
    CVH_ERR_UNSUPPORTED = 2,   /* head_dim / GQA ratio / block size / dtype not compiled */
    CVH_ERR_WORKSPACE = 3,     /* workspace missing or smaller than required */
    CVH_ERR_LAUNCH = 4         /* hipGetLastError() after a launch was not hipSuccess */
};

enum { CVH_SCALE_PER_TOKEN_HEAD = 0, CVH_SCALE_PER_TENSOR = 1 };
enum { CVH_DTYPE_BF16 = 0, CVH_DTYPE_F16 = 1, CVH_DTYPE_F32 = 2 };

/* ---------------------------------------------------------------------------------------------
 * Paged FP8 decode attention.
 * Replaces: void paged_attention_fp8(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
 *           const at::Tensor& v_cache, const at::Tensor& k_scale, const at::Tensor& v_scale,
 *           const at::Tensor& block_tables, const at::Tensor& token_seq,
 *           const at::Tensor& token_kv_len, double scale)      (kernels/paged_attention.h:5-7,
 *                                                                kernels/paged_attention.cu:459-473)
 *   out          bf16 [num_tokens][n_heads][head_dim]
 *   q            bf16 [num_tokens][n_heads][head_dim]
 *   block_tables int64 [num_seqs][table_width]; entries past a sequence's last block are ignored
 *   token_seq    int64 [num_tokens]  row of block_tables for each query token; a negative value
 *                                    marks a padding token, whose output row is all zero whatever
 *                                    its kv_len (the same rule in every attention entry point)
 *   token_kv_len int64 [num_tokens]  causal context length of each query token (positions+1);
 *                                    a token with kv_len <= 0 gets an all-zero output row
 *   scale        softmax scale (1/sqrt(head_dim) in the reference)
 * Supported: head_dim in {64,128}; n_heads/n_kv_heads in {1,2,4,8} (at head_dim 128, 4 and 8 run
 * on matrix cores with the query heads of a kv head as MFMA columns; at head_dim 64 they run as 2
 * and 4 virtual kv heads of 2 query heads per kv head, which halves / quarters the token limit
 * below); block_size a power of two in [16, 4096]; num_tokens <= 8192 for n_kv_heads <= 8
 * (num_tokens * n_kv_heads / 8 <= 8192 above): twice the reference engine's max_num_batched_tokens
 * (bench.cpp:25).
 * Queries of one sequence may be several tokens (chunked-prefill continuation).
 * workspace: device memory of at least cvh_paged_attention_workspace_bytes(...) bytes for the
 * same arguments (tile prefix and split partials). Its contents need no initialisation.
 * ------------------------------------------------------------------------------------------- */
int cvh_paged_attention_fp8(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                            const float* k_scale, const float* v_scale, const int64_t* block_tables,
                            int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                            int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim, int block_size,
                            int scale_mode, double scale, void* workspace, size_t workspace_bytes,
                            cvh_stream_t stream);

/* Same as cvh_paged_attention_fp8 with an explicit work partition count: the concatenated
 * 32-key tiles of all (token, kv-head group) rows are cut into `partitions` equal ranges, one
 * workgroup each; 0 = automatic (one per resident workgroup slot of an MI355X, at most 1024 and
 * at most 8 per row, fewer for small batches). Results agree to fp32 rounding for every partition count.
 * (No reference counterpart for the knob: the reference hard-codes a split heuristic,
 *  kernels/paged_attention.cu:403-409; tests use it to prove partition invariance.) */
int cvh_paged_attention_fp8_ex(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                               const float* k_scale, const float* v_scale, const int64_t* block_tables,
                               int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                               int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim, int block_size,
                               int scale_mode, double scale, int partitions, void* workspace,
                               size_t workspace_bytes, cvh_stream_t stream);

/* The two launches of cvh_paged_attention_fp8_ex, exposed separately (same arguments; run on one
 * stream, split phase first): the split phase runs the decode kernel, which finishes every
 * (token, head) whose keys one workgroup covered and writes (acc, max, sum) partials for the
 * others; the merge phase combines those partials. Callers use them to time the decode kernel
 * alone or to interleave other work between the phases.
 * (No reference counterpart: the reference launches both back to back,
 *  kernels/paged_attention.cu:423-441.) */
int cvh_paged_attention_fp8_split_phase(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                        const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                        int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                        int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                        int block_size, int scale_mode, double scale, int partitions,
                                        void* workspace, size_t workspace_bytes, cvh_stream_t stream);
int cvh_paged_attention_fp8_merge_phase(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                        const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                        int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                        int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                        int block_size, int scale_mode, double scale, int partitions,
                                        void* workspace, size_t workspace_bytes, cvh_stream_t stream);

/* Multi-token query rows on matrix cores: the same contract and result as cvh_paged_attention_fp8
 * (same arguments; no workspace), computed by a kernel that gives 16 consecutive query tokens one
 * K/V tile walk and runs the score and PV products on MFMA. Meant for chunked-prefill and prompt
 * rows (several consecutive tokens of one sequence), where it reads each K/V tile once per 16
 * tokens instead of once per token; any ragged batch is valid input (tokens of different
 * sequences in one 16-token tile are processed one sequence at a time).
 * Supported: head_dim 128; n_heads/n_kv_heads in {1, 2}; block_size a power of two in [16, 4096];
 * else CVH_ERR_UNSUPPORTED (use cvh_paged_attention_fp8).
 * Replaces the chunked-prefill route of paged_attention_fp8 (kernels/paged_attention.cu:459-473
 * with T > S; model/model_architecture.cpp:143-147,175-176). */
int cvh_paged_attention_fp8_prefill(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                    const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                    int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                    int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                    int scale_mode, double scale, cvh_stream_t stream);

/* Planned multi-query launches. The key walk of a 64-token group grows with its position in its
 * prompt, so in natural order the longest groups of the last prompts start late and end the
 * launch. cvh_paged_attention_prefill_plan sorts the groups by their largest (clamped)
 * token_kv_len, longest first, into the workspace (one 1024-thread workgroup; build it once per
 * step, stream-ordered before the planned calls, and again when token_seq, token_kv_len or
 * num_tokens change); cvh_paged_attention_fp8_prefill_planned dispatches (group, kv head) items in
 * that order, each on 8 waves that split the group's key tiles in two halves and combine their
 * softmax states in LDS. Same arguments and results as cvh_paged_attention_fp8_prefill (within the
 * attention tolerance: the two halves change the fp32 summation order); workspace_bytes >=
 * cvh_paged_attention_prefill_workspace_bytes(num_tokens), else CVH_ERR_WORKSPACE. */
size_t cvh_paged_attention_prefill_workspace_bytes(int64_t num_tokens);
int cvh_paged_attention_prefill_plan(const int64_t* token_seq, const int64_t* token_kv_len, int64_t num_tokens,
                                     int64_t table_width, int block_size, void* workspace, size_t workspace_bytes,
                                     cvh_stream_t stream);
int cvh_paged_attention_fp8_prefill_planned(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                            const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                            int64_t table_width, const int64_t* token_seq,
                                            const int64_t* token_kv_len, int64_t num_tokens, int n_heads,
                                            int n_kv_heads, int head_dim, int block_size, int scale_mode, double scale,
                                            const void* workspace, size_t workspace_bytes, cvh_stream_t stream);

/* Planned launches. A decode step runs the same attention layout (block tables, token_seq,
 * token_kv_len, partition count) once per layer; cvh_paged_attention_plan builds, once, what
 * every decode workgroup would otherwise derive at the start of each launch (row prefix, token
 * metadata, its first tiles' physical blocks) into the workspace, and the _planned calls read it,
 * so each layer's first K/V loads go out one memory round trip after launch instead of three.
 * Contract: the plan describes the arguments it was built from; rebuild it (stream-ordered before
 * the planned calls) whenever block_tables contents, token_seq, token_kv_len, num_tokens or
 * partitions change. Output equals cvh_paged_attention_fp8_ex bit for bit.
 * (No reference counterpart: the reference re-derives per call; its per-step metadata is built in
 *  model/model_architecture.cpp:137-147, where an engine would call the plan.) */
int cvh_paged_attention_plan(const int64_t* block_tables, int64_t table_width, const int64_t* token_seq,
                             const int64_t* token_kv_len, int64_t num_tokens, int n_heads, int n_kv_heads,
                             int head_dim, int block_size, int partitions, void* workspace, size_t workspace_bytes,
                             cvh_stream_t stream);
/* cvh_paged_attention_plan with prefix-cache sharing: shared_blocks[r] (int32, one per
 * block-table row) is how many leading blocks of row r are also referenced by other rows (the block
 * manager's reference counts). Query tokens whose rows start with the same physical blocks (same
 * first block, same shared key count s = min(kv_len, shared_blocks * block_size), same first
 * ceil(s / block_size) table entries) form a group; a group of two or more is split in token order
 * into units of up to 16 / (query heads per kv head) tokens. The _planned_shared launches (same
 * arguments as _planned) then read each unit's shared K/V once for all its tokens (one matrix-core
 * pass: the unit's tokens x their query heads of one kv head as 16 MFMA columns) and each token's
 * own tiles from key s on, and the merge combines the two per token. Units run at head_dim 128
 * (GQA 1, 2, 4, 8: units of 16, 8, 4, 2 tokens), at most 8 kv heads and at most 2048 query tokens; other launches, and tokens in no group, run as the plain plan. Results equal the plain
 * launches within the attention tolerance (another summation order), and are bitwise reproducible.
 * Workspace: cvh_paged_attention_workspace_bytes_shared bytes (the plan, the _shared launches and
 * their merge phase use the same layout).
 * (Prefix-shared block reuse; no reference counterpart: the reference re-reads shared blocks
 *  per sequence, engine/block_manager.cpp:80-116 hands out the shared ids.) */
int cvh_paged_attention_plan_shared(const int64_t* block_tables, int64_t table_width, const int64_t* token_seq,
                                    const int64_t* token_kv_len, const int32_t* shared_blocks, int64_t num_tokens,
                                    int n_heads, int n_kv_heads, int head_dim, int block_size, int partitions,
                                    void* workspace, size_t workspace_bytes, cvh_stream_t stream);
int cvh_paged_attention_fp8_planned_shared(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                           const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                           int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                           int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                           int block_size, int scale_mode, double scale, int partitions,
                                           void* workspace, size_t workspace_bytes, cvh_stream_t stream);
int cvh_paged_attention_fp8_planned_shared_split_phase(void* out, const void* q, const uint8_t* k_cache,
                                                       const uint8_t* v_cache, const float* k_scale,
                                                       const float* v_scale, const int64_t* block_tables,
                                                       int64_t table_width, const int64_t* token_seq,
                                                       const int64_t* token_kv_len, int64_t num_tokens, int n_heads,
                                                       int n_kv_heads, int head_dim, int block_size, int scale_mode,
                                                       double scale, int partitions, void* workspace,
                                                       size_t workspace_bytes, cvh_stream_t stream);
/* Merge phase of a _planned_shared_split_phase launch (the cut rows and every unit member). */
int cvh_paged_attention_fp8_planned_shared_merge_phase(void* out, const void* q, const uint8_t* k_cache,
                                                       const uint8_t* v_cache, const float* k_scale,
                                                       const float* v_scale, const int64_t* block_tables,
                                                       int64_t table_width, const int64_t* token_seq,
                                                       const int64_t* token_kv_len, int64_t num_tokens, int n_heads,
                                                       int n_kv_heads, int head_dim, int block_size, int scale_mode,
                                                       double scale, int partitions, void* workspace,
                                                       size_t workspace_bytes, cvh_stream_t stream);
int cvh_paged_attention_fp8_planned(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                    const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                    int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                    int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                    int scale_mode, double scale, int partitions, void* workspace,
                                    size_t workspace_bytes, cvh_stream_t stream);
int cvh_paged_attention_fp8_planned_split_phase(void* out, const void* q, const uint8_t* k_cache,
                                                const uint8_t* v_cache, const float* k_scale, const float* v_scale,
                                                const int64_t* block_tables, int64_t table_width,
                                                const int64_t* token_seq, const int64_t* token_kv_len,
                                                int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                                int block_size, int scale_mode, double scale, int partitions,
                                                void* workspace, size_t workspace_bytes, cvh_stream_t stream);

/* cvh_paged_attention_fp8_ex without a workspace argument: the split workspace is a fixed 24 MiB
 * device array inside the library (one per GPU, held until the process ends), so the call allocates
 * nothing and needs no caller buffer. No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Every launch with automatic partitions (partitions = 0) fits; a partition count whose
 * workspace (cvh_paged_attention_workspace_bytes) exceeds cvh_paged_attention_noalloc_max_workspace()
 * returns CVH_ERR_WORKSPACE before anything runs. Results equal cvh_paged_attention_fp8_ex bit for
 * bit. All calls on one GPU share the array and leave their data in it (nothing in it needs to start
 * at zero): calls that overlap on one GPU (two streams or two host threads) race. */
int cvh_paged_attention_fp8_noalloc(void* out, const void* q, const uint8_t* k_cache, const uint8_t* v_cache,
                                    const float* k_scale, const float* v_scale, const int64_t* block_tables,
                                    int64_t table_width, const int64_t* token_seq, const int64_t* token_kv_len,
                                    int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                    int scale_mode, double scale, int partitions, cvh_stream_t stream);
/* Bytes of that fixed array (the largest workspace cvh_paged_attention_fp8_noalloc accepts). */
size_t cvh_paged_attention_noalloc_max_workspace(void);

/* Workspace bytes needed by the calls above (replaces the per-call at::empty of
 * kernels/paged_attention.cu:415-421, which cannot run under graph capture). */
size_t cvh_paged_attention_workspace_bytes(int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                           int64_t table_width, int block_size, int partitions);

/* Workspace bytes of the prefix-sharing plan and launches (cvh_paged_attention_plan_shared). */
size_t cvh_paged_attention_workspace_bytes_shared(int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                                  int64_t table_width, int block_size, int partitions);

/* The partition count the automatic policy picks for these shapes (the same count the launches
 * and cvh_paged_attention_workspace_bytes use for partitions = 0). */
int cvh_paged_attention_partitions(int64_t num_tokens, int n_heads, int n_kv_heads, int head_dim,
                                   int64_t table_width, int block_size);

/* ---------------------------------------------------------------------------------------------
 * RMSNorm family. Replaces fused::rms_norm / fused::add_rms_norm (kernels/fused_ops.h:7-9,
 * kernels/fused_ops.cu:61-98,226-244). Rows are num_rows x dim, contiguous, of `dtype`.
 *   rms_norm    : out = rnd(rnd(x * inv) * w),  inv = 1/sqrt(sum(x^2)/dim + eps)
 *   add_rms_norm: v = rnd(resid + x); resid <- v (in place); out as above from v
 * dim must be a multiple of 8.
 * ------------------------------------------------------------------------------------------- */
int cvh_rms_norm(void* out, const void* x, const void* w, int64_t num_rows, int dim, double eps, int dtype,
                 cvh_stream_t stream);
int cvh_add_rms_norm(void* resid, const void* x, const void* w, void* out, int64_t num_rows, int dim, double eps,
                     int dtype, cvh_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Per-head QK-RMSNorm + neox RoPE + FP8 e4m3 quantise-and-scatter of K/V into the paged cache.
 * Replaces fused::qk_norm_rope_kv_write_fp8 (kernels/fused_ops.h:11-15, fused_ops.cu:104-207,246-259).
 *   q_out     bf16 [num_tokens][n_heads][head_dim]
 *   qkv       bf16 [num_tokens][(n_heads + 2*n_kv_heads) * head_dim]  (Q heads, then K, then V)
 *   q_norm, k_norm  bf16 [head_dim]
 *   cos_t, sin_t    float32 [max_position][head_dim/2]
 *   positions int64 [num_tokens]
 *   slots     int64 [num_tokens]; slots[t] < 0 => no K/V byte and no scale is written for t
 *             (extension: the reference writes unconditionally, kernels/fused_ops.cu:123)
 *   k_dense, v_dense  bf16 [num_tokens][n_kv_heads][head_dim] or NULL (reference's optional
 *             dense copies for the prefill path, kernels/fused_ops.cu:137-141,186-190)
 *   CVH_SCALE_PER_TOKEN_HEAD: scale = max(amax,1e-8)/448 per (token, kv head), written to
 *             k_scale/v_scale; CVH_SCALE_PER_TENSOR: k_scale[0]/v_scale[0] are read, not written.
 * head_dim in {64,128}; block_size a power of two in [16, 4096].
 * ------------------------------------------------------------------------------------------- */
int cvh_qk_norm_rope_kv_write_fp8(void* q_out, const void* qkv, const void* q_norm, const void* k_norm,
                                  const float* cos_t, const float* sin_t, const int64_t* positions,
                                  const int64_t* slots, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                                  float* v_scale, void* k_dense, void* v_dense, int64_t num_tokens, int n_heads,
                                  int n_kv_heads, int head_dim, int block_size, int scale_mode, double eps,
                                  cvh_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Per-token metadata of a ragged batch. Replaces the torch ops of Qwen3::forward_backbone
 * (model/model_architecture.cpp:137-147):
 *   token_seq[t] = #{ j in 1..num_seqs : cu_seqlens[j] <= t }   (searchsorted right)
 *   slot[t]      = block_tables[seq][pos/BS]*BS + pos%BS,  pos = positions[t]
 *   kv_len[t]    = pos + 1
 * Tokens past cu_seqlens[num_seqs] (padding) and tokens whose table entry is negative get
 * token_seq = -1, slot = -1, kv_len = 0. Any output pointer may be NULL.
 * ------------------------------------------------------------------------------------------- */
int cvh_build_token_metadata(const int64_t* cu_seqlens, int64_t num_seqs, const int64_t* positions,
                             int64_t num_tokens, const int64_t* block_tables, int64_t table_width,
                             int block_size, int64_t* token_seq, int64_t* slots, int64_t* token_kv_len,
                             cvh_stream_t stream);

/* Host-side RoPE tables (host pointers): inv_freq_i = 1/theta^(2i/head_dim) and
 * angle = pos*inv_freq in double, cos/sin in double, stored as float32 [max_position][head_dim/2].
 * Replaces Qwen3::build_rope_tables (model/model_architecture.cpp:67-75). */
int cvh_rope_tables_host(float* cos_t, float* sin_t, int64_t max_position, int head_dim, double theta);

/* OCP e4m3fn quantiser (round to nearest even, saturate to +-448, NaN -> 0x7F) of n floats:
 * dst[i] = e4m3(src[i] * inv_scale). The same encoder the cache writer uses
 * (reference: __nv_cvt_float_to_fp8(x, __NV_SATFINITE, __NV_E4M3), kernels/fused_ops.cu:42-44). */
int cvh_fp8_e4m3_quantize(uint8_t* dst, const float* src, int64_t n, float inv_scale, cvh_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Model ops around the attention path (used by the serving loop; not part of the decode kernel).
 * ------------------------------------------------------------------------------------------- */

/* SwiGLU: gate_up [num_rows][2*intermediate] (gate half first), out [num_rows][intermediate]:
 *   silu = round(g / (1 + exp(-g))) (exp evaluated in double), out = round(silu * u).
 * Replaces: void fused::swiglu(at::Tensor& out, const at::Tensor& gate_up)
 *           (kernels/fused_ops.h:17, kernels/fused_ops.cu:209-220,261-283). dtype: CVH_DTYPE_*. */
int cvh_swiglu(void* out, const void* gate_up, int64_t num_rows, int intermediate, int dtype, cvh_stream_t stream);

/* Token sampler: out[r] = arg-max over the vocab of row rows[r] of logits (rows == NULL: row r).
 * temps[r] <= 0 (or temps == NULL): greedy, lowest index wins ties. temps[r] > 0: Gumbel-max,
 * score = x/temp - log(-log(u)), u from Philox-4x32-10 keyed by seed with counter
 * (index/4, r, offset lo, offset hi). logits_dtype: CVH_DTYPE_F32 or CVH_DTYPE_BF16 (same values
 * as the reference's float copy of bf16 logits).
 * Replaces: void fused::sample_tokens(at::Tensor& out, const at::Tensor& logits, const at::Tensor& rows,
 *           const at::Tensor& temps, uint64_t seed, uint64_t offset)
 *           (kernels/fused_ops.h:19-20, kernels/fused_ops.cu:285-378). */
int cvh_sample_tokens(int64_t* out, const void* logits, int logits_dtype, const int64_t* rows, const float* temps,
                      int64_t num_rows, int vocab, uint64_t seed, uint64_t offset, cvh_stream_t stream);

/* Token feedback: tokens[i] = prev[src[i]] where src[i] >= 0.
 * Replaces: void fused::feed_tokens(at::Tensor& tokens, const at::Tensor& src, const at::Tensor& prev)
 *           (kernels/fused_ops.h:22, kernels/fused_ops.cu:379-397). */
int cvh_feed_tokens(int64_t* tokens, const int64_t* src, const int64_t* prev, int64_t n, cvh_stream_t stream);

/* Embedding gather of 16-bit rows: out[t] = table[ids[t]] ([num_tokens][dim], dim % 8 == 0);
 * ids outside [0, vocab) give a zero row. Replaces embed_.index_select(0, tokens)
 * (model/model_architecture.cpp:149). */
int cvh_embedding(void* out, const void* table, const int64_t* ids, int64_t num_tokens, int dim, int64_t vocab,
                  cvh_stream_t stream);

/* bf16 GEMM for decode-step projections: y[M][N] = bf16(x[M][K] . w[N][K]^T), fp32 accumulation,
 * round to nearest even (torch's linear layout: weight rows are output columns).
 * Replaces: at::linear(x, W) of the layer loop and the lm_head
 *           (model/model_architecture.cpp:155,178,182,185,224), which the reference runs on cuBLAS.
 * Requires N % 16 == 0 and K % 128 == 0. config: 0 = automatic (measured best per shape and row
 * count), otherwise one of the codes cvh_gemm_bf16_nt_configs lists; a code whose tile does not
 * divide N, or whose K split does not divide K, returns CVH_ERR_UNSUPPORTED. Codes:
 *   100*xlds + 10*mf + nwn                    streaming kernel (mf row fragments of 16 per wave,
 *                                             nwn waves across N, K split over 4/nwn waves)
 *   10000 + 100*nc + 10*mf + nwn              one-shot kernel (exactly nc 128-k chunks per wave)
 *   100000*st + 20000 + 1000*mf + 100*nf + 10*wm + nwn
 *                                             tiled kernel (mf x nf fragments per wave, wm x nwn
 *                                             waves, st LDS stages, 9 = as many as fit)
 * The sum order depends on the configuration only, so a given configuration is deterministic. */
int cvh_gemm_bf16_nt(void* y, const void* x, const void* w, int64_t M, int N, int K, int config,
                     cvh_stream_t stream);
/* The configuration cvh_gemm_bf16_nt picks for config == 0. */
int cvh_gemm_bf16_nt_config(int64_t M, int N, int K);
/* Codes of every compiled configuration: writes min(count, capacity) into codes (may be NULL)
 * and returns the count. */
int cvh_gemm_bf16_nt_configs(int* codes, int capacity);

/* Gate/up projection with the SwiGLU epilogue: act[M][I] = swiglu(x[M][K] . w[2I][K]^T), where w's
 * rows are the gate and up weight rows interleaved in blocks of 16 (rows 32b..32b+15 = gate rows
 * 16b..16b+15, rows 32b+16..32b+31 = up rows 16b..16b+15). Each product is rounded to bf16 and the
 * SwiGLU is cvh_swiglu's arithmetic, so act equals cvh_gemm_bf16_nt with the same config on the
 * same interleaved w, de-interleaved, followed by cvh_swiglu, bit for bit.
 * Replaces: at::linear(x, L.w_gate_up) + fused::swiglu(act, gu)
 *           (model/model_architecture.cpp:182-184, kernels/fused_ops.cu:209-220).
 * Requires I % 16 == 0, K % 128 == 0. config: 0 = automatic, otherwise a tiled code listed by
 * cvh_gemm_bf16_nt_swiglu_configs. */
int cvh_gemm_bf16_nt_swiglu(void* act, const void* x, const void* w, int64_t M, int I, int K, int config,
                            cvh_stream_t stream);
/* The configuration cvh_gemm_bf16_nt_swiglu picks for config == 0. */
int cvh_gemm_bf16_nt_swiglu_config(int64_t M, int I, int K);
/* Codes of the compiled SwiGLU-epilogue configurations (as cvh_gemm_bf16_nt_configs). */
int cvh_gemm_bf16_nt_swiglu_configs(int* codes, int capacity);

/* ---- Projections with the layer boundary fused into their epilogues (decode steps) ----------
 * The reference runs the projection, then a separate norm or QK-norm launch
 * (model/model_architecture.cpp:155-188, kernels/fused_ops.cu:61-207). These entry points do both
 * in one kernel; all take tiled configuration codes (as cvh_gemm_bf16_nt) listed by
 * cvh_gemm_fused_configs(kind), kind 0 = residual, 1 = SwiGLU-rownorm, 2 = QKV; config 0 picks the
 * measured best for the row count (cvh_gemm_fused_config).
 *
 * Residual epilogue (o_proj, down_proj): resid[M][N] <- bf16(resid + bf16(x . w^T)), the residual
 * add of cvh_add_rms_norm bit for bit, and row_ss[M][N/16] <- for each 16 columns n..n+15 of the new
 * residual v, the sum of v^2 as lanes holding columns 4j..4j+3 sum their four in order and the four
 * lane sums combine as (s0 + s1) + (s2 + s3). The row's norm sum is the in-order sum of its N/16
 * partials. Requires N % 32 == 0 (the tile width), K % 128 == 0. */
int cvh_gemm_bf16_nt_residual(void* resid, float* row_ss, const void* x, const void* w, int64_t M, int N, int K,
                              int config, cvh_stream_t stream);
/* Row-normed gate/up with the SwiGLU epilogue: x is the raw residual (the rows
 * cvh_gemm_bf16_nt_residual wrote), inv[m] = 1 / sqrt(sum(row_ss[m][0..K/16)) / K + eps) with the
 * sum taken as each of 4 lanes summing K/64 consecutive partials in order, then (q0 + q1) + (q2 + q3);
 * the accumulator is multiplied by inv before cvh_gemm_bf16_nt_swiglu's epilogue. w is the
 * interleaved gate/up weight with the RMSNorm gain multiplied into its columns and rounded to bf16,
 * so the result stands for swiglu(bf16(bf16(x * inv) * gain) . w^T) up to those roundings.
 * Requires K % 256 == 0 and K <= 1024. */
int cvh_gemm_bf16_nt_swiglu_rownorm(void* act, const void* x, const float* row_ss, double eps, const void* w,
                                    int64_t M, int I, int K, int config, cvh_stream_t stream);
/* QKV projection with cvh_qk_norm_rope_kv_write_fp8 in its epilogue: the bf16 tile of
 * qkv = x . w_qkv^T ([T][(H + 2KV) * 128]) is kept on chip and each (token, head) of it runs the
 * standalone kernel's task, so q_out and the cache bytes equal cvh_gemm_bf16_nt (same tiled config)
 * followed by cvh_qk_norm_rope_kv_write_fp8, bit for bit, when row_ss is NULL. With row_ss, x is the
 * raw residual and the accumulator is first multiplied by the row's RMSNorm factor (as
 * cvh_gemm_bf16_nt_swiglu_rownorm; x_eps is that norm's eps, w_qkv carries its gain). No dense K/V
 * copies. Requires head_dim == 128, dim % 128 == 0 (with row_ss: dim % 256 == 0, dim <= 1024). */
int cvh_gemm_qkv_norm_rope_kv_write_fp8(void* q_out, const void* x, const float* row_ss, double x_eps,
                                        const void* w_qkv, const void* q_norm, const void* k_norm, const float* cos_t,
                                        const float* sin_t, const int64_t* positions, const int64_t* slots,
                                        uint8_t* k_cache, uint8_t* v_cache, float* k_scale, float* v_scale,
                                        int64_t num_tokens, int dim, int n_heads, int n_kv_heads, int head_dim,
                                        int block_size, int scale_mode, double eps, int config, cvh_stream_t stream);
/* Codes of the compiled configurations of a fused kind (as cvh_gemm_bf16_nt_configs); returns the count. */
int cvh_gemm_fused_configs(int kind, int* codes, int capacity);
/* The configuration a fused kind picks for M rows with config == 0. */
int cvh_gemm_fused_config(int kind, int64_t M);

/* Library version string (static storage). */
const char* cvh_version(void);

#ifdef __cplusplus
}
#endif
#endif /* CPPVLLM_HIP_H */
