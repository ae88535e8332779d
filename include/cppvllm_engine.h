/* cppvllm_engine.h — host-side serving core (sequences, paged block manager with prefix
 * caching, continuous-batching scheduler with chunked prefill) behind a C ABI.
 *
 * This is the caller side of the attention path: it produces, every step, the ragged batch the
 * kernels of cppvllm_hip.h consume (token ids, positions, cu_seqlens, block tables, causal kv
 * lengths) and consumes the sampled token of every sequence that samples. It replaces
 * engine/sequence.h, engine/block_manager.{h,cpp} and engine/scheduler.{h,cpp} of the reference
 * (and the step bookkeeping of engine/llm_engine.cpp), without libtorch: plain C++17, no GPU.
 *
 * Conventions: every function returns CVE_OK (0) or a negative CVE_ERR_* code unless stated;
 * nothing throws across the ABI. An engine handle is used by one thread at a time.
 */
#ifndef CPPVLLM_ENGINE_H
#define CPPVLLM_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    CVE_OK = 0,
    CVE_ERR_INVALID_ARG = -1,
    CVE_ERR_TOO_LONG = -2,        /* a request needs more KV blocks than the cache has */
    CVE_ERR_STATE = -3,           /* call out of order (e.g. postprocess without a batch) */
    CVE_ERR_EMPTY = -4,           /* requests pending but nothing could be scheduled */
    CVE_ERR_BUSY = -5             /* nothing can be scheduled until the oldest step is post-processed */
};

/* Step groups, in the order they appear in a batch (model_runner.cpp:178-196 of the reference):
 * decode rows (one new token on a cached context, graph-eligible), fresh prefills (no cached
 * tokens, several new tokens), and the rest (continuations of chunked or prefix-cached prompts). */
enum { CVE_GROUP_DECODE = 0, CVE_GROUP_FRESH = 1, CVE_GROUP_CONT = 2, CVE_NUM_GROUPS = 3 };

typedef struct cve_config {
    int64_t max_num_batched_tokens; /* token budget per step (config.h:63: 4096) */
    int64_t max_num_seqs;           /* sequences per step (config.h:64: 256) */
    int64_t max_chunk_tokens;       /* prefill chunk cap per sequence, 0 = none (config.h:65: 1024) */
    int32_t block_size;             /* tokens per KV block (sequence.h:28: 16) */
    int32_t num_blocks;             /* KV blocks in the cache */
    int32_t graph_max_blocks;       /* decode rows whose table exceeds this go to CVE_GROUP_CONT */
    int32_t eos_token_id;           /* -1 = none */
} cve_config;

/* A scheduled step, in engine-owned memory valid until the next cve_schedule. Sequences are
 * ordered by group; group g holds sequences [group_start[g], group_start[g+1]). Row j of the
 * flat batch: tokens/positions [cu_seqlens[j], cu_seqlens[j+1]), kv_lens[j] = cached + new
 * tokens, block table row j (table_width entries, -1 padded), samples[j] = 1 when the step
 * produces the sequence's next token (its last scheduled token is the last of its context).
 * feed_src[t] >= 0 marks a token that the previous step (still unprocessed) is sampling:
 * tokens[t] is -1 and the runner must copy row feed_src[t] of that step's sampled tokens into it
 * on the device (kernels/fused_ops.cu:379-397, cvh_feed_tokens). */
typedef struct cve_batch {
    int64_t num_seqs, num_tokens, table_width;
    int64_t group_start[CVE_NUM_GROUPS + 1];
    const int64_t* tokens;
    const int64_t* positions;
    const int64_t* cu_seqlens;      /* [num_seqs + 1] */
    const int64_t* kv_lens;         /* [num_seqs] */
    const int64_t* block_tables;    /* [num_seqs][table_width] */
    const int8_t* samples;          /* [num_seqs] */
    const int64_t* seq_ids;         /* [num_seqs] request id of each row */
    const int64_t* feed_src;        /* [num_tokens] row of the previous step's sampled tokens, or -1 */
    const int32_t* shared_blocks;   /* [num_seqs] leading table blocks other live sequences also reference
                                       (cvh_paged_attention_plan_shared) */
} cve_batch;

typedef struct cve_stats {
    int64_t steps, tokens_scheduled, tokens_sampled, preemptions, finished;
    int64_t free_blocks, prefix_hit_tokens;
} cve_stats;

void* cve_create(const cve_config* cfg);
void cve_destroy(void* engine);

/* Queue a request (scheduler.cpp:17-27): returns its id (>= 0) or CVE_ERR_TOO_LONG /
 * CVE_ERR_INVALID_ARG. max_tokens = output tokens to generate; ignore_eos as in sequence.h:23. */
int64_t cve_add_request(void* engine, const int32_t* prompt, int64_t prompt_len, int32_t max_tokens,
                        int32_t ignore_eos);

/* Build the next step (scheduler.cpp:37-103 + on_launched :105-119). Up to two steps may be
 * outstanding (scheduled, not yet post-processed; the reference's launch ring, llm_engine.h:51):
 * a step built while another is outstanding never preempts and reads that step's samples through
 * feed_src. CVE_OK with out->num_seqs == 0 when nothing is pending; CVE_ERR_EMPTY if requests wait
 * but none fits; CVE_ERR_BUSY if nothing can run until the oldest step is post-processed;
 * CVE_ERR_STATE if two steps are already outstanding. */
int cve_schedule(void* engine, cve_batch* out);

/* Accept the sampled tokens of the OLDEST outstanding step, one per row in its batch order (rows
 * with samples[j] == 0 are ignored) (scheduler.cpp:121-154). A sequence that finished in an
 * older step ignores its row; its blocks are freed once no outstanding step contains it. */
int cve_postprocess(void* engine, const int64_t* sampled, int64_t num_seqs);

int cve_is_finished(void* engine);        /* 1 when no request is waiting or running and no step is outstanding */
int64_t cve_num_outstanding(void* engine); /* scheduled steps not yet post-processed (0..2) */
int cve_get_stats(void* engine, cve_stats* out);

/* Finished requests: cve_num_finished() of them, in request-id order; cve_finished_output copies
 * request i's generated tokens (up to cap) and returns their count (-1 if i is out of range).
 * cve_clear_finished forgets them. */
int64_t cve_num_finished(void* engine);
int64_t cve_finished_output(void* engine, int64_t i, int64_t* request_id, int32_t* tokens, int64_t cap);
void cve_clear_finished(void* engine);

/* Block-manager probes for tests: reference count of a block, and a request's block table
 * (copied up to cap entries; returns its length or -1 if the request is not live). */
int32_t cve_block_ref_count(void* engine, int32_t block_id);
int64_t cve_block_table(void* engine, int64_t request_id, int32_t* out, int64_t cap);

#ifdef __cplusplus
}
#endif
#endif /* CPPVLLM_ENGINE_H */
