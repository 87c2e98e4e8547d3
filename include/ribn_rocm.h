/*
 * librocm_ribn -- MI355X (gfx950) backend for ribn's autoregressive token loop.
 *
 * C ABI. Plain pointers and sizes only; every array argument is caller-owned
 * host memory that the library never retains past the call (the reference's
 * rule for borrowed batches, crates/runtime/src/executor.rs:213-215), unless
 * a function says "device pointer".
 *
 * Status codes: RIBN_OK (0); RIBN_PENDING (1, poll only); negative = error.
 * Every function that can fail takes (char *err, size_t err_len) and writes a
 * NUL-terminated diagnostic of at most min(err_len, 4096) bytes
 * (ExecutionError, executor.rs:134-152).
 *
 * Threading: one handle is used by one thread at a time (the reference trait
 * is Send, not Sync; every method takes &mut self, executor.rs:171).
 */
#ifndef RIBN_ROCM_H
#define RIBN_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RIBN_OK 0
#define RIBN_PENDING 1
#define RIBN_ERR_INVALID (-1)     /* bad argument / contract violation */
#define RIBN_ERR_IO (-2)          /* file access */
#define RIBN_ERR_FORMAT (-3)      /* GGUF parse / unsupported model */
#define RIBN_ERR_DEVICE (-4)      /* HIP failure (the handle is faulted) */
#define RIBN_ERR_FAULTED (-5)     /* handle faulted by an earlier error */
#define RIBN_ERR_BUSY (-6)        /* a preparation or submission is outstanding */
#define RIBN_ERR_CAPACITY (-7)    /* exceeds prepared limits */

/* GGML value types accepted by the kernels (crates/gguf/src/lib.rs:508-535). */
#define RIBN_GGML_F32 0
#define RIBN_GGML_F16 1
#define RIBN_GGML_Q8_0 8
#define RIBN_GGML_Q4_K 12
#define RIBN_GGML_Q6_K 14

typedef struct ribn_rocm_model ribn_rocm_model;

/* ------------------------------------------------------------------------ */
/* Loading. Replaces QwenCuda::load_gguf (crates/qwen/src/cuda.rs:30) and
 * loading::load (crates/qwen/src/loading.rs:93-190) with QwenLoadOptions
 * (loading.rs:30-81). Accepts dense general.architecture qwen2 / qwen3 with
 * Q8_0 / Q4_K / Q6_K matrices and F32 norms/biases. Unsupported architecture
 * or value types are rejected with a message naming the field
 * (the shape-generic counterpart of QwenCudaProfile::mismatch, profile.rs:70-142). */
typedef struct {
    uint32_t context_tokens;   /* per-sequence limit (0 -> min(GGUF context_length, 4096)) */
    uint32_t max_sequences;    /* 0 -> 8 */
    uint32_t max_batch_tokens; /* 0 -> 2048 */
    uint32_t kv_pages;         /* 16-token KV pages in the pool (0 -> max_sequences*context/16) */
    int32_t device;            /* HIP device ordinal */
    uint32_t flags;            /* RIBN_LOAD_* bits */
} ribn_rocm_load_options;
/* KV cache in bfloat16 instead of the default binary16 (binary16 is the reference
 * CUDA cache type, kv_append_f16 nvidia/src/model_ops.rs:1258-1276). */
#define RIBN_LOAD_KV_BF16 1u
/* Run each token step as one persistent kernel launch (grid barriers between the
 * stages) when one is compiled for the model's configuration, instead of the
 * default chain of per-stage launches replayed as HIP graphs. Measured slower
 * than the default; kept as an opt-in. Every grid-barrier wait is bounded (2 s):
 * a wait that runs out makes every kernel exit, the call returns RIBN_ERR_DEVICE
 * and the handle is faulted (every later call returns RIBN_ERR_FAULTED), as a
 * device error faults QwenExecution (qwen/src/execution.rs:305-316). The caller
 * frees the handle and loads the model again. */
#define RIBN_LOAD_PERSISTENT_STEP 2u
/* Keep a binary16 copy of every layer matrix and of the output head, dequantized
 * once at load (exactly, then rounded to binary16), and run chunked prefill and
 * batched decode as plain hipBLASLt GEMMs on it instead of the dequantizing MFMA
 * GEMM. Costs 2 bytes per weight of extra HBM (16.4 GB for an 8B model); the
 * batch-1 decode matvecs keep streaming the GGUF planes. libhipblaslt.so is
 * opened at load only when this flag is set (RIBN_ERR_DEVICE if it cannot be). */
#define RIBN_LOAD_RESIDENT_F16 4u
/* Integer-dot decode projections, the reference's experimental, lossy
 * GemvMode::IntegerDot (nvidia/src/decode.rs:298-312, CudaIntDotProjector
 * decode.rs:1409-1553): every sampled decode row (batched rows of several
 * sequences and single steps alike) packs each projection input to Q8_1
 * (quantize_q8_1, nvidia/src/activation.cu) and runs the integer-dot matvec
 * (q4_k_q8_1.cu, q6_k_q8_1.cu, q8_0_q8_1.cu; weights read once for up to 8 rows).
 * Prompt rows keep the float path. Not token-identical to the default mode. Not
 * with RIBN_LOAD_PERSISTENT_STEP or qwen35 hybrids; ribn_rocm_trace and
 * ribn_rocm_prefill_trace refuse such a model. */
#define RIBN_LOAD_INT_DOT 8u
/* Let the dequantizing GEMMs (chunked prefill, batched decode rows) read the
 * weights from the decode planes instead of the default GEMM-ordered copy of
 * every Q4_K / Q6_K layer matrix and head made at load (one more copy of those
 * weight bytes in HBM; same values, so the same results). For A/B comparison. */
#define RIBN_LOAD_GEMM_FROM_PLANES 16u
/* Merge a long context's decode-attention split partials (more than 8 splits)
 * inside the attention launch, one workgroup per KV head, instead of in the
 * separate merge launch the chain uses by default. Same log-sum-exp merge, so
 * the same results up to summation order. For A/B comparison. */
#define RIBN_LOAD_ATTN_MERGE_IN_LAUNCH 32u

int ribn_rocm_load_gguf(const char *path, const ribn_rocm_load_options *opts, ribn_rocm_model **out,
                        char *err, size_t err_len);
/* Synchronizes, then frees every device resource. Safe on NULL. */
void ribn_rocm_free(ribn_rocm_model *model);

/* ExecutorInfo + GenerationLimits (executor.rs:43-71). */
typedef struct {
    char name[128];
    uint32_t context_tokens;
    uint32_t max_sequences;
    uint32_t max_batch_tokens;
    uint32_t max_decode_tokens;
    /* model geometry */
    uint32_t hidden, layers, q_heads, kv_heads, head_dim, ffn, vocab, rope_dims;
    uint64_t weight_bytes;     /* encoded bytes of all matrices on device */
    uint64_t kv_bytes;         /* KV pool bytes */
    uint32_t kv_f16;           /* 1: binary16 KV cache, 0: bfloat16 */
    uint32_t persistent_step;  /* 1: token steps run as one persistent kernel launch */
    uint32_t step_workgroups;  /* its grid size (co-resident workgroups) */
} ribn_rocm_info_t;
int ribn_rocm_info(const ribn_rocm_model *model, ribn_rocm_info_t *out);

/* ------------------------------------------------------------------------ */
/* GenerationExecutor (crates/runtime/src/executor.rs:171-254). */
#define RIBN_ADMIT_READY 0
#define RIBN_ADMIT_REJECTED 1
#define RIBN_ADMIT_DEFERRED 2
#define RIBN_STEP_PREFILL 0
#define RIBN_STEP_DECODE 1

typedef struct {
    uint32_t max_output_tokens;
    float temperature;            /* only 0 (greedy) is accepted, as the reference */
    const uint32_t *stop_tokens;
    uint32_t n_stop_tokens;
} ribn_rocm_token_options;

/* BatchItem (executor.rs:75-85). */
typedef struct {
    uint64_t sequence;
    uint32_t kind;                /* RIBN_STEP_PREFILL / RIBN_STEP_DECODE */
    uint32_t prefix;
    uint32_t token_budget;
    uint32_t output_budget;
} ribn_rocm_batch_item;

/* StepCompletion (executor.rs:113-117); at most one sampled token per row. */
typedef struct {
    uint64_t sequence;
    uint32_t prefix;
    uint32_t n_tokens;            /* 0 or 1 */
    uint32_t token;
    uint32_t reserved;
} ribn_rocm_step_completion;

/* admit (executor.rs:186-191; Qwen rules crates/qwen/src/execution.rs:80-161).
 * *admission receives RIBN_ADMIT_*; a rejection message goes to err. Returns
 * RIBN_OK unless the owner faulted. */
int ribn_rocm_admit(ribn_rocm_model *model, uint64_t request_id, uint64_t sequence,
                    const uint32_t *tokens, uint32_t n_tokens, const ribn_rocm_token_options *options,
                    int32_t *admission, char *err, size_t err_len);
/* prepare (executor.rs:199). Every row accepted unchanged = BatchPreparation::Ready. */
int ribn_rocm_prepare(ribn_rocm_model *model, const ribn_rocm_batch_item *items, size_t n_items,
                      char *err, size_t err_len);
/* abandon_preparation (executor.rs:206), idempotent. */
int ribn_rocm_abandon(ribn_rocm_model *model, char *err, size_t err_len);
/* submit (executor.rs:214): items must equal the prepared batch. */
int ribn_rocm_submit(ribn_rocm_model *model, const ribn_rocm_batch_item *items, size_t n_items,
                     uint64_t *submission, char *err, size_t err_len);
/* poll (executor.rs:226): RIBN_OK and exactly n_items completions in batch
 * order, RIBN_PENDING while device work is in flight, <0 on a terminal error. */
int ribn_rocm_poll(ribn_rocm_model *model, uint64_t submission, ribn_rocm_step_completion *out,
                   size_t out_cap, size_t *n_out, char *err, size_t err_len);
/* release (executor.rs:236), idempotent after success. */
int ribn_rocm_release(ribn_rocm_model *model, uint64_t sequence, char *err, size_t err_len);
/* synchronize (executor.rs:245). */
int ribn_rocm_synchronize(ribn_rocm_model *model, char *err, size_t err_len);

/* ------------------------------------------------------------------------ */
/* Lower seam: the per-sequence greedy step chain
 * (CudaQwen35Decode::{prefill_step, decode_step, run_step}, nvidia/src/decode.rs:495-640,
 * run_output_head decode.rs:686-700). The whole loop stays on the device: the
 * argmax of step t is the input token of step t+1, and each step is one HIP
 * graph replay. out_tokens receives n_new tokens. */
typedef struct {
    double prefill_ms;        /* device time, prompt */
    double decode_ms;         /* device time, n_new-1 decode steps after the first token */
    uint32_t prefill_tokens;
    uint32_t decode_tokens;
} ribn_rocm_timing;
int ribn_rocm_generate(ribn_rocm_model *model, const uint32_t *prompt, uint32_t n_prompt,
                       uint32_t n_new, uint32_t *out_tokens, ribn_rocm_timing *timing, char *err,
                       size_t err_len);

/* Teacher-forced trace for parity tests: runs tokens[0..n) one position at a
 * time on a scratch sequence; for each position writes the argmax token, and
 * optionally the final-normed logits (n*vocab floats) and the residual stream
 * after the embedding and after every layer (n*(layers+1)*hidden floats). */
int ribn_rocm_trace(ribn_rocm_model *model, const uint32_t *tokens, uint32_t n, uint32_t *argmax_out,
                    float *logits_out, float *hidden_out, char *err, size_t err_len);

/* Chunked prefill parity trace: tokens[0..n) through the chunked prefill path
 * (prefill_chunk / run_prefill_chunk, nvidia/src/decode.rs:2124,2360) in chunks of
 * min(chunk, prepared) rows (0 = prepared) on a scratch sequence. logits_out
 * [n][vocab] (final RMSNorm + head for every row) and hidden_out
 * [(layers + 1)][n][hidden] (after the embedding and every layer) are optional. */
int ribn_rocm_prefill_trace(ribn_rocm_model *model, const uint32_t *tokens, uint32_t n, uint32_t chunk,
                            float *logits_out, float *hidden_out, char *err, size_t err_len);

/* Parity aid for batched decode (no reference counterpart; the reference's
 * dispatcher returns only the sampled token per row, adapter.rs:90-125): after
 * the last submission has been polled complete, copies the logits of the
 * decode rows that submission ran as one batched step, in batch order, into
 * out [n][vocab] and their sequence ids into sequences. *n_rows = 0 when the
 * last submission ran no batched step. RIBN_ERR_INVALID if cap_rows is too
 * small, RIBN_ERR_BUSY while a submission is pending. */
int ribn_rocm_batch_logits(ribn_rocm_model *model, uint64_t *sequences, float *out, size_t cap_rows,
                           size_t *n_rows, char *err, size_t err_len);

/* ------------------------------------------------------------------------ */
/* Kernel-level entry points (tests and bench). Host buffers in and out; the
 * weights go through the same load-time re-tiling as model tensors. */

/* Device dequantization of `rows` rows of `k` elements, bit-exact with
 * dequantize_block (crates/gguf/src/lib.rs:508-649). */
int ribn_rocm_dequantize(uint32_t type, const uint8_t *blocks, uint64_t rows, uint64_t k, float *out,
                         char *err, size_t err_len);
/* y = W x with the fused dequant-matvec kernel (gguf_gemv, nvidia/src/qwen_reference.rs:31-40;
 * q*_gemv_warp, kernels/quantized/q4_k.cu:103, q6_k.cu:45, q8_0.cu:27). If rms_weight
 * is not NULL the RMSNorm prologue is applied to x first (rms_norm, model_ops.rs:108). */
int ribn_rocm_gemv(uint32_t type, const uint8_t *blocks, uint64_t rows, uint64_t k, const float *x,
                   const float *rms_weight, float eps, float *y, char *err, size_t err_len);
/* Time `iters` launches of the matvec on device-resident data; *avg_ms gets the
 * HIP-event average per launch (on the launch stream). */
int ribn_rocm_bench_gemv(uint32_t type, uint64_t rows, uint64_t k, uint32_t iters, double *avg_ms,
                         char *err, size_t err_len);
/* Y[m][rows] = f16(X)[m][k] * dequantized(W)^T with the prefill MFMA GEMM (the
 * batched projection of gemv_batch, nvidia/src/decode.rs:1591-1633): X is rounded
 * to binary16, W dequantized exactly and rounded to binary16, fp32 accumulation. */
int ribn_rocm_prefill_gemm(uint32_t type, const uint8_t *blocks, uint64_t rows, uint64_t k, const float *x,
                           uint64_t m, float *y, char *err, size_t err_len);
/* Q8_1 packing of n values (n a positive multiple of 32) into n/32 * 9 words:
 * CudaQ8_1Quantizer::execute (nvidia/src/activation.rs; kernel activation.cu:1-28),
 * bit-identical words. */
int ribn_rocm_quantize_q8_1(const float *x, uint64_t n, uint32_t *out, char *err, size_t err_len);
/* Integer-dot matvec of `members` (1..8) Q8_1-packed inputs ([members][k/32 * 9]
 * words) against a Q8_0 / Q4_K / Q6_K matrix, y [members][rows]:
 * CudaQ4KQ8_1Gemv / CudaQ6KQ8_1Gemv / CudaQ8_0Q8_1Gemv ::execute and ::execute_batch
 * (nvidia/src/q4_q8_1.rs, q6_q8_1.rs, q8_0_q8_1.rs). */
int ribn_rocm_gemv_q8_1(uint32_t type, const uint8_t *blocks, uint64_t rows, uint64_t k, const uint32_t *packed,
                        uint32_t members, float *y, char *err, size_t err_len);
/* Time `iters` integer-dot launches on device-resident data (HIP events on the launch stream). */
int ribn_rocm_bench_gemv_q8_1(uint32_t type, uint64_t rows, uint64_t k, uint32_t members, uint32_t iters,
                              double *avg_ms, char *err, size_t err_len);
/* Greedy argmax (model_ops.rs:203-260): first maximum, NaN skipped. */
int ribn_rocm_argmax(const float *logits, uint64_t n, uint32_t *out, char *err, size_t err_len);

/* Allocation-free greedy argmax. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same kernel and result
 * as ribn_rocm_argmax, but d_logits (n floats) and d_out (one uint32) are device
 * pointers on the current device, and the work is enqueued on `stream` (a
 * hipStream_t; NULL = the default stream) without synchronizing. It calls no
 * allocator: the cross-workgroup partials and arrival counter live in a fixed
 * 8.4 KB device array per GPU, held until the process ends. Calls that overlap
 * on one GPU share that array and race; serialize them (one stream, or events).
 * n above RIBN_ARGMAX_NOALLOC_MAX returns RIBN_ERR_INVALID. */
#define RIBN_ARGMAX_NOALLOC_MAX 0x7fffffffull
int ribn_rocm_argmax_noalloc(const float *d_logits, uint64_t n, uint32_t *d_out, void *stream, char *err,
                             size_t err_len);

/* Model-resident timing of one launch of the decode chain, replayed `iters`
 * times on the model's stream: which = 0 fused gate/up (SwiGLU) of layer 0,
 * 1 ffn_down, 2 output head, 3 and 4 fused QKV, 5 attn_output, 6 decode attention of layer 0 (pass the context
 * length in the low 32 bits of *bytes and, in the high 32 bits, a split count to use instead of the default, or 0; the scratch sequence must hold that many positions, e.g.
 * after ribn_rocm_generate), 7 every layer's fused gate/up inside graph-replayed decode
 * steps, from its first workgroup's start to its last workgroup's end on the device
 * wall clock (the launch chain with the other launches in between; pass the
 * starting context in the low 32 bits of *bytes; the steps run on a scratch
 * sequence).
 * *avg_ms per launch; *bytes = encoded weight bytes one launch streams (0 for
 * attention). */
int ribn_rocm_bench_model_kernel(ribn_rocm_model *model, uint32_t which, uint32_t iters, double *avg_ms,
                                 uint64_t *bytes, char *err, size_t err_len);

/* Timing of one persistent decode step (no reference counterpart: a
 * profiling aid). Runs one step of the scratch sequence at context `ctx` (the
 * sequence must hold ctx positions, e.g. after ribn_rocm_generate) and writes
 * workgroup 0's wall clock in ns from the step's start at each mark: the start,
 * every grid-barrier arrival and release, every end of input staging and every
 * stage end. cap must be at least 64 * (layers + 1); *n receives the number of
 * marks. RIBN_ERR_INVALID if the model runs the launch chain. */
int ribn_rocm_step_stamps(ribn_rocm_model *model, uint32_t ctx, double *out_ns, size_t cap, size_t *n,
                          char *err, size_t err_len);

/* ------------------------------------------------------------------------ */
/* Synthetic model writer (test and benchmark inputs; no reference counterpart:
 * the reference loads real artifacts only). Seeded N(0, weight_std) weights,
 * quantized to GGML blocks, written as GGUF v3. */
/* ---- Gemma 4 text decoder (the GemmaDecode seam) ------------------------------
 * Replaces `trait GemmaDecode` (crates/gemma4/src/executor/backend.rs:10-33:
 * advance_prefill, prefill, decode, position, close) and its loader
 * TextOwner::load_gemma_cuda (crates/text/src/gemma_load.rs:63-101). The package
 * directory holds config.json and a single BF16 model.safetensors, checked as
 * Gemma4Source::open does (crates/gemma4/src/source.rs:56-160). Logits are BF16
 * bit patterns after the final soft cap, vocab entries. Failed chunks leave
 * the position unchanged. */
typedef struct ribn_rocm_gemma ribn_rocm_gemma;
typedef struct {
    uint32_t vocab, hidden, layers, context;
} ribn_rocm_gemma_info_t;
int ribn_rocm_gemma_open(const char *package_dir, int32_t device, ribn_rocm_gemma **out, char *err, size_t err_len);
void ribn_rocm_gemma_close(ribn_rocm_gemma *g);
int ribn_rocm_gemma_info(const ribn_rocm_gemma *g, ribn_rocm_gemma_info_t *out);
/* prefill (backend.rs:14): process the chunk, write its last token's logits */
int ribn_rocm_gemma_prefill(ribn_rocm_gemma *g, const uint32_t *tokens, uint32_t n, uint16_t *logits,
                            char *err, size_t err_len);
/* advance_prefill (backend.rs:12): process the chunk without the readout */
int ribn_rocm_gemma_advance_prefill(ribn_rocm_gemma *g, const uint32_t *tokens, uint32_t n, char *err,
                                    size_t err_len);
/* decode (backend.rs:16): one token, its logits */
int ribn_rocm_gemma_decode(ribn_rocm_gemma *g, uint32_t token, uint16_t *logits, char *err, size_t err_len);
/* position (backend.rs:18) */
uint32_t ribn_rocm_gemma_position(const ribn_rocm_gemma *g);
/* Gemma4CpuDecoder::reset (crates/gemma4/src/cpu/decoder.rs:98-105) */
int ribn_rocm_gemma_reset(ribn_rocm_gemma *g);

typedef struct {
    int32_t qwen3;            /* 1: qwen3 (q/k norm, no bias); 0: qwen2 (q/k/v bias) */
    uint32_t hidden, layers, q_heads, kv_heads, head_dim, ffn, vocab;
    uint32_t context_length;
    float rope_base, rms_eps, weight_std;
    float norm_jitter;        /* norm weights = 1 + N(0, norm_jitter) (0: exactly 1) */
    uint64_t seed;
    uint32_t weight_type;     /* default matrix type (0 -> Q4_K) */
    uint32_t attn_v_type, ffn_down_type, output_type, embd_type; /* 0 -> weight_type */
    int32_t tied_output;      /* 1: no output.weight (head tied to token_embd) */
    int32_t threads;          /* 0 -> min(16, cores) */
} ribn_rocm_synth_config;
int ribn_rocm_synth_qwen_gguf(const char *path, const ribn_rocm_synth_config *config, char *err,
                              size_t err_len);
/* The hybrid fields of a synthetic qwen35 model (Gated-DeltaNet + gated
 * attention, the reference's own architecture: crates/qwen/src/gguf/config.rs). */
typedef struct {
    uint32_t ssm_groups;      /* k heads of the recurrent layers (ssm.group_count) */
    uint32_t ssm_heads;       /* v heads (ssm.time_step_rank), a multiple of ssm_groups */
    uint32_t ssm_state;       /* head width of the recurrent layers (ssm.state_size) */
    uint32_t conv_kernel;     /* 0 -> 4 */
    uint32_t full_attention_interval;
    uint32_t rope_dims;       /* rotated dims of the attention heads (0 -> head_dim) */
    uint32_t ssm_type;        /* type of ssm_beta / ssm_alpha (0 -> Q8_0) */
} ribn_rocm_synth_hybrid;
/* Seeded synthetic qwen35 GGUF v3 (no reference counterpart: test inputs).
 * `config` gives the shared geometry (hidden, layers, attention heads and
 * head_dim, FFN, vocab, types, seed; rope_base 0 -> 1e7). */
int ribn_rocm_synth_qwen35_gguf(const char *path, const ribn_rocm_synth_config *config,
                                const ribn_rocm_synth_hybrid *hybrid, char *err, size_t err_len);
/* Quantize n floats into GGML blocks (n a multiple of the block size). */
int ribn_rocm_quantize(uint32_t type, const float *x, uint64_t n, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
