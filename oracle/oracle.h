/*
 * ribn-rocm CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's host arithmetic for the Qwen
 * autoregressive token loop. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline). The product library never links it.
 *
 * Pinning status of each function (what checks it besides its own formula):
 *   orc_f16_to_f32        pinned: reference KATs (lib.rs:1480-1497) + exhaustive
 *                         65536-pattern comparison against IEEE binary16 (numpy)
 *   orc_tensor_layout     pinned: byte_len KATs (lib.rs:1585-1625)
 *   orc_dequantize_block  pinned: reference KATs (lib.rs:1480-1583), dyadic block
 *                         builder identity (nvidia/tests/q4_q8_1.rs:15-50,205-228)
 *   orc_gguf_*            pinned: parser fixture (lib.rs:1219-1276), error cases
 *   orc_gemv_q            pinned: closed form (fp64 dot of dequantized values)
 *   orc_rms_norm          pinned: constant-vector closed form
 *   orc_rope_neox         pinned: pos 0 identity, norm preservation, pos-additivity
 *   orc_argmax            pinned: ties -> lowest index, NaN skipped
 *   orc_quantize_q8_1     pinned: reference KAT (nvidia/tests/cuda_activation.rs:8-44),
 *                         dyadic inputs packed without loss (q4_q8_1.rs:88-101,
 *                         200-222), |x - d q| <= d/2 and the header sum within
 *                         half rounding of the exact sum
 *   orc_gemv_q8_1         pinned: the reference's host fixtures and bounds
 *                         (q4_q8_1.rs, q6_q8_1.rs, q8_0_q8_1.rs: exact on dyadic
 *                         inputs, within the packing error bound of the float
 *                         product otherwise) and a brute force over dequantized
 *                         weights and dequantized Q8_1 activations
 *   orc_qwen_*            composition of the above; the reference cannot run dense
 *                         Qwen2/Qwen3, so the composed forward is pinned only by
 *                         its parts plus single-token closed forms (1-token
 *                         attention returns v).
 */
#ifndef RIBN_ORACLE_H
#define RIBN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes (mirror the GgufError variants the tests exercise). */
enum {
    ORC_OK = 0,
    ORC_ERR_UNSUPPORTED_TYPE = -1,
    ORC_ERR_BLOCK_LENGTH = -2,
    ORC_ERR_MAGIC = -3,
    ORC_ERR_VERSION = -4,
    ORC_ERR_TRUNCATED = -5,
    ORC_ERR_DUPLICATE_METADATA = -6,
    ORC_ERR_ALIGNMENT = -7,
    ORC_ERR_OFFSET = -8,
    ORC_ERR_DIMENSION = -9,
    ORC_ERR_IO = -10,
    ORC_ERR_LENGTH = -11,
    ORC_ERR_MISSING = -12,
    ORC_ERR_CONFIG = -13,
};

float orc_f16_to_f32(uint16_t bits);
int orc_tensor_layout(uint32_t value_type, uint64_t *block_elements, uint64_t *block_bytes);
/* Dequantize exactly one block. Returns the number of values written or an error. */
int orc_dequantize_block(uint32_t value_type, const uint8_t *encoded, size_t len, float *out);
/* Dequantize `nblocks` consecutive blocks. Returns values written or an error. */
int64_t orc_dequantize(uint32_t value_type, const uint8_t *encoded, size_t len, float *out);
/* byte_len of a tensor with the given dims (ne0 first), or a negative error. */
int64_t orc_tensor_byte_len(uint32_t value_type, const uint64_t *dims, uint32_t ndims);

/* ---- GGUF v3 reader ---- */
typedef struct orc_gguf orc_gguf;
int orc_gguf_open(const char *path, orc_gguf **out);
void orc_gguf_close(orc_gguf *g);
uint32_t orc_gguf_version(const orc_gguf *g);
uint64_t orc_gguf_tensor_count(const orc_gguf *g);
uint64_t orc_gguf_data_offset(const orc_gguf *g);
/* metadata accessors: return 0 on success, ORC_ERR_MISSING / ORC_ERR_CONFIG otherwise */
int orc_gguf_get_u64(const orc_gguf *g, const char *key, uint64_t *out);
int orc_gguf_get_f32(const orc_gguf *g, const char *key, float *out);
int orc_gguf_get_str(const orc_gguf *g, const char *key, char *out, size_t cap);
/* tensor lookup by name: fills type, dims (up to 4) and absolute byte range */
int orc_gguf_tensor(const orc_gguf *g, const char *name, uint32_t *type, uint64_t *dims,
                    uint32_t *ndims, uint64_t *start, uint64_t *len);
const uint8_t *orc_gguf_bytes(const orc_gguf *g);

/* ---- host equations ---- */
/* y[n] = sum_k dequant(W[n,k]) * x[k], block-streamed dequant then an f32
 * sequential dot per row (gguf_gemv, qwen_reference.rs:31-40). */
int orc_gemv_q(uint32_t value_type, const uint8_t *w, uint64_t rows, uint64_t k,
               const float *x, float *y, int threads);
void orc_rms_norm(const float *x, const float *w, float *y, int n, float eps);
void orc_rope_neox(float *v, int heads, int head_dim, int rot_dim, int64_t pos, float base);
uint32_t orc_argmax(const float *logits, int n);

/* ---- dense Qwen2/Qwen3 FP32 forward (composition) ---- */
typedef struct orc_qwen orc_qwen;
int orc_qwen_open(const char *gguf_path, int max_ctx, orc_qwen **out);
void orc_qwen_close(orc_qwen *m);
/* config: hidden, layers, q_heads, kv_heads, head_dim, ffn, vocab, rot_dim */
void orc_qwen_config(const orc_qwen *m, int32_t *cfg8, float *eps, float *rope_base);
/* Run one token at position `pos` (positions must be fed in order 0,1,2...).
 * logits (vocab floats) may be NULL; hidden_trace, if not NULL, receives
 * (layers+1)*hidden floats: the residual stream after embedding and after each
 * layer. final_norm (hidden floats) may be NULL. */
int orc_qwen_step(orc_qwen *m, uint32_t token, int pos, float *logits, float *hidden_trace,
                  float *final_norm);
/* Advance one position writing only what later positions read: every layer's
 * K/V cache entry. Layers before the last still run in full (their outputs feed
 * the next layer's K/V); the last layer stops after its cache append, and no
 * readout is computed. Equal to orc_qwen_step for every later position's
 * result, at a fraction of the cost on 1-layer models (long-context tests). */
int orc_qwen_append_kv(orc_qwen *m, uint32_t token, int pos);
void orc_qwen_reset(orc_qwen *m);
/* Round K/V as they enter the cache: 0 = keep f32 (reference host equations),
 * 1 = binary16 RNE (the reference CUDA cache, model_ops.rs:1210-1276),
 * 2 = bfloat16 RNE (the build's default device cache). */
void orc_qwen_set_kv_round(orc_qwen *m, int mode);
/* Worker threads of the forward's matvecs (default 1, as the reference's host
 * path). Rows are split between threads and each row's sum stays one sequential
 * chain, so the results are bit-identical for every thread count. */
void orc_qwen_set_threads(orc_qwen *m, int threads);
/* Projection mode of later steps: ORC_GEMV_FLOAT (default) or ORC_GEMV_INT_DOT,
 * the reference's GemvMode::IntegerDot (nvidia/src/decode.rs:298-312). */
enum { ORC_GEMV_FLOAT = 0, ORC_GEMV_INT_DOT = 2 };
void orc_qwen_set_gemv_mode(orc_qwen *m, int mode);
/* ---- qwen35 hybrid forward (qwen35.c): Gated-DeltaNet + gated attention ---- */
typedef struct orc_q35 orc_q35;
int orc_q35_open(const char *gguf_path, int max_ctx, orc_q35 **out);
void orc_q35_close(orc_q35 *m);
/* hidden, layers, q_heads, kv_heads, head_dim, ffn, vocab, rot, ssm k heads,
 * ssm v heads, ssm head width, full_attention_interval */
void orc_q35_config(const orc_q35 *m, int32_t *cfg12);
/* one token at `pos` (in order); logits and (layers+1)*hidden trace optional */
int orc_q35_step(orc_q35 *m, uint32_t token, int pos, float *logits, float *hidden_trace);
void orc_q35_reset(orc_q35 *m);
void orc_q35_set_kv_round(orc_q35 *m, int mode);
/* gdn_state_step on one head: state [kd][vd] (row = key index) updated in place,
 * k, q [kd], v and out [vd] */
void orc_gdn_state_step(float *state, const float *k, const float *v, const float *q, float decay, float beta,
                        int kd, int vd, float *out);
float orc_round_f16(float x);
/* quantize_q8_1 (nvidia/src/activation.cu): n % 32 == 0, out gets n/32 * 9 words. */
int orc_quantize_q8_1(const float *x, uint64_t n, uint32_t *out);
/* Integer-dot matvec over Q8_1-packed inputs (types Q8_0, Q4_K, Q6_K); `packed`
 * holds `members` inputs of k/32 * 9 words, y gets [members][rows]. */
int orc_gemv_q8_1(uint32_t value_type, const uint8_t *w, uint64_t rows, uint64_t k, const uint32_t *packed,
                  uint32_t members, float *y, int threads);
float orc_round_bf16(float x);

#ifdef __cplusplus
}
#endif
#endif
