/* Gemma 4 host CPU BF16 decoder: a C restatement of the reference's eager-rounded
 * CPU forward (crates/gemma4/src/cpu/), used as the configs[0] CPU baseline and
 * parity anchor. Test and benchmark infrastructure only; no product code links it.
 *
 * Values are BF16 bit patterns (uint16_t). Every operation computes in FP32 and
 * rounds its result to BF16 once (round to nearest even), as the reference's
 * "eager" policy does; matrix products accumulate in FP32 in source order.
 *
 * Pinning: the operations by the reference's literal KATs (tests/cpu_ops.rs:21-135,
 * cpu_attention.rs:22-92) and its rotary fixture bits; the composed decoder
 * (g4_open/g4_step) by an independent numpy forward written from decoder.rs,
 * bit-identical logits (tests/test_gemma_composition.py), and by the reference's
 * prefill-equals-serial-decode invariant. */
#ifndef RIBN_ORACLE_GEMMA4_H
#define RIBN_ORACLE_GEMMA4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4_MAX_LAYERS 64

enum { G4_SLIDING = 0, G4_FULL = 1 };

/* Text configuration after the reference's normalization (config.rs:59-124,
 * layer geometry :297-380). kv_owner[l] == l for owner layers; shared tail layers
 * name the last owner of the same attention kind. */
typedef struct {
    int32_t vocab, hidden, intermediate, heads, kv_heads;
    int32_t ple, ple_vocab, context, window, layers;
    float eps, softcap;
    int32_t kind[G4_MAX_LAYERS];        /* G4_SLIDING / G4_FULL */
    int32_t head_dim[G4_MAX_LAYERS];
    int32_t kv_owner[G4_MAX_LAYERS];
    int32_t proportional[G4_MAX_LAYERS]; /* quarter-proportional RoPE (full layers) */
    float theta[G4_MAX_LAYERS];
} g4_config;

/* Parameter tensors, row-major BF16 ([out][in] for projections), with the shapes
 * of parameters.rs:106-160. k, v and k_norm are only read for owner layers. */
typedef struct {
    const uint16_t *q, *k, *v, *o, *q_norm, *k_norm;
    const uint16_t *input_norm, *post_attention_norm, *pre_feedforward_norm, *post_feedforward_norm;
    const uint16_t *gate, *up, *down;
    const uint16_t *ple_gate, *ple_projection, *post_ple_norm, *layer_scalar;
} g4_layer_weights;

typedef struct {
    const uint16_t *embed;          /* [vocab][hidden] (tied output head) */
    const uint16_t *ple_embed;      /* [ple_vocab][layers * ple] */
    const uint16_t *ple_projection; /* [layers * ple][hidden] */
    const uint16_t *ple_norm;       /* [ple] */
    const uint16_t *final_norm;     /* [hidden] */
    g4_layer_weights layer[G4_MAX_LAYERS];
} g4_weights;

/* ---- operations (cpu/linear.rs, norm.rs, elementwise.rs, rotary.rs, attention.rs) ---- */
uint16_t g4_bf16(float value);
float g4_load(uint16_t bits);
void g4_project(const uint16_t *input, int rows, int inner, const uint16_t *weight, int columns, uint16_t *out);
/* worker threads of g4_project (default 1, the reference); results do not depend on it */
void g4_set_threads(int n);
/* scale == NULL: the scale-free value normalization */
void g4_rms_norm(const uint16_t *input, int rows, int width, float eps, const uint16_t *scale, uint16_t *out);
void g4_add(const uint16_t *a, const uint16_t *b, size_t n, uint16_t *out);
void g4_multiply(const uint16_t *a, const uint16_t *b, size_t n, uint16_t *out);
void g4_scale(const uint16_t *a, size_t n, float factor, uint16_t *out);
void g4_gelu_tanh(const uint16_t *a, size_t n, uint16_t *out);
void g4_softcap(const uint16_t *a, size_t n, float cap, uint16_t *out);
void g4_ple_combine(const uint16_t *context, const uint16_t *token, size_t n, uint16_t *out);
/* returns 0, or -1 for a pair outside the half head */
int g4_inverse_frequency(const g4_config *c, int layer, int pair, float *out);
/* cosine/sine [rows][head_dim] for the given positions */
int g4_factors(const g4_config *c, int layer, const uint32_t *positions, int rows, uint16_t *cosine, uint16_t *sine);
void g4_apply_rotary(const uint16_t *input, int rows, int heads, int width, const uint16_t *cosine,
                     const uint16_t *sine, uint16_t *out);
/* window <= 0: full attention. weights (optional) [heads][seq][kv_seq] */
int g4_attention(const uint16_t *query, int seq, const uint16_t *keys, const uint16_t *values, int kv_seq, int heads,
                 int kv_heads, int width, int window, int query_start, int key_start, uint16_t *out,
                 uint16_t *weights);
/* first maximum; -1 for an empty vector */
int64_t g4_argmax(const uint16_t *logits, int n);

/* ---- decoder (cpu/decoder.rs) ---- */
typedef struct g4_decoder g4_decoder;
/* weights must outlive the decoder; returns NULL with a message on invalid config */
g4_decoder *g4_open(const g4_config *c, const g4_weights *w, char *err, size_t err_len);
void g4_close(g4_decoder *d);
void g4_reset(g4_decoder *d);
int g4_position(const g4_decoder *d);
/* Process a chunk; logits (vocab BF16 values, post soft cap) of its last token are
 * written when logits != NULL (prefill/decode) and skipped otherwise
 * (advance_prefill). Returns 0, or -1 for an empty/overlong/out-of-range chunk,
 * leaving the decoder unchanged. */
int g4_step(g4_decoder *d, const uint32_t *tokens, int n, uint16_t *logits);

#ifdef __cplusplus
}
#endif
#endif
