/* Gemma 4 host CPU BF16 decoder, restated from the reference's Rust CPU path
 * (crates/gemma4/src/cpu/). TEST AND BENCHMARK INFRASTRUCTURE ONLY: it is the
 * configs[0] CPU baseline and the arithmetic anchor of the Gemma tests; no
 * product code links it. Built with -ffp-contract=off, so every FP32 multiply
 * and add rounds separately, in the reference's source order. The
 * transcendental functions are the C library's expf, tanhf, cosf, sinf, powf and
 * sqrtf, which is what Rust's f32 methods lower to on Linux. */
#include "gemma4.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* bf16 (cpu/linear.rs:10-16): round to nearest even; NaN -> canonical 0x7fc0 */
uint16_t g4_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

float g4_load(uint16_t bits) {
    const uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float bf16_f32(float v) { return g4_load(g4_bf16(v)); }

/* Threads for g4_project (1 = the reference's single-threaded loops). Each
 * output's sum is one sequential chain in one thread, so any thread count gives
 * bit-identical results; the multi-threaded run is a CPU baseline line only. */
static int g4_threads = 1;
void g4_set_threads(int n) { g4_threads = n < 1 ? 1 : n > 64 ? 64 : n; }

typedef struct {
    const uint16_t *input, *weight;
    uint16_t *out;
    int rows, inner, columns, c0, c1;
} g4_project_job;

static void *g4_project_range(void *arg) {
    const g4_project_job *j = (const g4_project_job *)arg;
    for (int r = 0; r < j->rows; r++) {
        const uint16_t *x = j->input + (size_t)r * j->inner;
        for (int c = j->c0; c < j->c1; c++) {
            const uint16_t *w = j->weight + (size_t)c * j->inner;
            float sum = 0.0f;
            for (int k = 0; k < j->inner; k++) {
                const float a = g4_load(x[k]), b = g4_load(w[k]);
                sum += a * b;
            }
            j->out[(size_t)r * j->columns + c] = g4_bf16(sum);
        }
    }
    return NULL;
}

/* project (cpu/linear.rs:23-66): per output, an FP32 sum over k in order of
 * separately rounded products, then one BF16 rounding */
void g4_project(const uint16_t *input, int rows, int inner, const uint16_t *weight, int columns, uint16_t *out) {
    int nt = g4_threads;
    if (nt > columns) nt = columns;
    if (nt <= 1) {
        g4_project_job j = {input, weight, out, rows, inner, columns, 0, columns};
        g4_project_range(&j);
        return;
    }
    pthread_t th[64];
    g4_project_job jobs[64];
    const int per = (columns + nt - 1) / nt;
    int started = 0;
    for (int t = 0; t < nt; t++) {
        const int c0 = t * per, c1 = c0 + per < columns ? c0 + per : columns;
        jobs[t] = (g4_project_job){input, weight, out, rows, inner, columns, c0, c1};
        if (c0 >= c1) continue;
        if (pthread_create(&th[started], NULL, g4_project_range, &jobs[t]) != 0) g4_project_range(&jobs[t]);
        else started++;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
}

/* normalize (cpu/norm.rs:41-82): FP32 energy, (mean + eps)^-0.5, direct BF16 scale, one rounding */
void g4_rms_norm(const uint16_t *input, int rows, int width, float eps, const uint16_t *scale, uint16_t *out) {
    for (int r = 0; r < rows; r++) {
        const uint16_t *x = input + (size_t)r * width;
        float energy = 0.0f;
        for (int i = 0; i < width; i++) {
            const float v = g4_load(x[i]);
            energy += v * v;
        }
        const float mean = energy / (float)width;
        const float inverse = powf(mean + eps, -0.5f);
        for (int i = 0; i < width; i++) {
            float v = g4_load(x[i]) * inverse;
            if (scale) v *= g4_load(scale[i]);
            out[(size_t)r * width + i] = g4_bf16(v);
        }
    }
}

/* elementwise (cpu/elementwise.rs:14-52) */
void g4_add(const uint16_t *a, const uint16_t *b, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = g4_bf16(g4_load(a[i]) + g4_load(b[i]));
}
void g4_multiply(const uint16_t *a, const uint16_t *b, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = g4_bf16(g4_load(a[i]) * g4_load(b[i]));
}
void g4_scale(const uint16_t *a, size_t n, float factor, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = g4_bf16(g4_load(a[i]) * factor);
}

/* gelu_tanh (elementwise.rs:60-75): 0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2))) */
void g4_gelu_tanh(const uint16_t *a, size_t n, uint16_t *out) {
    const float alpha = 0.7978846f, cubic = 0.044715f;
    for (size_t i = 0; i < n; i++) {
        const float x = g4_load(a[i]);
        const float inner = alpha * x * (1.0f + cubic * x * x);
        out[i] = g4_bf16(0.5f * x * (1.0f + tanhf(inner)));
    }
}

/* softcap (elementwise.rs:80-99): divide, tanh, multiply, BF16 rounding after each */
void g4_softcap(const uint16_t *a, size_t n, float cap, uint16_t *out) {
    for (size_t i = 0; i < n; i++) {
        const uint16_t divided = g4_bf16(g4_load(a[i]) / cap);
        const uint16_t hyperbolic = g4_bf16(tanhf(g4_load(divided)));
        out[i] = g4_bf16(g4_load(hyperbolic) * cap);
    }
}

/* ple_combine (elementwise.rs:101-107): (context + token) * 2^-1/2, each step rounded */
void g4_ple_combine(const uint16_t *context, const uint16_t *token, size_t n, uint16_t *out) {
    g4_add(context, token, n, out);
    g4_scale(out, n, 0.70710677f, out);
}

/* rotary_inverse_frequency (config.rs:217-247): 1 / theta^(2p / head_dim) with an FP32
 * exponent; quarter-proportional layers keep only the first pairs/4 and pad with +0 */
int g4_inverse_frequency(const g4_config *c, int layer, int pair, float *out) {
    if (layer < 0 || layer >= c->layers) return -1;
    const int pairs = c->head_dim[layer] / 2;
    if (pair < 0 || pair >= pairs) return -1;
    const int active = c->proportional[layer] ? pairs / 4 : pairs;
    if (pair >= active) {
        *out = 0.0f;
        return 0;
    }
    const float exponent = (float)(pair * 2) / (float)c->head_dim[layer];
    *out = 1.0f / powf(c->theta[layer], exponent);
    return 0;
}

/* factors (cpu/rotary.rs:33-81): phase = position * frequency in FP32, BF16 cos/sin,
 * halves duplicated */
int g4_factors(const g4_config *c, int layer, const uint32_t *positions, int rows, uint16_t *cosine, uint16_t *sine) {
    if (layer < 0 || layer >= c->layers || rows <= 0) return -1;
    const int width = c->head_dim[layer], half = width / 2;
    for (int r = 0; r < rows; r++) {
        if (positions[r] >= (1u << 24)) return -1;
        const float position = (float)positions[r];
        for (int p = 0; p < half; p++) {
            float frequency;
            g4_inverse_frequency(c, layer, p, &frequency);
            const float phase = position * frequency;
            const uint16_t cb = g4_bf16(cosf(phase)), sb = g4_bf16(sinf(phase));
            const size_t base = (size_t)r * width + p;
            cosine[base] = cosine[base + half] = cb;
            sine[base] = sine[base + half] = sb;
        }
    }
    return 0;
}

static float rounded_product(float a, float b) { return bf16_f32(a * b); }

/* apply_rotary (cpu/rotary.rs:88-134): channel j pairs with j + width/2; each product
 * rounds to BF16 before the FP32 addition, the sum rounds again */
void g4_apply_rotary(const uint16_t *input, int rows, int heads, int width, const uint16_t *cosine,
                     const uint16_t *sine, uint16_t *out) {
    const int half = width / 2;
    for (int r = 0; r < rows; r++)
        for (int h = 0; h < heads; h++) {
            const size_t base = ((size_t)r * heads + h) * width;
            for (int j = 0; j < half; j++) {
                const size_t f = (size_t)r * width + j;
                const float a = g4_load(input[base + j]), b = g4_load(input[base + j + half]);
                const float c1 = g4_load(cosine[f]), s1 = g4_load(sine[f]);
                const float c2 = g4_load(cosine[f + half]), s2 = g4_load(sine[f + half]);
                const float first = rounded_product(a, c1) + rounded_product(-b, s1);
                const float second = rounded_product(b, c2) + rounded_product(a, s2);
                out[base + j] = g4_bf16(first);
                out[base + j + half] = g4_bf16(second);
            }
        }
}

/* attention (cpu/attention.rs:33-277): BF16 scores (scale 1), FP32 softmax, BF16
 * weights, FP32 weights x values, BF16 output; causal, optionally sliding */
int g4_attention(const uint16_t *query, int seq, const uint16_t *keys, const uint16_t *values, int kv_seq, int heads,
                 int kv_heads, int width, int window, int query_start, int key_start, uint16_t *out,
                 uint16_t *weights) {
    if (heads <= 0 || kv_heads <= 0 || width <= 0 || heads % kv_heads || seq <= 0 || kv_seq <= 0) return -1;
    if (query_start + seq > key_start + kv_seq || query_start < key_start) return -1;
    const int head_step = heads * width, kv_step = kv_heads * width, groups = heads / kv_heads;
    float *scores = (float *)malloc(sizeof(float) * (size_t)kv_seq);
    float *acc = (float *)malloc(sizeof(float) * (size_t)width);
    if (!scores || !acc) {
        free(scores);
        free(acc);
        return -1;
    }
    if (weights) memset(weights, 0, sizeof(uint16_t) * (size_t)heads * seq * kv_seq);
    for (int pos = 0; pos < seq; pos++) {
        const int absolute = query_start + pos;
        int last = absolute - key_start;
        if (last > kv_seq - 1) last = kv_seq - 1;
        int first = 0;
        if (window > 0) {
            int a = absolute - (window - 1);
            if (a < 0) a = 0;
            a -= key_start;
            if (a < 0) a = 0;
            first = a < last ? a : last;
        }
        for (int h = 0; h < heads; h++) {
            const int kvh = h / groups;
            const uint16_t *q = query + (size_t)pos * head_step + (size_t)h * width;
            float maximum = -INFINITY;
            for (int t = first; t <= last; t++) {
                const uint16_t *k = keys + (size_t)t * kv_step + (size_t)kvh * width;
                float sum = 0.0f;
                for (int i = 0; i < width; i++) sum += g4_load(q[i]) * g4_load(k[i]);
                scores[t] = bf16_f32(sum);
                maximum = fmaxf(maximum, scores[t]);
            }
            float total = 0.0f;
            for (int t = first; t <= last; t++) {
                scores[t] = expf(scores[t] - maximum);
                total += scores[t];
            }
            for (int i = 0; i < width; i++) acc[i] = 0.0f;
            for (int t = first; t <= last; t++) {
                const uint16_t wgt = g4_bf16(scores[t] / total);
                if (weights) weights[((size_t)h * seq + pos) * kv_seq + t] = wgt;
                const uint16_t *v = values + (size_t)t * kv_step + (size_t)kvh * width;
                for (int i = 0; i < width; i++) acc[i] += g4_load(wgt) * g4_load(v[i]);
            }
            uint16_t *o = out + (size_t)pos * head_step + (size_t)h * width;
            for (int i = 0; i < width; i++) o[i] = g4_bf16(acc[i]);
        }
    }
    free(scores);
    free(acc);
    return 0;
}

/* argmax (cpu/decoder.rs:316-332): the first maximum; NaN never wins */
int64_t g4_argmax(const uint16_t *logits, int n) {
    if (n <= 0) return -1;
    int best = 0;
    for (int i = 1; i < n; i++)
        if (g4_load(logits[i]) > g4_load(logits[best])) best = i;
    return best;
}

/* ---- decoder ---- */

struct g4_decoder {
    g4_config c;
    const g4_weights *w;
    uint16_t *keys[G4_MAX_LAYERS], *values[G4_MAX_LAYERS];   /* owner layers: [context][kv_heads * head_dim] */
    int position;
    float embed_scale, ple_embed_scale, ple_projection_scale;
};

static void set_err(char *err, size_t len, const char *msg) {
    if (err && len) snprintf(err, len, "%s", msg);
}

g4_decoder *g4_open(const g4_config *c, const g4_weights *w, char *err, size_t err_len) {
    if (c->layers <= 0 || c->layers > G4_MAX_LAYERS || c->hidden <= 0 || c->heads <= 0 || c->kv_heads <= 0 ||
        c->heads % c->kv_heads || c->ple <= 0 || c->vocab <= 0 || c->ple_vocab < c->vocab || c->context <= 0 ||
        c->window <= 0 || !(c->eps > 0.0f) || !(c->softcap > 0.0f)) {
        set_err(err, err_len, "invalid Gemma 4 configuration");
        return NULL;
    }
    for (int l = 0; l < c->layers; l++)
        if (c->kv_owner[l] > l || c->kv_owner[l] < 0 || c->head_dim[l] <= 0 || c->head_dim[l] % 2 ||
            c->kind[c->kv_owner[l]] != c->kind[l] || c->head_dim[c->kv_owner[l]] != c->head_dim[l]) {
            set_err(err, err_len, "key/value owner must precede its consumer and share its geometry");
            return NULL;
        }
    g4_decoder *d = (g4_decoder *)calloc(1, sizeof(g4_decoder));
    if (!d) return NULL;
    d->c = *c;
    d->w = w;
    for (int l = 0; l < c->layers; l++) {
        if (c->kv_owner[l] != l) continue;
        const size_t n = (size_t)c->context * c->kv_heads * c->head_dim[l];
        d->keys[l] = (uint16_t *)malloc(2 * n);
        d->values[l] = (uint16_t *)malloc(2 * n);
        if (!d->keys[l] || !d->values[l]) {
            g4_close(d);
            set_err(err, err_len, "out of memory");
            return NULL;
        }
    }
    /* Scales (decoder.rs:78-95): sqrt(hidden) and sqrt(ple) rounded to BF16; 1/sqrt(hidden) in FP32 */
    d->embed_scale = bf16_f32(sqrtf((float)c->hidden));
    d->ple_embed_scale = bf16_f32(sqrtf((float)c->ple));
    d->ple_projection_scale = 1.0f / sqrtf((float)c->hidden);
    return d;
}

void g4_close(g4_decoder *d) {
    if (!d) return;
    for (int l = 0; l < G4_MAX_LAYERS; l++) {
        free(d->keys[l]);
        free(d->values[l]);
    }
    free(d);
}

void g4_reset(g4_decoder *d) { d->position = 0; }
int g4_position(const g4_decoder *d) { return d->position; }

static uint16_t *alloc16(size_t n) { return (uint16_t *)malloc(2 * (n ? n : 1)); }

/* attention_forward (decoder.rs:487-577) */
static void attention_forward(g4_decoder *d, int layer, int seq, const uint32_t *positions, uint16_t *hidden) {
    const g4_config *c = &d->c;
    const g4_layer_weights *lw = &d->w->layer[layer];
    const int H = c->hidden, heads = c->heads, kvh = c->kv_heads, width = c->head_dim[layer];
    const int owner = c->kv_owner[layer];
    uint16_t *normed = alloc16((size_t)seq * H), *q = alloc16((size_t)seq * heads * width);
    uint16_t *qn = alloc16((size_t)seq * heads * width), *cosine = alloc16((size_t)seq * width);
    uint16_t *sine = alloc16((size_t)seq * width);
    g4_rms_norm(hidden, seq, H, c->eps, lw->input_norm, normed);
    g4_project(normed, seq, H, lw->q, heads * width, q);
    g4_rms_norm(q, seq * heads, width, c->eps, lw->q_norm, qn);
    g4_factors(c, layer, positions, seq, cosine, sine);
    g4_apply_rotary(qn, seq, heads, width, cosine, sine, q);   /* q: rotated queries */
    if (owner == layer) {
        const size_t kw = (size_t)kvh * width;
        uint16_t *k = alloc16(seq * kw), *kn = alloc16(seq * kw), *v = alloc16(seq * kw);
        g4_project(normed, seq, H, lw->k, (int)kw, k);
        g4_rms_norm(k, seq * kvh, width, c->eps, lw->k_norm, kn);
        g4_apply_rotary(kn, seq, kvh, width, cosine, sine, d->keys[layer] + (size_t)d->position * kw);
        g4_project(normed, seq, H, lw->v, (int)kw, v);
        g4_rms_norm(v, seq * kvh, width, c->eps, NULL, d->values[layer] + (size_t)d->position * kw);
        free(k);
        free(kn);
        free(v);
    }
    const int kv_seq = d->position + seq;
    uint16_t *attended = alloc16((size_t)seq * heads * width);
    g4_attention(q, seq, d->keys[owner], d->values[owner], kv_seq, heads, kvh, width,
                 c->kind[layer] == G4_SLIDING ? c->window : 0, d->position, 0, attended, NULL);
    uint16_t *projected = alloc16((size_t)seq * H);
    g4_project(attended, seq, heads * width, lw->o, H, projected);
    g4_rms_norm(projected, seq, H, c->eps, lw->post_attention_norm, normed);
    g4_add(hidden, normed, (size_t)seq * H, hidden);
    free(normed);
    free(q);
    free(qn);
    free(cosine);
    free(sine);
    free(attended);
    free(projected);
}

/* feedforward_forward (decoder.rs:579-626): GELU-tanh gated FFN, then the PLE gate,
 * then the layer scalar */
static void feedforward_forward(g4_decoder *d, int layer, int seq, uint16_t *hidden, const uint16_t *per_layer) {
    const g4_config *c = &d->c;
    const g4_layer_weights *lw = &d->w->layer[layer];
    const int H = c->hidden, F = c->intermediate, P = c->ple;
    const size_t nh = (size_t)seq * H, nf = (size_t)seq * F, np = (size_t)seq * P;
    uint16_t *normed = alloc16(nh), *gate = alloc16(nf), *up = alloc16(nf), *down = alloc16(nh);
    g4_rms_norm(hidden, seq, H, c->eps, lw->pre_feedforward_norm, normed);
    g4_project(normed, seq, H, lw->gate, F, gate);
    g4_project(normed, seq, H, lw->up, F, up);
    g4_gelu_tanh(gate, nf, gate);
    g4_multiply(gate, up, nf, gate);
    g4_project(gate, seq, F, lw->down, H, down);
    g4_rms_norm(down, seq, H, c->eps, lw->post_feedforward_norm, normed);
    g4_add(hidden, normed, nh, hidden);
    uint16_t *pg = alloc16(np);
    g4_project(hidden, seq, H, lw->ple_gate, P, pg);
    g4_gelu_tanh(pg, np, pg);
    g4_multiply(pg, per_layer, np, pg);
    g4_project(pg, seq, P, lw->ple_projection, H, down);
    g4_rms_norm(down, seq, H, c->eps, lw->post_ple_norm, normed);
    g4_add(hidden, normed, nh, hidden);
    g4_scale(hidden, nh, g4_load(lw->layer_scalar[0]), hidden);
    free(normed);
    free(gate);
    free(up);
    free(down);
    free(pg);
}

/* step + run_body + project_logits (decoder.rs:129-192, 334-430) */
int g4_step(g4_decoder *d, const uint32_t *tokens, int n, uint16_t *logits) {
    const g4_config *c = &d->c;
    const g4_weights *w = d->w;
    if (n <= 0 || d->position + n > c->context) return -1;
    for (int i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)c->vocab) return -1;
    const int H = c->hidden, P = c->ple, packed = c->layers * P;
    uint16_t *hidden = alloc16((size_t)n * H), *identity = alloc16((size_t)n * packed);
    uint16_t *projection = alloc16((size_t)n * packed);
    for (int i = 0; i < n; i++) {
        g4_scale(w->embed + (size_t)tokens[i] * H, (size_t)H, d->embed_scale, hidden + (size_t)i * H);
        g4_scale(w->ple_embed + (size_t)tokens[i] * packed, (size_t)packed, d->ple_embed_scale,
                 identity + (size_t)i * packed);
    }
    g4_project(hidden, n, H, w->ple_projection, packed, projection);
    g4_scale(projection, (size_t)n * packed, d->ple_projection_scale, projection);
    uint16_t *per_layer = alloc16((size_t)c->layers * n * P), *slice = alloc16((size_t)n * P);
    uint16_t *slice_id = alloc16((size_t)n * P);
    for (int l = 0; l < c->layers; l++) {
        for (int t = 0; t < n; t++) {
            memcpy(slice + (size_t)t * P, projection + (size_t)t * packed + (size_t)l * P, 2 * (size_t)P);
            memcpy(slice_id + (size_t)t * P, identity + (size_t)t * packed + (size_t)l * P, 2 * (size_t)P);
        }
        uint16_t *ctx = per_layer + (size_t)l * n * P;
        g4_rms_norm(slice, n, P, c->eps, w->ple_norm, ctx);
        g4_ple_combine(ctx, slice_id, (size_t)n * P, ctx);
    }
    uint32_t *positions = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)n);
    for (int i = 0; i < n; i++) positions[i] = (uint32_t)(d->position + i);
    for (int l = 0; l < c->layers; l++) {
        attention_forward(d, l, n, positions, hidden);
        feedforward_forward(d, l, n, hidden, per_layer + (size_t)l * n * P);
    }
    if (logits) {
        uint16_t *normed = alloc16((size_t)H);
        g4_rms_norm(hidden + (size_t)(n - 1) * H, 1, H, c->eps, w->final_norm, normed);
        g4_project(normed, 1, H, w->embed, c->vocab, logits);
        g4_softcap(logits, (size_t)c->vocab, c->softcap, logits);
        free(normed);
    }
    d->position += n;
    free(hidden);
    free(identity);
    free(projection);
    free(per_layer);
    free(slice);
    free(slice_id);
    free(positions);
    return 0;
}
