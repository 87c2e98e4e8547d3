/*
 * ribn-rocm CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Plain C restatement of the reference's host arithmetic. Compiled with
 * -ffp-contract=off so that every multiply and add rounds separately, as the
 * reference's Rust code does.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* binary16 -> binary32, crates/gguf/src/lib.rs:539-551.
 * Subnormals: fraction * 2^-24; inf keeps its sign; every NaN becomes the
 * canonical quiet NaN 0x7fc00000 (f32::NAN), sign dropped. */
float orc_f16_to_f32(uint16_t bits) {
    float sign = (bits & 0x8000u) ? -1.0f : 1.0f;
    unsigned exponent = (bits >> 10) & 0x1fu;
    unsigned fraction = bits & 0x3ffu;
    if (exponent == 0) return sign * (float)fraction * ldexpf(1.0f, -24);
    if (exponent == 0x1f) {
        if (fraction == 0) return sign * INFINITY;
        uint32_t nan_bits = 0x7fc00000u;
        float f;
        memcpy(&f, &nan_bits, 4);
        return f;
    }
    return sign * (1.0f + (float)fraction / 1024.0f) * ldexpf(1.0f, (int)exponent - 15);
}

/* GGML (block elements, block bytes) table, crates/gguf/src/lib.rs:1039-1071. */
int orc_tensor_layout(uint32_t t, uint64_t *be, uint64_t *bb) {
    uint64_t e, b;
    switch (t) {
    case 0: case 26: e = 1; b = 4; break;
    case 1: case 25: case 30: e = 1; b = 2; break;
    case 2: case 20: e = 32; b = 18; break;
    case 3: e = 32; b = 20; break;
    case 6: e = 32; b = 22; break;
    case 7: e = 32; b = 24; break;
    case 8: e = 32; b = 34; break;
    case 9: e = 32; b = 36; break;
    case 10: e = 256; b = 84; break;
    case 11: case 21: e = 256; b = 110; break;
    case 12: e = 256; b = 144; break;
    case 13: e = 256; b = 176; break;
    case 14: e = 256; b = 210; break;
    case 15: e = 256; b = 292; break;
    case 16: case 35: e = 256; b = 66; break;
    case 17: e = 256; b = 74; break;
    case 18: e = 256; b = 98; break;
    case 19: e = 256; b = 50; break;
    case 22: e = 256; b = 82; break;
    case 23: e = 256; b = 136; break;
    case 24: e = 1; b = 1; break;
    case 27: case 28: e = 1; b = 8; break;
    case 29: e = 256; b = 56; break;
    case 34: e = 256; b = 54; break;
    case 39: e = 32; b = 17; break;
    case 40: e = 64; b = 36; break;
    case 41: e = 128; b = 18; break;
    case 42: e = 64; b = 18; break;
    default: return ORC_ERR_UNSUPPORTED_TYPE;
    }
    if (be) *be = e;
    if (bb) *bb = b;
    return ORC_OK;
}

/* TensorInfo::byte_len, crates/gguf/src/lib.rs:142-168. */
int64_t orc_tensor_byte_len(uint32_t t, const uint64_t *dims, uint32_t nd) {
    uint64_t be, bb;
    if (orc_tensor_layout(t, &be, &bb) != ORC_OK) return ORC_ERR_UNSUPPORTED_TYPE;
    if (nd == 0) return ORC_ERR_DIMENSION;
    if (dims[0] % be != 0) return ORC_ERR_DIMENSION;
    uint64_t n = 1;
    for (uint32_t i = 0; i < nd; i++) n *= dims[i];
    if (n % be != 0) return ORC_ERR_DIMENSION;
    return (int64_t)((n / be) * bb);
}

static float rd_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* q4_k_scales, crates/gguf/src/lib.rs:561-575: 6-bit scales/minima from 12 bytes. */
static void q4k_scales(const uint8_t *e, uint8_t sc[8], uint8_t mn[8]) {
    for (int i = 0; i < 4; i++) {
        sc[i] = e[i] & 0x3f;
        sc[i + 4] = (uint8_t)((e[8 + i] & 0x0f) | ((e[i] >> 2) & 0x30));
        mn[i] = e[4 + i] & 0x3f;
        mn[i + 4] = (uint8_t)((e[8 + i] >> 4) | ((e[4 + i] >> 2) & 0x30));
    }
}

/* dequantize_q8_0, lib.rs:577-582: d * q. */
static void deq_q8_0(const uint8_t *e, float *o) {
    float d = rd_f16(e);
    for (int i = 0; i < 32; i++) o[i] = d * (float)(int8_t)e[2 + i];
}

/* dequantize_q4_k, lib.rs:584-600: (d*sc)*q - (dmin*m), two separate roundings. */
static void deq_q4_k(const uint8_t *e, float *o) {
    float d = rd_f16(e), dmin = rd_f16(e + 2);
    uint8_t sc[8], mn[8];
    q4k_scales(e + 4, sc, mn);
    for (int g = 0; g < 8; g++) {
        const uint8_t *q = e + 16 + (g / 2) * 32;
        int shift = (g % 2) * 4;
        float gs = d * (float)sc[g];
        float gm = dmin * (float)mn[g];
        for (int i = 0; i < 32; i++) {
            float p = gs * (float)((q[i] >> shift) & 0x0f);
            o[g * 32 + i] = p - gm;
        }
    }
}

/* dequantize_q6_k, lib.rs:623-649: (d*sc)*(ql | qh<<4 - 32). */
static void deq_q6_k(const uint8_t *e, float *o) {
    const uint8_t *ql = e, *qh = e + 128, *scales = e + 192;
    float d = rd_f16(e + 208);
    int n = 0;
    for (int g = 0; g < 8; g++) {
        int chunk = g / 4, variant = g % 4;
        int lo_off = chunk * 64 + (variant % 2) * 32;
        int lo_shift = variant < 2 ? 0 : 4;
        int hi_off = chunk * 32;
        int hi_shift = variant % 4;
        for (int half = 0; half < 2; half++) {
            float gs = d * (float)(int8_t)scales[g * 2 + half];
            for (int i = 0; i < 16; i++) {
                int pos = half * 16 + i;
                int lo = (ql[lo_off + pos] >> lo_shift) & 0x0f;
                int hi = (qh[hi_off + pos] >> (hi_shift * 2)) & 0x03;
                int q = (lo | (hi << 4)) - 32;
                o[n++] = gs * (float)q;
            }
        }
    }
}

/* dequantize_block, lib.rs:508-535 (types in scope: F32, F16, Q8_0, Q4_K, Q6_K). */
int orc_dequantize_block(uint32_t t, const uint8_t *e, size_t len, float *o) {
    uint64_t be, bb;
    if (orc_tensor_layout(t, &be, &bb) != ORC_OK) return ORC_ERR_UNSUPPORTED_TYPE;
    if (len != bb) return ORC_ERR_BLOCK_LENGTH;
    switch (t) {
    case 0: memcpy(o, e, 4); return 1;
    case 1: o[0] = rd_f16(e); return 1;
    case 8: deq_q8_0(e, o); return 32;
    case 12: deq_q4_k(e, o); return 256;
    case 14: deq_q6_k(e, o); return 256;
    default: return ORC_ERR_UNSUPPORTED_TYPE;
    }
}

int64_t orc_dequantize(uint32_t t, const uint8_t *e, size_t len, float *o) {
    uint64_t be, bb;
    if (orc_tensor_layout(t, &be, &bb) != ORC_OK) return ORC_ERR_UNSUPPORTED_TYPE;
    if (len % bb) return ORC_ERR_BLOCK_LENGTH;
    int64_t n = 0;
    for (size_t off = 0; off < len; off += bb) {
        int r = orc_dequantize_block(t, e + off, bb, o + n);
        if (r < 0) return r;
        n += r;
    }
    return n;
}

/* ------------------------------------------------------------------------ */
/* GGUF v3 reader, crates/gguf/src/lib.rs:199-296 (read_value :1073-1116,
 * read_string :1130-1144, align :1178-1187). The whole file is read into
 * memory: the oracle only opens small models. */
#define GGUF_MAGIC 0x46554747u
#define MAX_STRING_BYTES (16ull * 1024 * 1024)
#define MAX_ARRAY_ITEMS 1000000ull
#define MAX_TENSORS 10000000ull

typedef struct {
    char *key;
    uint32_t type;      /* GGUF value type */
    uint64_t u;         /* integer payload (scalar ints / bool) */
    double f;           /* float payload */
    char *s;            /* string payload */
    int is_array;
} orc_kv;

typedef struct {
    char *name;
    uint32_t ndims;
    uint64_t dims[16];
    uint32_t type;
    uint64_t offset;
} orc_tensor;

struct orc_gguf {
    uint8_t *bytes;
    uint64_t len;
    uint32_t version;
    uint64_t n_kv, n_tensors;
    orc_kv *kv;
    orc_tensor *tensors;
    uint64_t data_offset;
};

typedef struct { const uint8_t *p; uint64_t len, pos; int err; } rd_t;

static int rd_need(rd_t *r, uint64_t n) {
    if (r->err) return 0;
    if (r->len - r->pos < n) { r->err = ORC_ERR_TRUNCATED; return 0; }
    return 1;
}
static uint64_t rd_uint(rd_t *r, int n) {
    if (!rd_need(r, (uint64_t)n)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)r->p[r->pos + i] << (8 * i);
    r->pos += (uint64_t)n;
    return v;
}
static char *rd_str(rd_t *r) {
    uint64_t n = rd_uint(r, 8);
    if (r->err) return NULL;
    if (n > MAX_STRING_BYTES) { r->err = ORC_ERR_LENGTH; return NULL; }
    if (!rd_need(r, n)) return NULL;
    char *s = (char *)malloc(n + 1);
    memcpy(s, r->p + r->pos, n);
    s[n] = 0;
    r->pos += n;
    return s;
}
static void rd_value(rd_t *r, uint32_t type, orc_kv *kv, int depth) {
    if (depth > 16) { r->err = ORC_ERR_LENGTH; return; }
    switch (type) {
    case 0: case 1: kv->u = rd_uint(r, 1); if (type == 1) kv->u = (uint64_t)(int64_t)(int8_t)kv->u; break;
    case 2: case 3: kv->u = rd_uint(r, 2); if (type == 3) kv->u = (uint64_t)(int64_t)(int16_t)kv->u; break;
    case 4: case 5: kv->u = rd_uint(r, 4); if (type == 5) kv->u = (uint64_t)(int64_t)(int32_t)kv->u; break;
    case 6: { uint32_t b = (uint32_t)rd_uint(r, 4); float f; memcpy(&f, &b, 4); kv->f = f; break; }
    case 7: kv->u = rd_uint(r, 1); if (kv->u > 1) r->err = ORC_ERR_CONFIG; break;
    case 8: kv->s = rd_str(r); break;
    case 9: {
        uint32_t et = (uint32_t)rd_uint(r, 4);
        uint64_t n = rd_uint(r, 8);
        if (r->err) return;
        if (n > MAX_ARRAY_ITEMS) { r->err = ORC_ERR_LENGTH; return; }
        kv->is_array = 1;
        kv->u = n;
        for (uint64_t i = 0; i < n && !r->err; i++) {
            orc_kv tmp = {0};
            rd_value(r, et, &tmp, depth + 1);
            free(tmp.s);
        }
        break;
    }
    case 10: case 11: kv->u = rd_uint(r, 8); break;
    case 12: { uint64_t b = rd_uint(r, 8); double d; memcpy(&d, &b, 8); kv->f = d; break; }
    default: r->err = ORC_ERR_CONFIG; break;
    }
}

void orc_gguf_close(orc_gguf *g) {
    if (!g) return;
    for (uint64_t i = 0; i < g->n_kv; i++) { free(g->kv[i].key); free(g->kv[i].s); }
    for (uint64_t i = 0; i < g->n_tensors; i++) free(g->tensors[i].name);
    free(g->kv);
    free(g->tensors);
    free(g->bytes);
    free(g);
}

static const orc_kv *find_kv(const orc_gguf *g, const char *key) {
    for (uint64_t i = 0; i < g->n_kv; i++)
        if (g->kv[i].key && strcmp(g->kv[i].key, key) == 0) return &g->kv[i];
    return NULL;
}

int orc_gguf_open(const char *path, orc_gguf **out) {
    *out = NULL;
    FILE *f = fopen(path, "rb");
    if (!f) return ORC_ERR_IO;
    fseek(f, 0, SEEK_END);
    long flen = ftell(f);
    fseek(f, 0, SEEK_SET);
    orc_gguf *g = (orc_gguf *)calloc(1, sizeof(*g));
    g->len = (uint64_t)flen;
    g->bytes = (uint8_t *)malloc(g->len ? g->len : 1);
    if (fread(g->bytes, 1, g->len, f) != g->len) { fclose(f); orc_gguf_close(g); return ORC_ERR_IO; }
    fclose(f);
    rd_t r = {g->bytes, g->len, 0, 0};
    uint32_t magic = (uint32_t)rd_uint(&r, 4);
    if (r.err) { orc_gguf_close(g); return r.err; }
    if (magic != GGUF_MAGIC) { orc_gguf_close(g); return ORC_ERR_MAGIC; }
    g->version = (uint32_t)rd_uint(&r, 4);
    if (!r.err && g->version != 3) { orc_gguf_close(g); return ORC_ERR_VERSION; }
    uint64_t nt = rd_uint(&r, 8);
    if (!r.err && nt > MAX_TENSORS) r.err = ORC_ERR_LENGTH;
    uint64_t nkv = rd_uint(&r, 8);
    if (!r.err && nkv > MAX_ARRAY_ITEMS) r.err = ORC_ERR_LENGTH;
    if (r.err) { orc_gguf_close(g); return r.err; }
    g->kv = (orc_kv *)calloc(nkv ? nkv : 1, sizeof(orc_kv));
    for (uint64_t i = 0; i < nkv && !r.err; i++) {
        orc_kv *kv = &g->kv[i];
        kv->key = rd_str(&r);
        kv->type = (uint32_t)rd_uint(&r, 4);
        if (r.err) break;
        g->n_kv = i + 1;
        rd_value(&r, kv->type, kv, 0);
        for (uint64_t j = 0; j < i && !r.err; j++)
            if (strcmp(g->kv[j].key, kv->key) == 0) r.err = ORC_ERR_DUPLICATE_METADATA;
    }
    g->n_kv = nkv;
    if (r.err) { orc_gguf_close(g); return r.err; }
    g->tensors = (orc_tensor *)calloc(nt ? nt : 1, sizeof(orc_tensor));
    g->n_tensors = nt;
    for (uint64_t i = 0; i < nt && !r.err; i++) {
        orc_tensor *t = &g->tensors[i];
        t->name = rd_str(&r);
        t->ndims = (uint32_t)rd_uint(&r, 4);
        if (!r.err && t->ndims > 16) { r.err = ORC_ERR_DIMENSION; break; }
        for (uint32_t d = 0; d < t->ndims; d++) t->dims[d] = rd_uint(&r, 8);
        t->type = (uint32_t)rd_uint(&r, 4);
        t->offset = rd_uint(&r, 8);
    }
    if (r.err) { orc_gguf_close(g); return r.err; }
    uint64_t alignment = 32;
    const orc_kv *a = find_kv(g, "general.alignment");
    if (a && !a->is_array && a->type != 6 && a->type != 8 && a->type != 12) alignment = a->u;
    if (alignment == 0 || (alignment & (alignment - 1))) { orc_gguf_close(g); return ORC_ERR_ALIGNMENT; }
    uint64_t off = r.pos;
    if (off % alignment) off += alignment - off % alignment;
    if (off > g->len) { orc_gguf_close(g); return ORC_ERR_TRUNCATED; }
    g->data_offset = off;
    for (uint64_t i = 0; i < nt; i++)
        if (g->tensors[i].offset > g->len - off) { orc_gguf_close(g); return ORC_ERR_OFFSET; }
    *out = g;
    return ORC_OK;
}

uint32_t orc_gguf_version(const orc_gguf *g) { return g->version; }
uint64_t orc_gguf_tensor_count(const orc_gguf *g) { return g->n_tensors; }
uint64_t orc_gguf_data_offset(const orc_gguf *g) { return g->data_offset; }
const uint8_t *orc_gguf_bytes(const orc_gguf *g) { return g->bytes; }

int orc_gguf_get_u64(const orc_gguf *g, const char *key, uint64_t *out) {
    const orc_kv *kv = find_kv(g, key);
    if (!kv) return ORC_ERR_MISSING;
    if (kv->is_array || kv->type == 6 || kv->type == 8 || kv->type == 12) return ORC_ERR_CONFIG;
    *out = kv->u;
    return ORC_OK;
}
int orc_gguf_get_f32(const orc_gguf *g, const char *key, float *out) {
    const orc_kv *kv = find_kv(g, key);
    if (!kv) return ORC_ERR_MISSING;
    if (kv->type == 6 || kv->type == 12) { *out = (float)kv->f; return ORC_OK; }
    return ORC_ERR_CONFIG;
}
int orc_gguf_get_str(const orc_gguf *g, const char *key, char *out, size_t cap) {
    const orc_kv *kv = find_kv(g, key);
    if (!kv) return ORC_ERR_MISSING;
    if (kv->type != 8 || !kv->s) return ORC_ERR_CONFIG;
    snprintf(out, cap, "%s", kv->s);
    return ORC_OK;
}

/* tensor_data_range, lib.rs:337-360. */
int orc_gguf_tensor(const orc_gguf *g, const char *name, uint32_t *type, uint64_t *dims,
                    uint32_t *ndims, uint64_t *start, uint64_t *len) {
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const orc_tensor *t = &g->tensors[i];
        if (strcmp(t->name, name) != 0) continue;
        int64_t bl = orc_tensor_byte_len(t->type, t->dims, t->ndims);
        if (bl < 0) return (int)bl;
        uint64_t s = g->data_offset + t->offset;
        if (s + (uint64_t)bl > g->len) return ORC_ERR_OFFSET;
        if (type) *type = t->type;
        if (ndims) *ndims = t->ndims;
        if (dims) for (uint32_t d = 0; d < t->ndims && d < 4; d++) dims[d] = t->dims[d];
        if (start) *start = s;
        if (len) *len = (uint64_t)bl;
        return ORC_OK;
    }
    return ORC_ERR_MISSING;
}

/* ------------------------------------------------------------------------ */
/* gguf_gemv (nvidia/src/qwen_reference.rs:31-40) over encoded rows: each row
 * is block-dequantized (dequantize_block) then dotted in f32, sequentially. */
typedef struct {
    uint32_t t; const uint8_t *w; uint64_t k, r0, r1, row_bytes; const float *x; float *y;
} gemv_job;

static void *gemv_worker(void *arg) {
    gemv_job *j = (gemv_job *)arg;
    uint64_t be, bb;
    orc_tensor_layout(j->t, &be, &bb);
    float *buf = (float *)malloc(sizeof(float) * (size_t)be);
    for (uint64_t n = j->r0; n < j->r1; n++) {
        const uint8_t *row = j->w + n * j->row_bytes;
        float acc = 0.0f;
        for (uint64_t b = 0; b < j->k / be; b++) {
            orc_dequantize_block(j->t, row + b * bb, (size_t)bb, buf);
            const float *xb = j->x + b * be;
            for (uint64_t i = 0; i < be; i++) acc = acc + xb[i] * buf[i];
        }
        j->y[n] = acc;
    }
    free(buf);
    return NULL;
}

int orc_gemv_q(uint32_t t, const uint8_t *w, uint64_t rows, uint64_t k, const float *x, float *y,
               int threads) {
    uint64_t be, bb;
    if (orc_tensor_layout(t, &be, &bb) != ORC_OK) return ORC_ERR_UNSUPPORTED_TYPE;
    if (k % be) return ORC_ERR_DIMENSION;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    gemv_job jobs[64];
    pthread_t th[64];
    uint64_t per = (rows + (uint64_t)threads - 1) / (uint64_t)threads;
    for (int i = 0; i < threads; i++) {
        uint64_t r0 = per * (uint64_t)i, r1 = r0 + per;
        if (r0 > rows) r0 = rows;
        if (r1 > rows) r1 = rows;
        jobs[i] = (gemv_job){t, w, k, r0, r1, (k / be) * bb, x, y};
        if (threads == 1) gemv_worker(&jobs[i]);
        else pthread_create(&th[i], NULL, gemv_worker, &jobs[i]);
    }
    if (threads > 1) for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    return ORC_OK;
}

/* rms_norm_raw, qwen_reference.rs:550-556: x * (1/sqrt(sum/n + eps)) * w. */
void orc_rms_norm(const float *x, const float *w, float *y, int n, float eps) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum = sum + x[i] * x[i];
    float inv = 1.0f / sqrtf(sum / (float)n + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv * w[i];
}

/* NeoX half-split rope, qwen_reference.rs:406-425 / model_ops.rs:395-424:
 * pairs (p, p + rot/2), theta = pos * base^(-2p/rot); dims >= rot pass through. */
void orc_rope_neox(float *v, int heads, int hd, int rot, int64_t pos, float base) {
    int half = rot / 2;
    for (int h = 0; h < heads; h++) {
        float *b = v + (size_t)h * hd;
        for (int p = 0; p < half; p++) {
            float theta = (float)pos * powf(base, -(2.0f * (float)p) / (float)rot);
            float s = sinf(theta), c = cosf(theta);
            float x0 = b[p], x1 = b[p + half];
            b[p] = x0 * c - x1 * s;
            b[p + half] = x0 * s + x1 * c;
        }
    }
}

/* argmax, model_ops.rs:203-260: first maximum, NaN skipped; all-NaN -> 0. */
uint32_t orc_argmax(const float *l, int n) {
    uint32_t best = 0;
    int have = 0;
    float bv = 0.0f;
    for (int i = 0; i < n; i++) {
        float v = l[i];
        if (v != v) continue;
        if (!have || v > bv) { bv = v; best = (uint32_t)i; have = 1; }
    }
    return best;
}

/* ------------------------------------------------------------------------ */
/* Dense Qwen2/Qwen3 forward. Layer order follows the reference host step
 * (qwen_reference.rs:368-461 attention, :529-539 FFN) with the dense-Qwen
 * adaptations: no q|gate split and no sigmoid gate, rope over all of
 * head_dim, optional q/k/v bias (Qwen2) and optional q/k norm (Qwen3). */
typedef struct {
    float *attn_norm, *ffn_norm, *q_norm, *k_norm, *q_bias, *k_bias, *v_bias;
    uint32_t tq, tk, tv, to, tg, tu, td;
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    float *kcache, *vcache;
} orc_layer;

struct orc_qwen {
    orc_gguf *g;
    int hidden, layers, hq, hkv, hd, ffn, vocab, rot, max_ctx;
    float eps, base;
    uint32_t t_embd, t_out;
    const uint8_t *embd, *out;
    float *out_norm;
    orc_layer *L;
    int pos_next;
    int kv_round;
    int threads;   /* matvec worker threads (1 = the reference's host path); results do not depend on it */
    int intdot;    /* 1: projections in the integer-dot mode (Q8_1 activations) */
};

static int get_tensor(orc_gguf *g, const char *name, uint32_t *type, const uint8_t **ptr,
                      uint64_t *dims) {
    uint64_t start, len, d[4] = {0, 0, 0, 0};
    uint32_t nd;
    int r = orc_gguf_tensor(g, name, type, d, &nd, &start, &len);
    if (r) return r;
    *ptr = orc_gguf_bytes(g) + start;
    if (dims) memcpy(dims, d, sizeof(d));
    return 0;
}

static float *get_f32(orc_gguf *g, const char *name, uint64_t n, int required, int *err) {
    uint32_t t;
    const uint8_t *p;
    uint64_t d[4];
    int r = get_tensor(g, name, &t, &p, d);
    if (r) { if (required) *err = r; return NULL; }
    float *o = (float *)malloc(sizeof(float) * n);
    uint64_t be, bb;
    orc_tensor_layout(t, &be, &bb);
    if (d[0] != n || orc_dequantize(t, p, (size_t)(n / be * bb), o) != (int64_t)n) {
        free(o);
        *err = ORC_ERR_CONFIG;
        return NULL;
    }
    return o;
}

void orc_qwen_close(orc_qwen *m) {
    if (!m) return;
    if (m->L) {
        for (int l = 0; l < m->layers; l++) {
            orc_layer *y = &m->L[l];
            free(y->attn_norm); free(y->ffn_norm); free(y->q_norm); free(y->k_norm);
            free(y->q_bias); free(y->k_bias); free(y->v_bias); free(y->kcache); free(y->vcache);
        }
        free(m->L);
    }
    free(m->out_norm);
    orc_gguf_close(m->g);
    free(m);
}

int orc_qwen_open(const char *path, int max_ctx, orc_qwen **out) {
    *out = NULL;
    orc_gguf *g;
    int r = orc_gguf_open(path, &g);
    if (r) return r;
    orc_qwen *m = (orc_qwen *)calloc(1, sizeof(*m));
    m->g = g;
    char arch[64];
    if (orc_gguf_get_str(g, "general.architecture", arch, sizeof arch)) { orc_qwen_close(m); return ORC_ERR_CONFIG; }
    if (strcmp(arch, "qwen2") && strcmp(arch, "qwen3")) { orc_qwen_close(m); return ORC_ERR_CONFIG; }
    char key[160];
    uint64_t v;
#define U(field, suffix) \
    snprintf(key, sizeof key, "%s.%s", arch, suffix); \
    if (orc_gguf_get_u64(g, key, &v)) { orc_qwen_close(m); return ORC_ERR_CONFIG; } \
    m->field = (int)v;
    U(hidden, "embedding_length");
    U(layers, "block_count");
    U(hq, "attention.head_count");
    U(hkv, "attention.head_count_kv");
    U(ffn, "feed_forward_length");
#undef U
    snprintf(key, sizeof key, "%s.attention.key_length", arch);
    m->hd = orc_gguf_get_u64(g, key, &v) ? m->hidden / m->hq : (int)v;
    snprintf(key, sizeof key, "%s.rope.dimension_count", arch);
    m->rot = orc_gguf_get_u64(g, key, &v) ? m->hd : (int)v;
    snprintf(key, sizeof key, "%s.attention.layer_norm_rms_epsilon", arch);
    if (orc_gguf_get_f32(g, key, &m->eps)) m->eps = 1e-6f;
    snprintf(key, sizeof key, "%s.rope.freq_base", arch);
    if (orc_gguf_get_f32(g, key, &m->base)) m->base = 10000.0f;
    m->max_ctx = max_ctx;
    uint64_t d[4];
    if (get_tensor(g, "token_embd.weight", &m->t_embd, &m->embd, d)) { orc_qwen_close(m); return ORC_ERR_MISSING; }
    m->vocab = (int)d[1];
    if (get_tensor(g, "output.weight", &m->t_out, &m->out, NULL)) { m->t_out = m->t_embd; m->out = m->embd; }
    int err = 0;
    m->out_norm = get_f32(g, "output_norm.weight", (uint64_t)m->hidden, 1, &err);
    m->L = (orc_layer *)calloc((size_t)m->layers, sizeof(orc_layer));
    int qd = m->hq * m->hd, kd = m->hkv * m->hd;
    for (int l = 0; l < m->layers && !err; l++) {
        orc_layer *y = &m->L[l];
        char n[128];
#define T(field, tfield, nm) snprintf(n, sizeof n, "blk.%d.%s.weight", l, nm); \
        if (get_tensor(g, n, &y->tfield, &y->field, NULL)) err = ORC_ERR_MISSING;
        T(wq, tq, "attn_q"); T(wk, tk, "attn_k"); T(wv, tv, "attn_v"); T(wo, to, "attn_output");
        T(wg, tg, "ffn_gate"); T(wu, tu, "ffn_up"); T(wd, td, "ffn_down");
#undef T
        snprintf(n, sizeof n, "blk.%d.attn_norm.weight", l);
        y->attn_norm = get_f32(g, n, (uint64_t)m->hidden, 1, &err);
        snprintf(n, sizeof n, "blk.%d.ffn_norm.weight", l);
        y->ffn_norm = get_f32(g, n, (uint64_t)m->hidden, 1, &err);
        snprintf(n, sizeof n, "blk.%d.attn_q_norm.weight", l);
        y->q_norm = get_f32(g, n, (uint64_t)m->hd, 0, &err);
        snprintf(n, sizeof n, "blk.%d.attn_k_norm.weight", l);
        y->k_norm = get_f32(g, n, (uint64_t)m->hd, 0, &err);
        snprintf(n, sizeof n, "blk.%d.attn_q.bias", l);
        y->q_bias = get_f32(g, n, (uint64_t)qd, 0, &err);
        snprintf(n, sizeof n, "blk.%d.attn_k.bias", l);
        y->k_bias = get_f32(g, n, (uint64_t)kd, 0, &err);
        snprintf(n, sizeof n, "blk.%d.attn_v.bias", l);
        y->v_bias = get_f32(g, n, (uint64_t)kd, 0, &err);
        y->kcache = (float *)calloc((size_t)max_ctx * (size_t)kd, sizeof(float));
        y->vcache = (float *)calloc((size_t)max_ctx * (size_t)kd, sizeof(float));
    }
    if (err) { orc_qwen_close(m); return err; }
    *out = m;
    return ORC_OK;
}

void orc_qwen_config(const orc_qwen *m, int32_t *c, float *eps, float *base) {
    c[0] = m->hidden; c[1] = m->layers; c[2] = m->hq; c[3] = m->hkv;
    c[4] = m->hd; c[5] = m->ffn; c[6] = m->vocab; c[7] = m->rot;
    if (eps) *eps = m->eps;
    if (base) *base = m->base;
}

void orc_qwen_reset(orc_qwen *m) { m->pos_next = 0; }
void orc_qwen_set_kv_round(orc_qwen *m, int mode) { m->kv_round = mode; }

/* binary32 -> binary16 -> binary32 with round-to-nearest-even (finite inputs;
 * overflow saturates to inf). */
float orc_round_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = u & 0x80000000u, ax = u & 0x7fffffffu;
    if (ax >= 0x7f800000u) return x;
    float a;
    memcpy(&a, &ax, 4);
    float r;
    if (a >= 65520.0f) r = INFINITY;
    else if (a < ldexpf(1.0f, -14)) {
        /* subnormal range: quantum 2^-24 */
        r = rintf(a * 16777216.0f) / 16777216.0f;
    } else {
        int e;
        frexpf(a, &e);                    /* a in [2^(e-1), 2^e) */
        float q = ldexpf(1.0f, e - 11);   /* 10 fraction bits */
        r = rintf(a / q) * q;
    }
    uint32_t rb;
    memcpy(&rb, &r, 4);
    rb |= sign;
    memcpy(&r, &rb, 4);
    return r;
}
float orc_round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}
static void kv_round(float *v, int n, int mode) {
    if (mode == 1) for (int i = 0; i < n; i++) v[i] = orc_round_f16(v[i]);
    else if (mode == 2) for (int i = 0; i < n; i++) v[i] = orc_round_bf16(v[i]);
}

static int g_qwen_threads = 1;   /* set per call from the model being stepped */
static int g_qwen_intdot = 0;
/* One projection. In the integer-dot mode the input is packed to Q8_1 first and
 * the projection runs on the packed words (CudaIntDotProjector::project,
 * nvidia/src/decode.rs:1441-1497; every type of these models has an
 * integer-dot kernel, so there is no float fallback here). */
static void gemv(uint32_t t, const uint8_t *w, int rows, int k, const float *x, float *y) {
    if (g_qwen_intdot && (t == 8 || t == 12 || t == 14)) {
        uint32_t *pk = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(k / 32) * 9);
        orc_quantize_q8_1(x, (uint64_t)k, pk);
        orc_gemv_q8_1(t, w, (uint64_t)rows, (uint64_t)k, pk, 1, y, g_qwen_threads);
        free(pk);
        return;
    }
    orc_gemv_q(t, w, (uint64_t)rows, (uint64_t)k, x, y, g_qwen_threads);
}

void orc_qwen_set_gemv_mode(orc_qwen *m, int mode) { m->intdot = mode == ORC_GEMV_INT_DOT; }

void orc_qwen_set_threads(orc_qwen *m, int threads) { m->threads = threads < 1 ? 1 : threads > 64 ? 64 : threads; }

static int qwen_step(orc_qwen *m, uint32_t token, int pos, float *logits, float *trace, float *fnorm,
                     int kv_only) {
    if (pos != m->pos_next || pos >= m->max_ctx || (int)token >= m->vocab) return ORC_ERR_CONFIG;
    g_qwen_threads = m->threads > 0 ? m->threads : 1;
    g_qwen_intdot = m->intdot;
    int H = m->hidden, hd = m->hd, qd = m->hq * hd, kd = m->hkv * hd, F = m->ffn;
    float *h = (float *)malloc(sizeof(float) * H), *xn = (float *)malloc(sizeof(float) * H);
    float *q = (float *)malloc(sizeof(float) * qd), *k = (float *)malloc(sizeof(float) * kd);
    float *v = (float *)malloc(sizeof(float) * kd), *att = (float *)malloc(sizeof(float) * qd);
    float *o = (float *)malloc(sizeof(float) * H), *gt = (float *)malloc(sizeof(float) * F);
    float *up = (float *)malloc(sizeof(float) * F), *sc = (float *)malloc(sizeof(float) * (pos + 1));
    float *tmp = (float *)malloc(sizeof(float) * hd);
    /* embedding row: dequantize row `token` of token_embd (ne0 = hidden) */
    uint64_t be, bb;
    orc_tensor_layout(m->t_embd, &be, &bb);
    orc_dequantize(m->t_embd, m->embd + (uint64_t)token * (H / be) * bb, (size_t)(H / be * bb), h);
    if (trace) memcpy(trace, h, sizeof(float) * H);
    float scale = 1.0f / sqrtf((float)hd);
    int group = m->hq / m->hkv;
    for (int l = 0; l < m->layers; l++) {
        orc_layer *y = &m->L[l];
        orc_rms_norm(h, y->attn_norm, xn, H, m->eps);
        const int last_kv = kv_only && l == m->layers - 1;   /* q is not needed */
        if (!last_kv) gemv(y->tq, y->wq, qd, H, xn, q);
        gemv(y->tk, y->wk, kd, H, xn, k);
        gemv(y->tv, y->wv, kd, H, xn, v);
        if (y->q_bias && !last_kv) for (int i = 0; i < qd; i++) q[i] = q[i] + y->q_bias[i];
        if (y->k_bias) for (int i = 0; i < kd; i++) k[i] = k[i] + y->k_bias[i];
        if (y->v_bias) for (int i = 0; i < kd; i++) v[i] = v[i] + y->v_bias[i];
        if (y->q_norm && !last_kv)
            for (int hh = 0; hh < m->hq; hh++) {
                orc_rms_norm(q + hh * hd, y->q_norm, tmp, hd, m->eps);
                memcpy(q + hh * hd, tmp, sizeof(float) * hd);
            }
        if (y->k_norm)
            for (int hh = 0; hh < m->hkv; hh++) {
                orc_rms_norm(k + hh * hd, y->k_norm, tmp, hd, m->eps);
                memcpy(k + hh * hd, tmp, sizeof(float) * hd);
            }
        if (!last_kv) orc_rope_neox(q, m->hq, hd, m->rot, pos, m->base);
        orc_rope_neox(k, m->hkv, hd, m->rot, pos, m->base);
        memcpy(y->kcache + (size_t)pos * kd, k, sizeof(float) * kd);
        memcpy(y->vcache + (size_t)pos * kd, v, sizeof(float) * kd);
        kv_round(y->kcache + (size_t)pos * kd, kd, m->kv_round);
        kv_round(y->vcache + (size_t)pos * kd, kd, m->kv_round);
        if (kv_only && l == m->layers - 1) break;   /* nothing after the last cache append is needed */
        int tokens = pos + 1;
        for (int qh = 0; qh < m->hq; qh++) {
            int kh = qh / group;
            const float *qv = q + qh * hd;
            float mx = -INFINITY;
            for (int t = 0; t < tokens; t++) {
                const float *kk = y->kcache + ((size_t)t * m->hkv + kh) * hd;
                float s = 0.0f;
                for (int i = 0; i < hd; i++) s = s + qv[i] * kk[i];
                sc[t] = s * scale;
                if (sc[t] > mx) mx = sc[t];
            }
            float total = 0.0f;
            for (int t = 0; t < tokens; t++) { sc[t] = expf(sc[t] - mx); total = total + sc[t]; }
            float *ao = att + qh * hd;
            for (int i = 0; i < hd; i++) ao[i] = 0.0f;
            for (int t = 0; t < tokens; t++) {
                const float *vv = y->vcache + ((size_t)t * m->hkv + kh) * hd;
                float wgt = sc[t] / total;
                for (int i = 0; i < hd; i++) ao[i] = ao[i] + wgt * vv[i];
            }
        }
        gemv(y->to, y->wo, H, qd, att, o);
        for (int i = 0; i < H; i++) h[i] = h[i] + o[i];
        orc_rms_norm(h, y->ffn_norm, xn, H, m->eps);
        gemv(y->tg, y->wg, F, H, xn, gt);
        gemv(y->tu, y->wu, F, H, xn, up);
        for (int i = 0; i < F; i++) gt[i] = gt[i] / (1.0f + expf(-gt[i])) * up[i];
        gemv(y->td, y->wd, H, F, gt, o);
        for (int i = 0; i < H; i++) h[i] = h[i] + o[i];
        if (trace) memcpy(trace + (size_t)(l + 1) * H, h, sizeof(float) * H);
    }
    if (!kv_only) {
        orc_rms_norm(h, m->out_norm, xn, H, m->eps);
        if (fnorm) memcpy(fnorm, xn, sizeof(float) * H);
        if (logits) gemv(m->t_out, m->out, m->vocab, H, xn, logits);
    }
    m->pos_next = pos + 1;
    free(h); free(xn); free(q); free(k); free(v); free(att); free(o); free(gt); free(up);
    free(sc); free(tmp);
    return ORC_OK;
}

int orc_qwen_step(orc_qwen *m, uint32_t token, int pos, float *logits, float *trace, float *fnorm) {
    return qwen_step(m, token, pos, logits, trace, fnorm, 0);
}

int orc_qwen_append_kv(orc_qwen *m, uint32_t token, int pos) {
    return qwen_step(m, token, pos, NULL, NULL, NULL, 1);
}

/* ------------------------------------------------------------------------ */
/* Integer-dot projections: the reference's experimental GemvMode::IntegerDot
 * (nvidia/src/decode.rs:298-312), lossy by design. */

/* Bits of a value already representable in binary16 (finite, or +-inf). */
static uint16_t f16_bits(float r) {
    uint32_t u;
    memcpy(&u, &r, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    float a = fabsf(r);
    if (a == 0.0f) return sign;
    if (isinf(a)) return (uint16_t)(sign | 0x7c00u);
    if (a < ldexpf(1.0f, -14)) return (uint16_t)(sign | (uint16_t)(a * 16777216.0f));
    int e;
    float f = frexpf(a, &e);   /* a = f 2^e, f in [0.5, 1) */
    uint16_t mant = (uint16_t)((f * 2.0f - 1.0f) * 1024.0f);
    return (uint16_t)(sign | (uint16_t)((e - 1 + 15) << 10) | mant);
}

/* quantize_q8_1 (nvidia/src/activation.cu:1-28): per 32 values, d = max|x| /
 * 127, q = round-half-away(x / d) (0 when the block is all zero), word 0 =
 * half(d) | half(sum) << 16 (round to nearest even), words 1..8 = q as signed
 * bytes, little endian. The sum follows the warp's xor butterfly (offsets 16,
 * 8, 4, 2, 1): lane 0 ends with ((..(x0 + x16) + (x8 + x24)) ..). */
int orc_quantize_q8_1(const float *x, uint64_t n, uint32_t *out) {
    if (n == 0 || n % 32) return ORC_ERR_DIMENSION;
    for (uint64_t b = 0; b < n / 32; b++) {
        const float *v = x + b * 32;
        float s[32], mx = 0.0f;
        for (int i = 0; i < 32; i++) { s[i] = v[i]; mx = fmaxf(mx, fabsf(v[i])); }
        for (int off = 16; off > 0; off >>= 1)
            for (int i = 0; i < off; i++) s[i] = s[i] + s[i + off];
        const float d = mx / 127.0f;
        uint32_t *w = out + b * 9;
        w[0] = (uint32_t)f16_bits(orc_round_f16(d)) | ((uint32_t)f16_bits(orc_round_f16(s[0])) << 16);
        for (int j = 0; j < 8; j++) {
            uint32_t word = 0;
            for (int i = 0; i < 4; i++) {
                const int q = mx == 0.0f ? 0 : (int)roundf(v[4 * j + i] / d);
                word |= ((uint32_t)q & 0xffu) << (8 * i);
            }
            w[1 + j] = word;
        }
    }
    return ORC_OK;
}

/* One output of the integer-dot matvec for one packed input (`nb` blocks of
 * the row, `act` = K/32 nine-word Q8_1 blocks), in exact binary64 arithmetic:
 * the value every kernel ordering approximates.
 *   Q4_K (q4_k_q8_1.cu:40-81):  sum_g (d sc_g) da_g dot_g - (dmin m_g) S_g
 *   Q6_K (q6_k_q8_1.cu:37-90):  sum_h (d sc_h) da dot(q6 + 32 ... ) with the
 *                               bias removed through the packed byte sums,
 *                               i.e. sum_h (d sc_h) da (dot_h - 32 A_h)
 *   Q8_0 (q8_0_q8_1.cu:27-55):  sum_b d_b da_b dot_b
 * with da, S the half-precision scale and sum of the Q8_1 block. */
static double intdot_row(uint32_t t, const uint8_t *row, uint64_t k, const uint32_t *act) {
    double acc = 0.0;
    if (t == 8) {
        for (uint64_t b = 0; b < k / 32; b++) {
            const uint8_t *e = row + b * 34;
            const uint32_t *a = act + b * 9;
            int dot = 0;
            for (int i = 0; i < 32; i++) dot += (int)(int8_t)e[2 + i] * (int)(int8_t)(a[1 + i / 4] >> (8 * (i % 4)));
            acc += (double)rd_f16(e) * (double)orc_f16_to_f32((uint16_t)a[0]) * (double)dot;
        }
        return acc;
    }
    for (uint64_t b = 0; b < k / 256; b++) {
        if (t == 12) {
            const uint8_t *e = row + b * 144;
            const double d = rd_f16(e), dmin = rd_f16(e + 2);
            uint8_t sc[8], mn[8];
            q4k_scales(e + 4, sc, mn);
            for (int g = 0; g < 8; g++) {
                const uint32_t *a = act + (b * 8 + (uint64_t)g) * 9;
                int dot = 0;
                for (int i = 0; i < 32; i++) {
                    const int q = (e[16 + (g / 2) * 32 + i] >> ((g % 2) * 4)) & 15;
                    dot += q * (int)(int8_t)(a[1 + i / 4] >> (8 * (i % 4)));
                }
                const double da = orc_f16_to_f32((uint16_t)a[0]), S = orc_f16_to_f32((uint16_t)(a[0] >> 16));
                acc += d * sc[g] * da * (double)dot - dmin * mn[g] * S;
            }
        } else {
            const uint8_t *e = row + b * 210;
            const double d = rd_f16(e + 208);
            for (int g = 0; g < 8; g++) {
                const uint32_t *a = act + (b * 8 + (uint64_t)g) * 9;
                const double da = orc_f16_to_f32((uint16_t)a[0]);
                const int chunk = g / 4, variant = g % 4;
                for (int half = 0; half < 2; half++) {
                    int dot = 0, asum = 0;
                    for (int i = 0; i < 16; i++) {
                        const int pos = half * 16 + i;
                        const int lo = (e[chunk * 64 + (variant % 2) * 32 + pos] >> (variant < 2 ? 0 : 4)) & 15;
                        const int hi = (e[128 + chunk * 32 + pos] >> (2 * variant)) & 3;
                        const int qa = (int)(int8_t)(a[1 + pos / 4] >> (8 * (pos % 4)));
                        dot += (lo | (hi << 4)) * qa;
                        asum += qa;
                    }
                    acc += d * (double)(int8_t)e[192 + g * 2 + half] * da * (double)(dot - 32 * asum);
                }
            }
        }
    }
    return acc;
}

typedef struct {
    uint32_t t; const uint8_t *w; uint64_t k, rows, r0, r1, row_bytes; const uint32_t *pk; uint32_t members; float *y;
} intdot_job;

static void *intdot_worker(void *arg) {
    intdot_job *j = (intdot_job *)arg;
    for (uint32_t m = 0; m < j->members; m++)
        for (uint64_t n = j->r0; n < j->r1; n++)
            j->y[(uint64_t)m * j->rows + n] =
                (float)intdot_row(j->t, j->w + n * j->row_bytes, j->k, j->pk + (uint64_t)m * (j->k / 32) * 9);
    return NULL;
}

/* y[m][n] for `members` packed inputs (batch-major, K/32 * 9 words each), the
 * batched variant reading each weight row once for every member
 * (q4_k_q8_1_gemv_batch, q4_k_q8_1.cu:86-140). */
int orc_gemv_q8_1(uint32_t t, const uint8_t *w, uint64_t rows, uint64_t k, const uint32_t *packed,
                  uint32_t members, float *y, int threads) {
    uint64_t be, bb;
    if (t != 8 && t != 12 && t != 14) return ORC_ERR_UNSUPPORTED_TYPE;
    orc_tensor_layout(t, &be, &bb);
    if (k == 0 || k % be || members == 0) return ORC_ERR_DIMENSION;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    intdot_job jobs[64];
    pthread_t th[64];
    uint64_t per = (rows + (uint64_t)threads - 1) / (uint64_t)threads;
    for (int i = 0; i < threads; i++) {
        uint64_t r0 = per * (uint64_t)i, r1 = r0 + per;
        if (r0 > rows) r0 = rows;
        if (r1 > rows) r1 = rows;
        jobs[i] = (intdot_job){t, w, k, rows, r0, r1, (k / be) * bb, packed, members, y};
        if (threads == 1) intdot_worker(&jobs[i]);
        else pthread_create(&th[i], NULL, intdot_worker, &jobs[i]);
    }
    if (threads > 1) for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    return ORC_OK;
}
