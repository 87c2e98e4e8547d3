/* qwen35 hybrid decoder (Gated-DeltaNet recurrent layers + gated full-attention
 * layers) -- TEST INFRASTRUCTURE ONLY, the checker of the GPU hybrid path.
 *
 * A plain-C restatement of the reference's host equations, in their arithmetic
 * order, generalized from the pinned 27B geometry to any geometry a qwen35
 * GGUF declares:
 *   gguf_gemv                    crates/nvidia/src/qwen_reference.rs:31-40
 *   l2_normalize, softplus       qwen_reference.rs:44-59
 *   gdn_state_step               qwen_reference.rs:61-103
 *   gdn_conv_step                qwen_reference.rs:105-134
 *   host_gdn_ar_step_traced      qwen_reference.rs:199-281
 *   host_full_attn_ar_step       qwen_reference.rs:370-480 (gated q, partial NeoX rope)
 *   host_ffn_step, rms_norm_raw  qwen_reference.rs:505-556
 *   layer wiring and head        crates/nvidia/src/decode.rs:550-700 (attn_norm ->
 *                                GDN or attention (+residual) -> post_attention_norm ->
 *                                SwiGLU FFN (+residual); output_norm -> output -> argmax)
 *   layer schedule               crates/qwen/src/gguf/config.rs:93-128: layer i is full
 *                                attention when (i + 1) is a multiple of
 *                                full_attention_interval, recurrent otherwise
 * Built with -ffp-contract=off like the rest of the oracle. Pinned by an
 * independent FP64 numpy forward of the same equations (tests/test_qwen35_oracle.py)
 * and by the reference's chunked-versus-recurrent identity for the delta rule
 * (crates/nvidia/tests/gdn_chunk_reference.rs). */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int recurrent;
    float *attn_norm, *post_norm;
    uint32_t tg, tu, td;
    const uint8_t *wg, *wu, *wd;
    /* recurrent */
    uint32_t tqkv, tz, tbeta, talpha, tout;
    const uint8_t *wqkv, *wz, *wbeta, *walpha, *wout;
    float *dt_bias, *ssm_a, *conv_w, *ssm_norm;
    float *state, *conv;    /* [hv][d][d], [C][conv - 1] */
    /* full attention */
    uint32_t tq, tk, tv, to;
    const uint8_t *wq, *wk, *wv, *wo;
    float *q_norm, *k_norm;
    float *kcache, *vcache;
} q35_layer;

struct orc_q35 {
    orc_gguf *g;
    int hidden, layers, hq, hkv, hd, ffn, vocab, rot, max_ctx, interval;
    int hk, hv, d, conv_k, channels, inner;
    float eps, base;
    uint32_t t_embd, t_out;
    const uint8_t *embd, *out;
    float *out_norm;
    q35_layer *L;
    int pos_next;
    int kv_round;
};

static int tensor(orc_gguf *g, const char *name, uint32_t *type, const uint8_t **ptr, uint64_t *dims) {
    uint32_t nd;
    uint64_t d[4] = {0, 0, 0, 0}, start, len;
    int r = orc_gguf_tensor(g, name, type, d, &nd, &start, &len);
    if (r) return r;
    *ptr = orc_gguf_bytes(g) + start;
    if (dims) memcpy(dims, d, sizeof d);
    return 0;
}

static float *f32vec(orc_gguf *g, const char *name, uint64_t n, int *err) {
    uint32_t t;
    const uint8_t *p;
    uint64_t d[4];
    if (tensor(g, name, &t, &p, d) || t != 0) { *err = ORC_ERR_MISSING; return NULL; }
    uint64_t total = d[0] * (d[1] ? d[1] : 1);
    if (total != n) { *err = ORC_ERR_DIMENSION; return NULL; }
    float *v = (float *)malloc(sizeof(float) * n);
    memcpy(v, p, sizeof(float) * n);
    return v;
}

static void gemv(uint32_t t, const uint8_t *w, int rows, int k, const float *x, float *y) {
    orc_gemv_q(t, w, (uint64_t)rows, (uint64_t)k, x, y, 1);
}

void orc_q35_close(orc_q35 *m) {
    if (!m) return;
    if (m->L) {
        for (int l = 0; l < m->layers; l++) {
            q35_layer *y = &m->L[l];
            free(y->attn_norm); free(y->post_norm); free(y->dt_bias); free(y->ssm_a); free(y->conv_w);
            free(y->ssm_norm); free(y->state); free(y->conv); free(y->q_norm); free(y->k_norm);
            free(y->kcache); free(y->vcache);
        }
        free(m->L);
    }
    free(m->out_norm);
    if (m->g) orc_gguf_close(m->g);
    free(m);
}

int orc_q35_open(const char *path, int max_ctx, orc_q35 **out) {
    *out = NULL;
    orc_gguf *g;
    int r = orc_gguf_open(path, &g);
    if (r) return r;
    orc_q35 *m = (orc_q35 *)calloc(1, sizeof(*m));
    m->g = g;
    char arch[64];
    if (orc_gguf_get_str(g, "general.architecture", arch, sizeof arch) || strcmp(arch, "qwen35")) {
        orc_q35_close(m);
        return ORC_ERR_CONFIG;
    }
    uint64_t v;
#define U(field, key) if (orc_gguf_get_u64(g, "qwen35." key, &v)) { orc_q35_close(m); return ORC_ERR_CONFIG; } m->field = (int)v;
    U(hidden, "embedding_length");
    U(layers, "block_count");
    U(hq, "attention.head_count");
    U(hkv, "attention.head_count_kv");
    U(hd, "attention.key_length");
    U(ffn, "feed_forward_length");
    U(hk, "ssm.group_count");
    U(hv, "ssm.time_step_rank");
    U(d, "ssm.state_size");
    U(inner, "ssm.inner_size");
    U(conv_k, "ssm.conv_kernel");
#undef U
    m->rot = orc_gguf_get_u64(g, "qwen35.rope.dimension_count", &v) ? m->hd : (int)v;
    m->interval = orc_gguf_get_u64(g, "qwen35.full_attention_interval", &v) ? 4 : (int)v;
    if (orc_gguf_get_f32(g, "qwen35.attention.layer_norm_rms_epsilon", &m->eps)) { orc_q35_close(m); return ORC_ERR_CONFIG; }
    if (orc_gguf_get_f32(g, "qwen35.rope.freq_base", &m->base)) m->base = 10000.0f;
    if (m->inner != m->hv * m->d || m->hv % m->hk || m->interval < 1 || m->conv_k < 2) {
        orc_q35_close(m);
        return ORC_ERR_CONFIG;
    }
    m->channels = 2 * m->hk * m->d + m->hv * m->d;
    m->max_ctx = max_ctx;
    uint64_t d4[4];
    if (tensor(g, "token_embd.weight", &m->t_embd, &m->embd, d4)) { orc_q35_close(m); return ORC_ERR_MISSING; }
    m->vocab = (int)d4[1];
    if (tensor(g, "output.weight", &m->t_out, &m->out, NULL)) { m->t_out = m->t_embd; m->out = m->embd; }
    int err = 0;
    m->out_norm = f32vec(g, "output_norm.weight", (uint64_t)m->hidden, &err);
    m->L = (q35_layer *)calloc((size_t)m->layers, sizeof(q35_layer));
    char n[160];
    for (int l = 0; l < m->layers && !err; l++) {
        q35_layer *y = &m->L[l];
        y->recurrent = (l + 1) % m->interval != 0;
#define T(tf, wf, nm) snprintf(n, sizeof n, "blk.%d." nm, l); if (tensor(g, n, &y->tf, &y->wf, NULL)) err = ORC_ERR_MISSING;
#define V(f, nm, cnt) snprintf(n, sizeof n, "blk.%d." nm, l); y->f = f32vec(g, n, (uint64_t)(cnt), &err);
        V(attn_norm, "attn_norm.weight", m->hidden);
        V(post_norm, "post_attention_norm.weight", m->hidden);
        T(tg, wg, "ffn_gate.weight"); T(tu, wu, "ffn_up.weight"); T(td, wd, "ffn_down.weight");
        if (y->recurrent) {
            T(tqkv, wqkv, "attn_qkv.weight"); T(tz, wz, "attn_gate.weight");
            T(tbeta, wbeta, "ssm_beta.weight"); T(talpha, walpha, "ssm_alpha.weight");
            T(tout, wout, "ssm_out.weight");
            V(dt_bias, "ssm_dt.bias", m->hv);
            V(ssm_a, "ssm_a", m->hv);
            V(conv_w, "ssm_conv1d.weight", (uint64_t)m->conv_k * m->channels);
            V(ssm_norm, "ssm_norm.weight", m->d);
            y->state = (float *)calloc((size_t)m->hv * m->d * m->d, sizeof(float));
            y->conv = (float *)calloc((size_t)m->channels * (m->conv_k - 1), sizeof(float));
        } else {
            T(tq, wq, "attn_q.weight"); T(tk, wk, "attn_k.weight"); T(tv, wv, "attn_v.weight");
            T(to, wo, "attn_output.weight");
            V(q_norm, "attn_q_norm.weight", m->hd);
            V(k_norm, "attn_k_norm.weight", m->hd);
            y->kcache = (float *)calloc((size_t)max_ctx * m->hkv * m->hd, sizeof(float));
            y->vcache = (float *)calloc((size_t)max_ctx * m->hkv * m->hd, sizeof(float));
        }
#undef T
#undef V
    }
    if (err) { orc_q35_close(m); return err; }
    *out = m;
    return ORC_OK;
}

void orc_q35_config(const orc_q35 *m, int32_t *c) {
    c[0] = m->hidden; c[1] = m->layers; c[2] = m->hq; c[3] = m->hkv; c[4] = m->hd; c[5] = m->ffn;
    c[6] = m->vocab; c[7] = m->rot; c[8] = m->hk; c[9] = m->hv; c[10] = m->d; c[11] = m->interval;
}

void orc_q35_reset(orc_q35 *m) {
    m->pos_next = 0;
    for (int l = 0; l < m->layers; l++) {
        q35_layer *y = &m->L[l];
        if (y->recurrent) {
            memset(y->state, 0, sizeof(float) * (size_t)m->hv * m->d * m->d);
            memset(y->conv, 0, sizeof(float) * (size_t)m->channels * (m->conv_k - 1));
        }
    }
}

void orc_q35_set_kv_round(orc_q35 *m, int mode) { m->kv_round = mode; }

/* l2_normalize (qwen_reference.rs:44-49): x / max(sqrt(sum x^2), eps) */
static void l2_normalize(float *x, int n, float eps) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum = sum + x[i] * x[i];
    float nrm = sqrtf(sum);
    float scale = 1.0f / (nrm > eps ? nrm : eps);
    for (int i = 0; i < n; i++) x[i] = x[i] * scale;
}

/* softplus with the large-input shortcut (qwen_reference.rs:52-59) */
static float softplus(float v) { return v > 20.0f ? v : logf(1.0f + expf(v)); }

/* gdn_state_step (qwen_reference.rs:61-103): S *= decay; sk = S^T k;
 * d = (v - sk) beta; S += k d^T; o = (S^T q) / sqrt(head_dim). S row-major [k row][v col]. */
static void state_step(float *S, const float *k, const float *v, const float *q, float decay, float beta, int kd,
                       int vd, float *o, float *sk, float *dv) {
    for (int i = 0; i < kd * vd; i++) S[i] = S[i] * decay;
    for (int c = 0; c < vd; c++) sk[c] = 0.0f;
    for (int r = 0; r < kd; r++)
        for (int c = 0; c < vd; c++) sk[c] = sk[c] + S[r * vd + c] * k[r];
    for (int c = 0; c < vd; c++) dv[c] = (v[c] - sk[c]) * beta;
    for (int r = 0; r < kd; r++)
        for (int c = 0; c < vd; c++) S[r * vd + c] = S[r * vd + c] + k[r] * dv[c];
    const float scale = 1.0f / sqrtf((float)kd);
    for (int c = 0; c < vd; c++) {
        float acc = 0.0f;
        for (int r = 0; r < kd; r++) acc = acc + S[r * vd + c] * q[r];
        o[c] = acc * scale;
    }
}

static void kv_round(float *v, int n, int mode) {
    if (mode == 1) for (int i = 0; i < n; i++) v[i] = orc_round_f16(v[i]);
    else if (mode == 2) for (int i = 0; i < n; i++) v[i] = orc_round_bf16(v[i]);
}

/* one recurrent layer's attention block: returns ssm_out(gated) in `out` (host_gdn_ar_step_traced) */
static void gdn_block(orc_q35 *m, q35_layer *y, const float *xn, float *out) {
    const int C = m->channels, hd = m->d, HK = m->hk, HV = m->hv, KC = m->conv_k;
    float *mixed = (float *)malloc(sizeof(float) * C), *z = (float *)malloc(sizeof(float) * m->inner);
    float *beta = (float *)malloc(sizeof(float) * HV), *gate = (float *)malloc(sizeof(float) * HV);
    float *act = (float *)malloc(sizeof(float) * C), *o = (float *)malloc(sizeof(float) * m->inner);
    float *gated = (float *)malloc(sizeof(float) * m->inner);
    float *sk = (float *)malloc(sizeof(float) * hd), *dv = (float *)malloc(sizeof(float) * hd);
    gemv(y->tqkv, y->wqkv, C, m->hidden, xn, mixed);
    gemv(y->tz, y->wz, m->inner, m->hidden, xn, z);
    gemv(y->tbeta, y->wbeta, HV, m->hidden, xn, beta);
    for (int h = 0; h < HV; h++) beta[h] = 1.0f / (1.0f + expf(-beta[h]));
    gemv(y->talpha, y->walpha, HV, m->hidden, xn, gate);
    for (int h = 0; h < HV; h++) gate[h] = softplus(gate[h] + y->dt_bias[h]) * y->ssm_a[h];
    /* gdn_conv_step (qwen_reference.rs:105-134): taps over [history | new], weight (tap, ch) at tap + ch * KC */
    const int hist = KC - 1;
    for (int ch = 0; ch < C; ch++) {
        float s = 0.0f;
        for (int tap = 0; tap < KC; tap++) {
            const float in = tap < hist ? y->conv[ch * hist + tap] : mixed[ch];
            s = s + in * y->conv_w[tap + ch * KC];
        }
        act[ch] = s;
    }
    for (int ch = 0; ch < C; ch++) {
        float *hb = y->conv + (size_t)ch * hist;
        for (int t = 0; t + 1 < hist; t++) hb[t] = hb[t + 1];
        hb[hist - 1] = mixed[ch];
    }
    for (int ch = 0; ch < C; ch++) act[ch] = act[ch] / (1.0f + expf(-act[ch]));
    /* q and k heads l2-normalized; V head j reads k-head j mod HK (tiled GGUF V ordering) */
    for (int h = 0; h < HK; h++) {
        l2_normalize(act + (size_t)h * hd, hd, m->eps);
        l2_normalize(act + (size_t)(HK + h) * hd, hd, m->eps);
    }
    for (int j = 0; j < HV; j++) {
        const int kh = j % HK;
        state_step(y->state + (size_t)j * hd * hd, act + (size_t)(HK + kh) * hd, act + (size_t)(2 * HK + j) * hd,
                   act + (size_t)kh * hd, expf(gate[j]), beta[j], hd, hd, o + (size_t)j * hd, sk, dv);
    }
    /* gated norm: rms(o) * ssm_norm * silu(z) per head (ssm_norm used raw) */
    for (int j = 0; j < HV; j++) {
        const float *oh = o + (size_t)j * hd;
        float sum = 0.0f;
        for (int i = 0; i < hd; i++) sum = sum + oh[i] * oh[i];
        const float inv = 1.0f / sqrtf(sum / (float)hd + m->eps);
        for (int i = 0; i < hd; i++) {
            const float zv = z[j * hd + i];
            const float silu = zv / (1.0f + expf(-zv));
            gated[j * hd + i] = oh[i] * inv * y->ssm_norm[i] * silu;
        }
    }
    gemv(y->tout, y->wout, m->hidden, m->inner, gated, out);
    free(mixed); free(z); free(beta); free(gate); free(act); free(o); free(gated); free(sk); free(dv);
}

/* one full-attention layer's block (host_full_attn_ar_step): gated q, q/k RMS norm, partial NeoX rope,
 * softmax attention, sigmoid gate, output projection */
static void attn_block(orc_q35 *m, q35_layer *y, const float *xn, int pos, float *out) {
    const int hd = m->hd, HQ = m->hq, HKV = m->hkv, qd = HQ * hd, kd = HKV * hd;
    float *qg = (float *)malloc(sizeof(float) * 2 * qd), *q = (float *)malloc(sizeof(float) * qd);
    float *gate = (float *)malloc(sizeof(float) * qd), *k = (float *)malloc(sizeof(float) * kd);
    float *v = (float *)malloc(sizeof(float) * kd), *att = (float *)calloc((size_t)qd, sizeof(float));
    float *sc = (float *)malloc(sizeof(float) * (pos + 1));
    gemv(y->tq, y->wq, 2 * qd, m->hidden, xn, qg);
    for (int h = 0; h < HQ; h++) {
        orc_rms_norm(qg + (size_t)h * 2 * hd, y->q_norm, q + (size_t)h * hd, hd, m->eps);
        memcpy(gate + (size_t)h * hd, qg + (size_t)h * 2 * hd + hd, sizeof(float) * hd);
    }
    gemv(y->tk, y->wk, kd, m->hidden, xn, k);
    for (int h = 0; h < HKV; h++) {
        float tmp[1024];
        orc_rms_norm(k + (size_t)h * hd, y->k_norm, tmp, hd, m->eps);
        memcpy(k + (size_t)h * hd, tmp, sizeof(float) * hd);
    }
    gemv(y->tv, y->wv, kd, m->hidden, xn, v);
    orc_rope_neox(q, HQ, hd, m->rot, pos, m->base);
    orc_rope_neox(k, HKV, hd, m->rot, pos, m->base);
    memcpy(y->kcache + (size_t)pos * kd, k, sizeof(float) * kd);
    memcpy(y->vcache + (size_t)pos * kd, v, sizeof(float) * kd);
    kv_round(y->kcache + (size_t)pos * kd, kd, m->kv_round);
    kv_round(y->vcache + (size_t)pos * kd, kd, m->kv_round);
    const int group = HQ / HKV, tokens = pos + 1;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int qh = 0; qh < HQ; qh++) {
        const int kh = qh / group;
        const float *qv = q + (size_t)qh * hd;
        float mx = -INFINITY;
        for (int t = 0; t < tokens; t++) {
            const float *kk = y->kcache + ((size_t)t * HKV + kh) * hd;
            float s = 0.0f;
            for (int i = 0; i < hd; i++) s = s + qv[i] * kk[i];
            sc[t] = s * scale;
            if (sc[t] > mx) mx = sc[t];
        }
        float total = 0.0f;
        for (int t = 0; t < tokens; t++) { sc[t] = expf(sc[t] - mx); total = total + sc[t]; }
        float *ao = att + (size_t)qh * hd;
        for (int t = 0; t < tokens; t++) {
            const float *vv = y->vcache + ((size_t)t * HKV + kh) * hd;
            const float wgt = sc[t] / total;
            for (int i = 0; i < hd; i++) ao[i] = ao[i] + wgt * vv[i];
        }
    }
    for (int i = 0; i < qd; i++) att[i] = att[i] * (1.0f / (1.0f + expf(-gate[i])));
    gemv(y->to, y->wo, m->hidden, qd, att, out);
    free(qg); free(q); free(gate); free(k); free(v); free(att); free(sc);
}

int orc_q35_step(orc_q35 *m, uint32_t token, int pos, float *logits, float *trace) {
    if (pos != m->pos_next || pos >= m->max_ctx || (int)token >= m->vocab) return ORC_ERR_CONFIG;
    const int H = m->hidden, F = m->ffn;
    float *h = (float *)malloc(sizeof(float) * H), *xn = (float *)malloc(sizeof(float) * H);
    float *o = (float *)malloc(sizeof(float) * H), *gt = (float *)malloc(sizeof(float) * F);
    float *up = (float *)malloc(sizeof(float) * F);
    uint64_t be, bb;
    orc_tensor_layout(m->t_embd, &be, &bb);
    orc_dequantize(m->t_embd, m->embd + (uint64_t)token * (H / be) * bb, (size_t)(H / be * bb), h);
    if (trace) memcpy(trace, h, sizeof(float) * H);
    for (int l = 0; l < m->layers; l++) {
        q35_layer *y = &m->L[l];
        orc_rms_norm(h, y->attn_norm, xn, H, m->eps);
        if (y->recurrent) gdn_block(m, y, xn, o);
        else attn_block(m, y, xn, pos, o);
        for (int i = 0; i < H; i++) h[i] = h[i] + o[i];
        orc_rms_norm(h, y->post_norm, xn, H, m->eps);
        gemv(y->tg, y->wg, F, H, xn, gt);
        gemv(y->tu, y->wu, F, H, xn, up);
        for (int i = 0; i < F; i++) gt[i] = gt[i] / (1.0f + expf(-gt[i])) * up[i];
        gemv(y->td, y->wd, H, F, gt, o);
        for (int i = 0; i < H; i++) h[i] = h[i] + o[i];
        if (trace) memcpy(trace + (size_t)(l + 1) * H, h, sizeof(float) * H);
    }
    orc_rms_norm(h, m->out_norm, xn, H, m->eps);
    if (logits) gemv(m->t_out, m->out, m->vocab, H, xn, logits);
    m->pos_next = pos + 1;
    free(h); free(xn); free(o); free(gt); free(up);
    return ORC_OK;
}

/* The delta rule on its own (gdn_state_step), for closed-form and algebra checks. */
void orc_gdn_state_step(float *state, const float *k, const float *v, const float *q, float decay, float beta,
                        int kd, int vd, float *out) {
    float *sk = (float *)malloc(sizeof(float) * vd), *dv = (float *)malloc(sizeof(float) * vd);
    state_step(state, k, v, q, decay, beta, kd, vd, out, sk, dv);
    free(sk); free(dv);
}
