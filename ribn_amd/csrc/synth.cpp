// Seeded synthetic dense-Qwen GGUF v3 writer with GGML block quantizers.
//
// The reference ships no quantizer; this one follows the Q8_0 / Q4_K / Q6_K
// block formats that crates/gguf/src/lib.rs:577-649 decodes, with a simple
// per-group min/max (Q4_K) and abs-max (Q6_K, Q8_0) search of our own. Parity
// never depends on quantizer quality: it is checked after dequantization.
//
// Weights: N(0, std) from a counter-based generator (splitmix64 + Box-Muller),
// so any element can be generated independently and tensors are produced by
// several threads without changing the bytes.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <thread>
#include <vector>

#include "common.h"
#include "../../include/ribn_rocm.h"

namespace ribn {
namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

// Element `i` of tensor `tid`: standard normal scaled by `stdev`.
inline float gauss(uint64_t seed, uint64_t tid, uint64_t i, float stdev) {
    uint64_t r = splitmix64(splitmix64(seed ^ (tid * 0x632be59bd9b4e019ull)) + (i >> 1));
    double u1 = ((double)(r >> 32) + 0.5) * (1.0 / 4294967296.0);
    double u2 = ((double)(r & 0xffffffffull) + 0.5) * (1.0 / 4294967296.0);
    double rad = std::sqrt(-2.0 * std::log(u1));
    double ang = 6.283185307179586 * u2;
    double z = (i & 1) ? rad * std::sin(ang) : rad * std::cos(ang);
    return (float)(z * stdev);
}

inline int nearest(float v) { return (int)std::lrintf(v); }

void quant_q8_0(const float* x, uint8_t* out) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    uint16_t dh = f32_to_f16(amax / 127.f);
    float d = f16_to_f32(dh);
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 32; i++) {
        int q = d > 0.f ? nearest(x[i] / d) : 0;
        q = std::min(127, std::max(-128, q));
        out[2 + i] = (uint8_t)(int8_t)q;
    }
}

// Q4_K: 8 groups of 32, value = (d*sc)*q - (dmin*m), q in [0,15], sc/m 6-bit.
void quant_q4_k(const float* x, uint8_t* out) {
    float scale[8], minv[8];
    for (int g = 0; g < 8; g++) {
        float lo = x[g * 32], hi = x[g * 32];
        for (int i = 1; i < 32; i++) { lo = std::min(lo, x[g * 32 + i]); hi = std::max(hi, x[g * 32 + i]); }
        if (lo > 0.f) lo = 0.f;
        scale[g] = (hi - lo) / 15.f;
        minv[g] = -lo;
    }
    float smax = 0.f, mmax = 0.f;
    for (int g = 0; g < 8; g++) { smax = std::max(smax, scale[g]); mmax = std::max(mmax, minv[g]); }
    uint16_t dh = f32_to_f16(smax / 63.f), mh = f32_to_f16(mmax / 63.f);
    float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    uint8_t sc[8], mn[8];
    for (int g = 0; g < 8; g++) {
        sc[g] = (uint8_t)std::min(63, std::max(0, d > 0.f ? nearest(scale[g] / d) : 0));
        mn[g] = (uint8_t)std::min(63, std::max(0, dmin > 0.f ? nearest(minv[g] / dmin) : 0));
    }
    std::memset(out, 0, 144);
    out[0] = (uint8_t)(dh & 0xff); out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 0xff); out[3] = (uint8_t)(mh >> 8);
    uint8_t* e = out + 4;
    for (int g = 0; g < 4; g++) {
        e[g] = (uint8_t)(sc[g] | ((sc[g + 4] >> 4) << 6));
        e[4 + g] = (uint8_t)(mn[g] | ((mn[g + 4] >> 4) << 6));
        e[8 + g] = (uint8_t)((sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4));
    }
    for (int g = 0; g < 8; g++) {
        float gs = d * (float)sc[g], gm = dmin * (float)mn[g];
        for (int i = 0; i < 32; i++) {
            int q = gs > 0.f ? nearest((x[g * 32 + i] + gm) / gs) : 0;
            q = std::min(15, std::max(0, q));
            out[16 + (g / 2) * 32 + i] |= (uint8_t)(q << ((g % 2) * 4));
        }
    }
}

// Q6_K: 16 sub-blocks of 16, value = (d*sc)*(q-32), q in [0,63], sc int8.
void quant_q6_k(const float* x, uint8_t* out) {
    float scale[16];
    for (int s = 0; s < 16; s++) {
        float amax = 0.f;
        for (int i = 0; i < 16; i++) amax = std::max(amax, std::fabs(x[s * 16 + i]));
        scale[s] = amax / 31.f;
    }
    float smax = 0.f;
    for (int s = 0; s < 16; s++) smax = std::max(smax, scale[s]);
    uint16_t dh = f32_to_f16(smax / 127.f);
    float d = f16_to_f32(dh);
    std::memset(out, 0, 210);
    uint8_t *ql = out, *qh = out + 128, *scales = out + 192;
    int8_t sc[16];
    for (int s = 0; s < 16; s++) {
        sc[s] = (int8_t)std::min(127, std::max(-128, d > 0.f ? nearest(scale[s] / d) : 0));
        scales[s] = (uint8_t)sc[s];
    }
    out[208] = (uint8_t)(dh & 0xff);
    out[209] = (uint8_t)(dh >> 8);
    for (int e = 0; e < 256; e++) {
        int g = e / 32, pos = e % 32, chunk = g / 4, variant = g % 4;
        float gs = d * (float)sc[g * 2 + pos / 16];
        int q = gs > 0.f ? nearest(x[e] / gs) : 0;
        q = std::min(31, std::max(-32, q)) + 32;
        ql[chunk * 64 + (variant % 2) * 32 + pos] |= (uint8_t)((q & 15) << (variant < 2 ? 0 : 4));
        qh[chunk * 32 + pos] |= (uint8_t)((q >> 4) << (2 * variant));
    }
}

struct TensorPlan {
    std::string name;
    std::vector<uint64_t> dims;  // ne0 first
    uint32_t type;
    float stdev;   // for random tensors
    float fill;    // constant fill (norms) when stdev == 0
    uint64_t tid;
    float jitter = -1.f;   // fill + N(0, jitter); < 0: the config's norm jitter for norm tensors
    uint64_t offset = 0;
    uint64_t bytes = 0;
};

void put_u32(std::vector<uint8_t>& b, uint32_t v) { for (int i = 0; i < 4; i++) b.push_back((uint8_t)(v >> (8 * i))); }
void put_u64(std::vector<uint8_t>& b, uint64_t v) { for (int i = 0; i < 8; i++) b.push_back((uint8_t)(v >> (8 * i))); }
void put_str(std::vector<uint8_t>& b, const std::string& s) { put_u64(b, s.size()); b.insert(b.end(), s.begin(), s.end()); }
void kv_u32(std::vector<uint8_t>& b, const std::string& k, uint32_t v) { put_str(b, k); put_u32(b, 4); put_u32(b, v); }
void kv_f32(std::vector<uint8_t>& b, const std::string& k, float v) {
    put_str(b, k); put_u32(b, 6); uint32_t u; std::memcpy(&u, &v, 4); put_u32(b, u);
}
void kv_str(std::vector<uint8_t>& b, const std::string& k, const std::string& v) { put_str(b, k); put_u32(b, 8); put_str(b, v); }

// Generate one tensor's encoded bytes (rows split across threads).
void encode_tensor(const TensorPlan& t, uint64_t seed, float jitter, uint8_t* out, int threads) {
    uint64_t be, bb;
    type_layout(t.type, &be, &bb);
    uint64_t ne0 = t.dims[0], rows = 1;
    for (size_t i = 1; i < t.dims.size(); i++) rows *= t.dims[i];
    uint64_t row_bytes = ne0 / be * bb;
    auto work = [&](uint64_t r0, uint64_t r1) {
        std::vector<float> buf(ne0);
        for (uint64_t r = r0; r < r1; r++) {
            for (uint64_t i = 0; i < ne0; i++) {
                uint64_t idx = r * ne0 + i;
                if (t.stdev > 0.f) buf[i] = gauss(seed, t.tid, idx, t.stdev);
                else buf[i] = t.fill + (jitter > 0.f ? gauss(seed, t.tid, idx, jitter) : 0.f);
            }
            uint8_t* o = out + r * row_bytes;
            for (uint64_t b = 0; b < ne0 / be; b++) {
                const float* xb = buf.data() + b * be;
                uint8_t* ob = o + b * bb;
                switch (t.type) {
                case GGML_F32: std::memcpy(ob, xb, 4); break;
                case GGML_F16: { uint16_t h = f32_to_f16(xb[0]); std::memcpy(ob, &h, 2); break; }
                case GGML_Q8_0: quant_q8_0(xb, ob); break;
                case GGML_Q4_K: quant_q4_k(xb, ob); break;
                case GGML_Q6_K: quant_q6_k(xb, ob); break;
                }
            }
        }
    };
    int nt = (int)std::max<uint64_t>(1, std::min<uint64_t>((uint64_t)threads, rows / 64 + 1));
    if (nt == 1) { work(0, rows); return; }
    std::vector<std::thread> th;
    uint64_t per = (rows + nt - 1) / nt;
    for (int i = 0; i < nt; i++) {
        uint64_t r0 = std::min(rows, per * i), r1 = std::min(rows, per * (i + 1));
        th.emplace_back(work, r0, r1);
    }
    for (auto& x : th) x.join();
}

// Lay out `plan`, write the header (metadata entries already encoded in
// `kvs`, n_kv of them) and the tensor data.
int write_gguf(const char* path, std::vector<TensorPlan>& plan, const std::vector<uint8_t>& kvs, uint64_t n_kv,
               const ribn_rocm_synth_config* c, char* err, size_t err_len) {
    uint64_t off = 0;
    for (auto& t : plan) {
        uint64_t be, bb;
        if (!type_layout(t.type, &be, &bb) || t.dims[0] % be) {
            set_err(err, err_len, "tensor " + t.name + ": type " + std::to_string(t.type) +
                                      " does not fit dimension " + std::to_string(t.dims[0]));
            return RIBN_ERR_INVALID;
        }
        uint64_t n = 1;
        for (auto d : t.dims) n *= d;
        t.bytes = n / be * bb;
        t.offset = off;
        off += (t.bytes + 31) / 32 * 32;
    }
    std::vector<uint8_t> hdr;
    put_u32(hdr, 0x46554747u);
    put_u32(hdr, 3);
    put_u64(hdr, plan.size());
    put_u64(hdr, n_kv);
    hdr.insert(hdr.end(), kvs.begin(), kvs.end());
    for (auto& t : plan) {
        put_str(hdr, t.name);
        put_u32(hdr, (uint32_t)t.dims.size());
        for (auto d : t.dims) put_u64(hdr, d);
        put_u32(hdr, t.type);
        put_u64(hdr, t.offset);
    }
    while (hdr.size() % 32) hdr.push_back(0);
    FILE* f = std::fopen(path, "wb");
    if (!f) { set_err(err, err_len, std::string("cannot create ") + path); return RIBN_ERR_IO; }
    bool ok = std::fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
    int threads = c->threads > 0 ? c->threads : (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<uint8_t> buf;
    for (auto& t : plan) {
        if (!ok) break;
        uint64_t padded = (t.bytes + 31) / 32 * 32;
        buf.assign(padded, 0);
        const bool is_norm = t.name.find("norm") != std::string::npos;
        const float jitter = t.jitter >= 0.f ? t.jitter : is_norm ? c->norm_jitter : 0.f;
        encode_tensor(t, c->seed, jitter, buf.data(), threads);
        ok = std::fwrite(buf.data(), 1, padded, f) == padded;
    }
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) { set_err(err, err_len, std::string("write failed: ") + path); return RIBN_ERR_IO; }
    return RIBN_OK;
}

}  // namespace
}  // namespace ribn

using namespace ribn;

extern "C" int ribn_rocm_synth_qwen_gguf(const char* path, const ribn_rocm_synth_config* c, char* err,
                                         size_t err_len) {
    if (!path || !c) { set_err(err, err_len, "null argument"); return RIBN_ERR_INVALID; }
    std::string arch = c->qwen3 ? "qwen3" : "qwen2";
    uint64_t H = c->hidden, L = c->layers, hq = c->q_heads, hkv = c->kv_heads, hd = c->head_dim;
    uint64_t F = c->ffn, V = c->vocab;
    if (!H || !L || !hq || !hkv || !hd || !F || !V || hq % hkv) {
        set_err(err, err_len, "invalid synthetic geometry");
        return RIBN_ERR_INVALID;
    }
    uint32_t def = c->weight_type ? c->weight_type : GGML_Q4_K;
    uint32_t vt = c->attn_v_type ? c->attn_v_type : def;
    uint32_t dt = c->ffn_down_type ? c->ffn_down_type : def;
    uint32_t ot = c->output_type ? c->output_type : def;
    uint32_t et = c->embd_type ? c->embd_type : def;
    float sd = c->weight_std > 0.f ? c->weight_std : 0.02f;
    std::vector<TensorPlan> plan;
    uint64_t tid = 1;
    auto add = [&](const std::string& n, std::vector<uint64_t> dims, uint32_t t, float stdev, float fill) {
        plan.push_back(TensorPlan{n, dims, t, stdev, fill, tid++});
    };
    add("token_embd.weight", {H, V}, et, sd, 0.f);
    for (uint64_t l = 0; l < L; l++) {
        std::string p = "blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", {H}, GGML_F32, 0.f, 1.f);
        add(p + "attn_q.weight", {H, hq * hd}, def, sd, 0.f);
        add(p + "attn_k.weight", {H, hkv * hd}, def, sd, 0.f);
        add(p + "attn_v.weight", {H, hkv * hd}, vt, sd, 0.f);
        if (c->qwen3) {
            add(p + "attn_q_norm.weight", {hd}, GGML_F32, 0.f, 1.f);
            add(p + "attn_k_norm.weight", {hd}, GGML_F32, 0.f, 1.f);
        } else {
            add(p + "attn_q.bias", {hq * hd}, GGML_F32, sd, 0.f);
            add(p + "attn_k.bias", {hkv * hd}, GGML_F32, sd, 0.f);
            add(p + "attn_v.bias", {hkv * hd}, GGML_F32, sd, 0.f);
        }
        add(p + "attn_output.weight", {hq * hd, H}, def, sd, 0.f);
        add(p + "ffn_norm.weight", {H}, GGML_F32, 0.f, 1.f);
        add(p + "ffn_gate.weight", {H, F}, def, sd, 0.f);
        add(p + "ffn_up.weight", {H, F}, def, sd, 0.f);
        add(p + "ffn_down.weight", {F, H}, dt, sd, 0.f);
    }
    add("output_norm.weight", {H}, GGML_F32, 0.f, 1.f);
    if (!c->tied_output) add("output.weight", {H, V}, ot, sd, 0.f);

    std::vector<uint8_t> kvs;
    kv_str(kvs, "general.architecture", arch);
    kv_u32(kvs, "general.alignment", 32);
    kv_str(kvs, "general.name", "ribn-rocm synthetic " + arch);
    kv_u32(kvs, arch + ".context_length", c->context_length ? c->context_length : 32768);
    kv_u32(kvs, arch + ".embedding_length", (uint32_t)H);
    kv_u32(kvs, arch + ".block_count", (uint32_t)L);
    kv_u32(kvs, arch + ".feed_forward_length", (uint32_t)F);
    kv_u32(kvs, arch + ".attention.head_count", (uint32_t)hq);
    kv_u32(kvs, arch + ".attention.head_count_kv", (uint32_t)hkv);
    kv_u32(kvs, arch + ".attention.key_length", (uint32_t)hd);
    kv_u32(kvs, arch + ".attention.value_length", (uint32_t)hd);
    kv_f32(kvs, arch + ".rope.freq_base", c->rope_base > 0.f ? c->rope_base : 1e6f);
    kv_f32(kvs, arch + ".attention.layer_norm_rms_epsilon", c->rms_eps > 0.f ? c->rms_eps : 1e-6f);
    return write_gguf(path, plan, kvs, 13, c, err, err_len);
}

// qwen35 hybrid (Gated-DeltaNet recurrent layers + gated full attention): the
// tensor names of crates/nvidia/src/decode.rs:52-82 and the metadata keys of
// crates/qwen/src/gguf/config.rs:17-37. Layer i is full attention when (i + 1)
// is a multiple of the interval. attn_q holds [q | gate] per head (2 * head_dim
// rows each). ssm_a = -exp(A_log) is drawn negative, ssm_conv1d and the dt bias
// from N(0, 0.3), the norms as 1 (+ jitter).
extern "C" int ribn_rocm_synth_qwen35_gguf(const char* path, const ribn_rocm_synth_config* c,
                                           const ribn_rocm_synth_hybrid* y, char* err, size_t err_len) {
    if (!path || !c || !y) { set_err(err, err_len, "null argument"); return RIBN_ERR_INVALID; }
    const uint64_t H = c->hidden, L = c->layers, hq = c->q_heads, hkv = c->kv_heads, hd = c->head_dim;
    const uint64_t F = c->ffn, V = c->vocab, HK = y->ssm_groups, HV = y->ssm_heads, D = y->ssm_state;
    const uint64_t KC = y->conv_kernel ? y->conv_kernel : 4, every = y->full_attention_interval;
    if (!H || !L || !hq || !hkv || !hd || !F || !V || hq % hkv || !HK || !HV || !D || HV % HK || !every) {
        set_err(err, err_len, "invalid synthetic hybrid geometry");
        return RIBN_ERR_INVALID;
    }
    const uint64_t C = 2 * HK * D + HV * D, inner = HV * D;
    const uint32_t def = c->weight_type ? c->weight_type : GGML_Q4_K;
    const uint32_t vt = c->attn_v_type ? c->attn_v_type : def, dt = c->ffn_down_type ? c->ffn_down_type : def;
    const uint32_t ot = c->output_type ? c->output_type : def, et = c->embd_type ? c->embd_type : def;
    const uint32_t st = y->ssm_type ? y->ssm_type : GGML_Q8_0;
    const float sd = c->weight_std > 0.f ? c->weight_std : 0.02f;
    std::vector<TensorPlan> plan;
    uint64_t tid = 1;
    auto add = [&](const std::string& n, std::vector<uint64_t> dims, uint32_t t, float stdev, float fill,
                   float jitter = -1.f) {
        TensorPlan p{n, dims, t, stdev, fill, tid++};
        p.jitter = jitter;
        plan.push_back(p);
    };
    add("token_embd.weight", {H, V}, et, sd, 0.f);
    for (uint64_t l = 0; l < L; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", {H}, GGML_F32, 0.f, 1.f);
        if ((l + 1) % every != 0) {
            add(p + "attn_qkv.weight", {H, C}, def, sd, 0.f);
            add(p + "attn_gate.weight", {H, inner}, def, sd, 0.f);
            add(p + "ssm_beta.weight", {H, HV}, st, sd, 0.f);
            add(p + "ssm_alpha.weight", {H, HV}, st, sd, 0.f);
            add(p + "ssm_dt.bias", {HV}, GGML_F32, 0.3f, 0.f);
            add(p + "ssm_a", {HV}, GGML_F32, 0.f, -1.f, 0.4f);
            add(p + "ssm_conv1d.weight", {KC, C}, GGML_F32, 0.3f, 0.f);
            add(p + "ssm_norm.weight", {D}, GGML_F32, 0.f, 1.f);
            add(p + "ssm_out.weight", {inner, H}, def, sd, 0.f);
        } else {
            add(p + "attn_q.weight", {H, 2 * hq * hd}, def, sd, 0.f);
            add(p + "attn_k.weight", {H, hkv * hd}, def, sd, 0.f);
            add(p + "attn_v.weight", {H, hkv * hd}, vt, sd, 0.f);
            add(p + "attn_q_norm.weight", {hd}, GGML_F32, 0.f, 1.f);
            add(p + "attn_k_norm.weight", {hd}, GGML_F32, 0.f, 1.f);
            add(p + "attn_output.weight", {hq * hd, H}, def, sd, 0.f);
        }
        add(p + "post_attention_norm.weight", {H}, GGML_F32, 0.f, 1.f);
        add(p + "ffn_gate.weight", {H, F}, def, sd, 0.f);
        add(p + "ffn_up.weight", {H, F}, def, sd, 0.f);
        add(p + "ffn_down.weight", {F, H}, dt, sd, 0.f);
    }
    add("output_norm.weight", {H}, GGML_F32, 0.f, 1.f);
    if (!c->tied_output) add("output.weight", {H, V}, ot, sd, 0.f);
    const std::string a = "qwen35";
    std::vector<uint8_t> kvs;
    kv_str(kvs, "general.architecture", a);
    kv_u32(kvs, "general.alignment", 32);
    kv_str(kvs, "general.name", "ribn-rocm synthetic qwen35");
    kv_u32(kvs, a + ".context_length", c->context_length ? c->context_length : 32768);
    kv_u32(kvs, a + ".embedding_length", (uint32_t)H);
    kv_u32(kvs, a + ".block_count", (uint32_t)L);
    kv_u32(kvs, a + ".nextn_predict_layers", 0);
    kv_u32(kvs, a + ".feed_forward_length", (uint32_t)F);
    kv_u32(kvs, a + ".attention.head_count", (uint32_t)hq);
    kv_u32(kvs, a + ".attention.head_count_kv", (uint32_t)hkv);
    kv_u32(kvs, a + ".attention.key_length", (uint32_t)hd);
    kv_u32(kvs, a + ".attention.value_length", (uint32_t)hd);
    kv_f32(kvs, a + ".attention.layer_norm_rms_epsilon", c->rms_eps > 0.f ? c->rms_eps : 1e-6f);
    kv_u32(kvs, a + ".rope.dimension_count", y->rope_dims ? y->rope_dims : (uint32_t)hd);
    kv_f32(kvs, a + ".rope.freq_base", c->rope_base > 0.f ? c->rope_base : 1e7f);
    kv_u32(kvs, a + ".full_attention_interval", (uint32_t)every);
    kv_u32(kvs, a + ".ssm.group_count", (uint32_t)HK);
    kv_u32(kvs, a + ".ssm.inner_size", (uint32_t)inner);
    kv_u32(kvs, a + ".ssm.state_size", (uint32_t)D);
    kv_u32(kvs, a + ".ssm.time_step_rank", (uint32_t)HV);
    kv_u32(kvs, a + ".ssm.conv_kernel", (uint32_t)KC);
    return write_gguf(path, plan, kvs, 21, c, err, err_len);
}

// Quantize `n` floats (a multiple of the block size) into GGML blocks.
extern "C" int ribn_rocm_quantize(uint32_t type, const float* x, uint64_t n, uint8_t* out) {
    uint64_t be, bb;
    if (!type_layout(type, &be, &bb) || n % be) return RIBN_ERR_INVALID;
    for (uint64_t b = 0; b < n / be; b++) {
        const float* xb = x + b * be;
        uint8_t* ob = out + b * bb;
        switch (type) {
        case GGML_F32: std::memcpy(ob, xb, 4); break;
        case GGML_F16: { uint16_t h = f32_to_f16(xb[0]); std::memcpy(ob, &h, 2); break; }
        case GGML_Q8_0: quant_q8_0(xb, ob); break;
        case GGML_Q4_K: quant_q4_k(xb, ob); break;
        case GGML_Q6_K: quant_q6_k(xb, ob); break;
        }
    }
    return RIBN_OK;
}
