// librocm_ribn host side: GGUF loading with weight re-tiling, the per-token
// launch chain captured in HIP graphs, the device-resident greedy loop, and
// the GenerationExecutor-shaped C ABI (include/ribn_rocm.h).
//
// Reference counterparts: loading::load (crates/qwen/src/loading.rs:93-190),
// CudaQwen35Weights::stage (nvidia/src/staging.rs:263), CudaQwen35Decode::run_step
// (nvidia/src/decode.rs:550-640), QwenExecution admit/prepare/submit/poll/commit
// (crates/qwen/src/execution.rs:80-414).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/ribn_rocm.h"
#include "common.h"
#include "gguf.h"
#include "kernels.h"

using namespace ribn;

namespace {

struct Layer {
    QMat q, k, v, o, gate, up, down;
    // qwen35 hybrid: a recurrent (Gated-DeltaNet) layer uses the gdn_* matrices and
    // o = ssm_out; a gated full-attention layer adds the gate half of attn_q
    bool recurrent = false;
    QMat gdn_mix, gdn_z, gdn_ba, q_gate;
    float *dt_bias = nullptr, *ssm_a = nullptr, *conv_w = nullptr, *ssm_norm = nullptr;
    size_t state_off = 0, conv_off = 0;   // floats into a slot's recurrent state
    float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float *q_bias = nullptr, *k_bias = nullptr, *v_bias = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    // resident binary16 weights (RIBN_LOAD_RESIDENT_F16): q|k|v and gate|up
    // concatenated by output row, with the q|k|v bias concatenated likewise
    uint16_t *w16_qkv = nullptr, *w16_o = nullptr, *w16_gu = nullptr, *w16_down = nullptr;
    float* qkv_bias = nullptr;
};

struct Sequence {
    int slot = -1;
    uint32_t prompt_len = 0;
    uint32_t committed = 0;   // logical prefix
    bool has_next = false;
    uint32_t next = 0;
    bool in_flight = false;
    std::vector<int32_t> pages;
};

struct Submission {
    uint64_t id = 0;
    std::vector<ribn_rocm_batch_item> items;
    hipEvent_t done = nullptr;
};


std::string hip_msg(const char* what, hipError_t e) {
    return std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
}

}  // namespace

struct ribn_rocm_model {
    // geometry
    int H = 0, L = 0, hq = 0, hkv = 0, hd = 0, F = 0, V = 0, rot = 0;
    float eps = 1e-6f, base = 1e6f;
    bool qwen3 = false;
    bool kv_f16 = false;
    std::string name;
    uint32_t context = 0, max_seqs = 0, max_batch_tokens = 0, kv_pages = 0;
    int max_pages = 0;
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void*> dev_allocs;
    std::vector<void*> host_allocs;
    uint64_t weight_bytes = 0, kv_bytes = 0;

    QMat embd{}, out{};
    // qwen35 hybrid geometry (hybrid == false: dense qwen2/qwen3)
    bool hybrid = false;
    int ssm_hk = 0, ssm_hv = 0, ssm_d = 0, conv_k = 0, channels = 0, inner = 0, interval = 0;
    float *mixed = nullptr, *zbuf = nullptr, *ba = nullptr, *gdn_act = nullptr, *gated = nullptr, *att_gate = nullptr;
    float* d_rec = nullptr;          // [slots][rec_floats] recurrent state
    size_t rec_floats = 0;
    std::vector<MvArgs> mv_aux;      // gated attention: the gate projection
    std::vector<int> wg_aux;
    uint16_t* w16_head = nullptr;   // resident binary16 output head
    BlasGemm* blas = nullptr;       // hipBLASLt state when the weights are resident
    float* out_norm = nullptr;
    std::vector<Layer> layers;

    // activations / scratch
    float *h = nullptr, *raw = nullptr, *qbuf = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    float* part = nullptr;
    uint32_t* counters = nullptr;   // [hkv] attention, [1] head
    float *inv_freq = nullptr, *rope = nullptr;
    uint64_t* head_partial = nullptr;
    int head_wgs = 0;

    // sequence slots (max_seqs + 1; the last one is the scratch slot of generate/trace)
    SeqState* d_slots = nullptr;
    int32_t* d_pages = nullptr;
    uint32_t* d_tokens = nullptr;
    StepCtl* d_ctl = nullptr;
    StepCtl* h_ctl = nullptr;          // pinned: per-slot StepCtl images
    SeqState* h_state = nullptr;        // pinned mirrors
    int32_t* h_pages = nullptr;
    uint32_t* h_tokens = nullptr;
    uint32_t* h_out = nullptr;          // pinned sampled tokens per submitted row
    std::vector<int> free_slots;
    std::vector<int32_t> free_pages;

    std::vector<MvArgs> mv_qkv, mv_o, mv_gu, mv_down;
    std::vector<int> wg_qkv, wg_o, wg_gu, wg_down;
    MvArgs mv_head{};
    std::map<int, hipGraphExec_t> graphs;   // key: n_splits * 2 + head
    std::map<int, hipGraphExec_t> row_graphs;   // decode rows, key: rows * 64 + n_splits

    // chunked prefill buffers (prefill.hip), rows per chunk = chunk
    int chunk = 0;
    float *p_h = nullptr, *p_qkv = nullptr, *p_q = nullptr, *p_gu = nullptr, *p_part = nullptr;
    // batched decode (one row per sequence through the prefill GEMMs): rows <= max_rows
    int b_rows = 0;
    int32_t* d_brows = nullptr;            // [2][b_rows]: slot, pos
    std::vector<int32_t> h_brows;
    uint32_t* d_btokens = nullptr;
    float *b_att = nullptr, *b_rope = nullptr, *b_part = nullptr, *b_logits = nullptr;
    std::vector<uint64_t> last_batch_seqs;   // sequences of the last submission's batched decode rows
    size_t b_part_stride = 0;
    uint32_t* b_counters = nullptr;
    uint64_t* b_argmax = nullptr;          // [b_rows][64] per-chunk argmax keys
    size_t p_part_floats = 0;
    uint16_t *p_x16 = nullptr, *p_att16 = nullptr, *p_act16 = nullptr;
    // integer-dot decode (RIBN_LOAD_INT_DOT): Q8_1 words of the decode rows' inputs, SwiGLU rows
    bool int_dot = false;
    bool merge_in_launch = false;   // RIBN_LOAD_ATTN_MERGE_IN_LAUNCH: long-context split partials merged in the attention launch
    unsigned long long* gu_clk = nullptr;   // set only while ribn_rocm_bench_model_kernel 7 captures its step
    uint32_t* b_xq = nullptr;
    float* b_act = nullptr;
    int cur_slot = 0;   // the slot select_slot last pointed the step at

    // persistent step (one launch per token); step_wg == 0: launch chain only
    int step_wg = 0;
    size_t step_lds = 0;
    StepKey step_key{};
    StepArgs step_args{};
    LayerDev* d_layers = nullptr;
    uint32_t* step_bar = nullptr;
    float* arena_h0 = nullptr;
    std::vector<float*> arena_h2;   // residual stream after each layer

    // executor state
    std::map<uint64_t, Sequence> seqs;
    bool faulted = false;
    bool has_prepared = false;
    std::vector<ribn_rocm_batch_item> prepared;
    bool has_pending = false;
    Submission pending;
    uint64_t next_submission = 1;
};

namespace {

int fail(ribn_rocm_model* M, char* err, size_t err_len, const std::string& msg, int code = RIBN_ERR_DEVICE) {
    if (M && code == RIBN_ERR_DEVICE) M->faulted = true;
    set_err(err, err_len, msg);
    return code;
}

#define HIPCHK(expr)                                                             \
    do {                                                                         \
        hipError_t e_ = (expr);                                                  \
        if (e_ != hipSuccess) return fail(M, err, err_len, hip_msg(#expr, e_)); \
    } while (0)

template <typename T>
hipError_t dalloc(ribn_rocm_model* M, T** p, size_t bytes) {
    void* v = nullptr;
    hipError_t e = hipMalloc(&v, bytes ? bytes : 256);
    if (e == hipSuccess) {
        M->dev_allocs.push_back(v);
        *p = static_cast<T*>(v);
    }
    return e;
}
template <typename T>
hipError_t halloc(ribn_rocm_model* M, T** p, size_t bytes) {
    void* v = nullptr;
    hipError_t e = hipHostMalloc(&v, bytes ? bytes : 256, hipHostMallocDefault);
    if (e == hipSuccess) {
        M->host_allocs.push_back(v);
        *p = static_cast<T*>(v);
    }
    return e;
}

// Split GGUF blocks into the device planes described in kernels.h (QMat).
void retile(uint32_t type, const uint8_t* src, uint64_t n_blocks, uint8_t* a, uint8_t* b, uint8_t* c, uint8_t* d) {
    auto work = [&](uint64_t b0, uint64_t b1) {
        for (uint64_t i = b0; i < b1; i++) {
            if (type == GGML_Q4_K) {
                // scale unpacking as q4_k_scales (crates/gguf/src/lib.rs:561-575)
                const uint8_t* s = src + i * 144;
                const uint8_t* e = s + 4;
                uint8_t sc[8], mn[8];
                for (int j = 0; j < 4; j++) {
                    sc[j] = e[j] & 0x3f;
                    sc[j + 4] = (uint8_t)((e[8 + j] & 0x0f) | ((e[j] >> 2) & 0x30));
                    mn[j] = e[4 + j] & 0x3f;
                    mn[j + 4] = (uint8_t)((e[8 + j] >> 4) | ((e[4 + j] >> 2) & 0x30));
                }
                uint8_t* o = b + i * 16;
                for (int p = 0; p < 4; p++) {
                    o[4 * p] = sc[2 * p];
                    o[4 * p + 1] = sc[2 * p + 1];
                    o[4 * p + 2] = mn[2 * p];
                    o[4 * p + 3] = mn[2 * p + 1];
                }
                std::memcpy(c + i * 4, s, 4);
                std::memcpy(a + i * 128, s + 16, 128);
            } else if (type == GGML_Q6_K) {
                const uint8_t* s = src + i * 210;
                std::memcpy(a + i * 128, s, 128);
                std::memcpy(b + i * 64, s + 128, 64);
                for (int cc = 0; cc < 8; cc++) {
                    const int il = 8 * (cc / 4) + cc % 4;
                    c[i * 16 + 2 * cc] = s[192 + il];
                    c[i * 16 + 2 * cc + 1] = s[192 + il + 4];
                }
                std::memcpy(d + i * 2, s + 208, 2);
            } else {
                const uint8_t* s = src + i * 34;
                std::memcpy(b + i * 2, s, 2);
                std::memcpy(a + i * 32, s + 2, 32);
            }
        }
    };
    int nt = (int)std::min<uint64_t>(16, std::max<uint64_t>(1, n_blocks / 65536));
    if (nt <= 1) { work(0, n_blocks); return; }
    std::vector<std::thread> th;
    uint64_t per = (n_blocks + nt - 1) / nt;
    for (int t = 0; t < nt; t++) th.emplace_back(work, std::min(n_blocks, per * t), std::min(n_blocks, per * (t + 1)));
    for (auto& x : th) x.join();
}

// The GEMM-ordered copy of a Q4_K / Q6_K matrix (QMat::g), from its host
// planes. Block (n16, kt) holds what the 64 lanes of a wave read for the
// B fragments of rows 16 n16 .. 16 n16 + 15 (rows past the matrix repeat its
// last row) and K tile kt (128 values: half a super-block, h = kt % 2), lane =
// bn + 16 bj reading row 16 n16 + bn:
//   Q4_K (kGemmBlkQ4 = 1216): [0, 1024) lane's 16 qs bytes (32 (bj/2) + 16 (bj%2)
//        into the half block), [1024, 1152) scale dword of (bn, bj/2),
//        [1152, 1216) d|dmin dword of bn;
//   Q6_K (kGemmBlkQ6 = 1696): [0, 1024) lane's ql bytes 8 bj .. +8 and 32 + 8 bj ..
//        +8, [1024, 1536) its qh bytes 8 bj .. +8, [1536, 1664) the two 8-bit
//        sub-block scales of (bn, bj/2) (bytes 0-1: v = 0/2, 2-3: v = 1/3),
//        [1664, 1696) d of bn.
// Every read of the GEMM is then one coalesced access per plane of a block.
size_t gemm_pack_bytes(uint32_t type, uint64_t rows, uint64_t k) {
    const uint64_t n16 = (rows + 15) / 16, nkt = k / 128;
    return type == GGML_Q4_K ? n16 * nkt * kGemmBlkQ4 : type == GGML_Q6_K ? n16 * nkt * kGemmBlkQ6 : 0;
}

void gemm_pack(uint32_t type, uint64_t rows, uint64_t nb, const uint8_t* a, const uint8_t* b, const uint8_t* c,
               const uint8_t* d, uint8_t* out) {
    const uint64_t n16c = (rows + 15) / 16, nkt = nb * 2;
    auto work = [&](uint64_t g0, uint64_t g1) {
        for (uint64_t n16 = g0; n16 < g1; n16++)
            for (uint64_t kt = 0; kt < nkt; kt++) {
                const uint64_t kb = kt >> 1, h = kt & 1;
                for (int lane = 0; lane < 64; lane++) {
                    const int bn = lane & 15, bj = lane >> 4;
                    const uint64_t r = std::min<uint64_t>(n16 * 16 + bn, rows - 1), bi = r * nb + kb;
                    if (type == GGML_Q4_K) {
                        uint8_t* o = out + (n16 * nkt + kt) * kGemmBlkQ4;
                        std::memcpy(o + lane * 16, a + bi * 128 + 64 * h + 32 * (bj >> 1) + 16 * (bj & 1), 16);
                        if ((bj & 1) == 0) std::memcpy(o + 1024 + (bn * 2 + (bj >> 1)) * 4, b + bi * 16 + 8 * h + 4 * (bj >> 1), 4);
                        if (bj == 0) std::memcpy(o + 1152 + bn * 4, c + bi * 4, 4);
                    } else {
                        uint8_t* o = out + (n16 * nkt + kt) * kGemmBlkQ6;
                        std::memcpy(o + lane * 16, a + bi * 128 + 64 * h + 8 * bj, 8);
                        std::memcpy(o + lane * 16 + 8, a + bi * 128 + 64 * h + 32 + 8 * bj, 8);
                        std::memcpy(o + 1024 + lane * 8, b + bi * 64 + 32 * h + 8 * bj, 8);
                        if ((bj & 1) == 0) {
                            const uint8_t* sp = c + bi * 16 + 8 * h + 2 * (bj >> 1);
                            uint8_t* sd = o + 1536 + (bn * 2 + (bj >> 1)) * 4;
                            sd[0] = sp[0]; sd[1] = sp[1]; sd[2] = sp[4]; sd[3] = sp[5];
                        }
                        if (bj == 0) std::memcpy(o + 1664 + bn * 2, d + bi * 2, 2);
                    }
                }
            }
    };
    const int nt = (int)std::min<uint64_t>(16, std::max<uint64_t>(1, n16c / 64));
    if (nt <= 1) { work(0, n16c); return; }
    std::vector<std::thread> th;
    const uint64_t per = (n16c + nt - 1) / nt;
    for (int t = 0; t < nt; t++) th.emplace_back(work, std::min(n16c, per * t), std::min(n16c, per * (t + 1)));
    for (auto& x : th) x.join();
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Plane sizes for a [rows][k] matrix of `type`.
void plane_sizes(uint32_t type, uint64_t nblocks, size_t* sa, size_t* sb, size_t* sc, size_t* sd) {
    *sa = *sb = *sc = *sd = 0;
    if (type == GGML_Q4_K) { *sa = nblocks * 128; *sb = nblocks * 16; *sc = nblocks * 4; }
    else if (type == GGML_Q6_K) { *sa = nblocks * 128; *sb = nblocks * 64; *sc = nblocks * 16; *sd = nblocks * 2; }
    else { *sa = nblocks * 32; *sb = nblocks * 2; }
}

// Allocate planes and upload re-tiled blocks. `blocks` may be host memory of
// exactly rows*k/block_elems GGUF blocks.
hipError_t upload_qmat(ribn_rocm_model* M, uint32_t type, uint64_t rows, uint64_t k, const uint8_t* blocks, QMat* out,
                       std::vector<uint8_t>& staging, bool gemm_copy = false) {
    uint64_t be, bb;
    type_layout(type, &be, &bb);
    const uint64_t nblocks = rows * (k / be);
    size_t sa, sb, sc, sd;
    plane_sizes(type, nblocks, &sa, &sb, &sc, &sd);
    const size_t total = align256(sa) + align256(sb) + align256(sc) + align256(sd);
    uint8_t* dev = nullptr;
    hipError_t e = dalloc(M, &dev, total);
    if (e != hipSuccess) return e;
    staging.resize(total);
    uint8_t* ha = staging.data();
    uint8_t* hb = ha + align256(sa);
    uint8_t* hc = hb + align256(sb);
    uint8_t* hdp = hc + align256(sc);
    retile(type, blocks, nblocks, ha, hb, hc, hdp);
    e = hipMemcpy(dev, staging.data(), total, hipMemcpyHostToDevice);
    if (e != hipSuccess) return e;
    QMat q{};
    q.type = type;
    q.rows = (uint32_t)rows;
    q.k = (uint32_t)k;
    q.nb = (uint32_t)(k / be);
    q.a = dev;
    q.b = dev + (hb - ha);
    q.c = dev + (hc - ha);
    q.d = dev + (hdp - ha);
    q.g = nullptr;
    const size_t gbytes = gemm_copy ? gemm_pack_bytes(type, rows, k) : 0;
    if (gbytes) {
        std::vector<uint8_t> packed(gbytes);
        gemm_pack(type, rows, q.nb, ha, hb, hc, hdp, packed.data());
        uint8_t* gdev = nullptr;
        if ((e = dalloc(M, &gdev, gbytes)) != hipSuccess) return e;
        if ((e = hipMemcpy(gdev, packed.data(), gbytes, hipMemcpyHostToDevice)) != hipSuccess) return e;
        q.g = gdev;
    }
    *out = q;
    M->weight_bytes += nblocks * bb;
    return hipSuccess;
}

// Items per wave for a launch of `items` two-row items: the largest power of two
// (<= cap) that still leaves >= 2048 workgroups of 4 waves.
int choose_ipw(int items, int cap) {
    int ipw = 1;
    while (ipw < cap && items / (4 * ipw * 2) >= 2048) ipw *= 2;
    return ipw;
}

}  // namespace

namespace {

// ---------------------------------------------------------------------------
// Per-launch argument blocks, built once at load (only positions, page tables
// and tokens change between steps, and those live in device memory).
MvArgs mv_base(const float* x, const float* norm_w, float eps, int k, int mode, const StepCtl* ctl) {
    MvArgs a{};
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.k = k;
    a.mode = mode;
    a.ctl = ctl;
    return a;
}

// Assign workgroups to segments; returns the grid size.
int layout_segments(MvArgs& a) {
    const int rpi = matvec_rows_per_wg(a) / std::max(a.items_per_wave, 1);   // rows per item across the waves
    int wg = 0;
    for (int i = 0; i < a.nseg; i++) {
        // a segment keeps an items-per-wave count set beforehand (q|k|v balance)
        if (a.seg[i].ipw <= 0) a.seg[i].ipw = a.items_per_wave;
        const int rpw = rpi * a.seg[i].ipw;
        if (!a.seg[i].res) a.seg[i].res = a.seg[i].out;   // standalone launches add in place
        a.seg[i].wg_begin = wg;
        wg += ((int)a.seg[i].w.rows + rpw - 1) / rpw;
    }
    return wg;
}

// Lay a launch out on a fixed grid of n_wg workgroups (the persistent step):
// each segment gets ceil(items / (4 ipw)) workgroups; items per wave start at 1
// and grow, one segment at a time where the longest per-wave work grows least,
// until the segments fit. Returns the workgroups used (<= n_wg).
int layout_grid(MvArgs& a, int n_wg) {
    const bool pair = a.mode == MV_SILU;
    int items[3] = {0, 0, 0}, ipw[3] = {1, 1, 1}, wgs[3] = {0, 0, 0};
    double item_bytes[3] = {0, 0, 0};
    for (int i = 0; i < a.nseg; i++) {
        const QMat& w = a.seg[i].w;
        uint64_t be, bb;
        type_layout(w.type, &be, &bb);
        items[i] = pair ? (int)w.rows : ((int)w.rows + 1) / 2;
        item_bytes[i] = 2.0 * (double)w.k / (double)be * (double)bb;
    }
    auto total = [&]() {
        int t = 0;
        for (int i = 0; i < a.nseg; i++) {
            wgs[i] = (items[i] + 4 * ipw[i] - 1) / (4 * ipw[i]);
            t += wgs[i];
        }
        return t;
    };
    while (total() > n_wg) {
        int best = -1;
        double best_cost = 0;
        for (int i = 0; i < a.nseg; i++) {
            if (wgs[i] <= 1) continue;
            const double cost = (ipw[i] + 1) * item_bytes[i];
            if (best < 0 || cost < best_cost) { best = i; best_cost = cost; }
        }
        if (best < 0) break;
        ipw[best]++;
    }
    int wg = 0;
    for (int i = 0; i < a.nseg; i++) {
        a.seg[i].ipw = ipw[i];
        if (!a.seg[i].res) a.seg[i].res = a.seg[i].out;
        a.seg[i].wg_begin = wg;
        wg += wgs[i];
    }
    a.items_per_wave = ipw[0];
    for (int i = 0; i < a.nseg; i++)   // per-row addends are held one per lane
        if ((a.mode == MV_ADD || a.seg[i].bias) && a.seg[i].ipw > 32) return -1;
    return wg;
}

// Items per wave that lay a launch of `items` out as at most one workgroup per
// compute unit: measured on the 8B shape (gate/up, down, o, q|k|v), a launch whose
// workgroups all start at once beats both smaller workgroups and a second round
// (gate/up at 8 waves: 256 workgroups 13.4 us, 308 workgroups 18.6 us).
int one_pass_ipw(int items, int waves, int n_cu, int cap = 16) {
    const int per = waves * std::max(n_cu, 1);
    return std::min(cap, std::max(1, (items + per - 1) / per));
}

// Encoded bytes of one row of a quantized matrix.
double qrow_bytes(const QMat& w) {
    uint64_t be = 1, bb = 0;
    type_layout(w.type, &be, &bb);
    return (double)w.k / (double)be * (double)bb;
}

void build_launches(ribn_rocm_model* M) {
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd;
    int n_cu = 256;
    hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, M->device);
    M->mv_qkv.clear(); M->mv_o.clear(); M->mv_gu.clear(); M->mv_down.clear();
    M->wg_qkv.clear(); M->wg_o.clear(); M->wg_gu.clear(); M->wg_down.clear();
    M->mv_aux.clear(); M->wg_aux.clear();
    for (int l = 0; l < M->L; l++) {
        Layer& y = M->layers[l];
        M->mv_aux.push_back(MvArgs{});
        M->wg_aux.push_back(0);
        if (y.recurrent) {
            // Gated-DeltaNet input: mix (q|k|v), z gate and beta|alpha in one launch
            MvArgs q = mv_base(M->h, y.attn_norm, M->eps, M->H, MV_STORE, M->d_ctl);
            q.waves = 8;
            q.items_per_wave = one_pass_ipw((M->channels + M->inner + 2 * M->ssm_hv) / 2, q.waves, n_cu);
            q.nseg = 3;
            q.type_a = y.gdn_mix.type;
            q.type_b = y.gdn_ba.type;
            q.seg[0].w = y.gdn_mix; q.seg[0].out = M->mixed;
            q.seg[1].w = y.gdn_z; q.seg[1].out = M->zbuf;
            q.seg[2].w = y.gdn_ba; q.seg[2].out = M->ba;
            M->wg_qkv.push_back(layout_segments(q));
            M->mv_qkv.push_back(q);
            MvArgs o = mv_base(M->gated, nullptr, 0.f, M->inner, MV_ADD, M->d_ctl);   // ssm_out + residual
            o.nseg = 1;
            o.seg[0].w = y.o; o.seg[0].out = M->h;
            o.type_a = o.type_b = y.o.type;
            o.waves = 8;
            o.items_per_wave = one_pass_ipw(M->H / 2, o.waves, n_cu);
            M->wg_o.push_back(layout_segments(o));
            M->mv_o.push_back(o);
        } else {
        MvArgs q = mv_base(M->h, y.attn_norm, M->eps, M->H, MV_STORE, M->d_ctl);
        q.waves = 8;
        q.items_per_wave = one_pass_ipw((qd + 2 * kd) / 2, q.waves, n_cu);
        q.nseg = 3;
        q.type_a = y.q.type;
        q.type_b = y.v.type;
        q.seg[0].w = y.q; q.seg[0].out = M->raw; q.seg[0].bias = y.q_bias;
        q.seg[1].w = y.k; q.seg[1].out = M->raw + qd; q.seg[1].bias = y.k_bias;
        q.seg[2].w = y.v; q.seg[2].out = M->raw + qd + kd; q.seg[2].bias = y.v_bias;
        {   // k and v: as many items per wave as keep a wave's bytes at most q's, so
            // the smaller segments fill the CUs q leaves free without becoming the slowest
            const double bq = qrow_bytes(y.q);
            q.seg[1].ipw = std::max(1, (int)(q.items_per_wave * bq / qrow_bytes(y.k)));
            q.seg[2].ipw = std::max(1, (int)(q.items_per_wave * bq / qrow_bytes(y.v)));
        }
        M->wg_qkv.push_back(layout_segments(q));
        M->mv_qkv.push_back(q);

        MvArgs o = mv_base(M->attn, nullptr, 0.f, qd, MV_ADD, M->d_ctl);
        o.nseg = 1;
        o.seg[0].w = y.o; o.seg[0].out = M->h;
        o.type_a = o.type_b = y.o.type;
        o.waves = 8;
        o.items_per_wave = one_pass_ipw(M->H / 2, o.waves, n_cu);
        M->wg_o.push_back(layout_segments(o));
        M->mv_o.push_back(o);
        if (M->hybrid) {   // gated attention: the gate half of attn_q, from the same normed input
            MvArgs ga = mv_base(M->h, y.attn_norm, M->eps, M->H, MV_STORE, M->d_ctl);
            ga.nseg = 1;
            ga.seg[0].w = y.q_gate; ga.seg[0].out = M->att_gate;
            ga.type_a = ga.type_b = y.q_gate.type;
            ga.waves = 8;
            ga.items_per_wave = one_pass_ipw(qd / 2, ga.waves, n_cu);
            M->wg_aux.back() = layout_segments(ga);
            M->mv_aux.back() = ga;
        }
        }

        MvArgs g = mv_base(M->h, y.ffn_norm, M->eps, M->H, MV_SILU, M->d_ctl);
        g.nseg = 1;
        g.seg[0].w = y.gate; g.seg[0].w2 = y.up; g.seg[0].out = M->act;
        g.type_a = g.type_b = y.gate.type;
        g.waves = 8;
        g.items_per_wave = one_pass_ipw(M->F, g.waves, n_cu);
        M->wg_gu.push_back(layout_segments(g));
        M->mv_gu.push_back(g);

        MvArgs d = mv_base(M->act, nullptr, 0.f, M->F, MV_ADD, M->d_ctl);
        d.nseg = 1;
        d.seg[0].w = y.down; d.seg[0].out = M->h;
        d.type_a = d.type_b = y.down.type;
        d.waves = 8;
        d.items_per_wave = one_pass_ipw(M->H / 2, d.waves, n_cu);
        M->wg_down.push_back(layout_segments(d));
        M->mv_down.push_back(d);
    }
    MvArgs hdv = mv_base(M->h, M->out_norm, M->eps, M->H, MV_HEAD, M->d_ctl);
    hdv.nseg = 1;
    hdv.seg[0].w = M->out; hdv.seg[0].out = M->logits;
    hdv.type_a = hdv.type_b = M->out.type;
    // the head also runs in a single pass of workgroups (8B, 151936 rows: 250
    // workgroups of 8 waves x 38 items, 93.4 us against 99.0 us for 2374
    // workgroups of 4 waves x 8 items); it has no addends, so no 32-item limit
    hdv.waves = 8;
    hdv.items_per_wave = one_pass_ipw((M->V + 1) / 2, hdv.waves, n_cu, 64);
    hdv.head.partial = M->head_partial;
    hdv.head.counter = M->counters + M->hkv;
    M->head_wgs = layout_segments(hdv);
    M->mv_head = hdv;
}

// The bs1 chain merges more than kDeferMaxSplits split partials in a separate
// launch (attention_merge_kernel) when the geometry allows it.
bool merge_apart_for(const ribn_rocm_model* M, int n_splits) {
    return !M->hybrid && !M->merge_in_launch && n_splits > kDeferMaxSplits && n_splits <= kMergeMaxSplits &&
           (M->hd == 64 || M->hd == 128);
}

AttnArgs attn_args(ribn_rocm_model* M, int l, int n_splits) {
    AttnArgs at{};
    const Layer& y = M->layers[l];
    at.raw = M->raw;
    at.q_norm = y.q_norm;
    at.k_norm = y.k_norm;
    at.rope = M->rope;
    at.kcache = y.kc;
    at.vcache = y.vc;
    at.part = M->part;
    at.counters = M->counters;
    at.out = M->attn;
    at.ctl = M->d_ctl;
    at.hq = M->hq; at.hkv = M->hkv; at.hd = M->hd; at.rot = M->rot;
    at.n_splits = n_splits;
    at.kv_f16 = M->kv_f16 ? 1 : 0;
    at.eps = M->eps;
    at.scale_log2 = 1.4426950408889634f / std::sqrt((float)M->hd);
    return at;
}

size_t align_floats(size_t n) { return (n + 63) / 64 * 64; }   // 256-byte sub-buffers

// Persistent-step configuration: a compiled kernel must exist for the model's
// value types, head dimension, query heads per KV head and KV element type,
// with every layer using the same types. Activations go to a per-step arena
// where every stage has its own buffer (see step.h).
hipError_t build_step(ribn_rocm_model* M, bool allow) {
    M->step_wg = 0;
    if (!allow || M->hybrid) return hipSuccess;   // the persistent step has no recurrent stages
    const Layer& y0 = M->layers[0];
    StepKey key{(int)y0.q.type, (int)y0.v.type, (int)y0.o.type, (int)y0.gate.type, (int)y0.down.type,
                (int)M->out.type, M->hd, M->hq / M->hkv, M->kv_f16 ? 1 : 0};
    for (const Layer& y : M->layers)
        if ((int)y.q.type != key.qa || (int)y.v.type != key.qb || (int)y.o.type != key.o ||
            (int)y.gate.type != key.gu || (int)y.down.type != key.dn)
            return hipSuccess;
    size_t lds = 0;
    const int max_k = std::max(std::max(M->H, M->F), M->hq * M->hd);
    const int n_wg = step_grid(key, max_k, M->device, &lds);
    if (n_wg < 64) return hipSuccess;

    const int qd = M->hq * M->hd, kd = M->hkv * M->hd;
    const size_t s_raw = align_floats(qd + 2 * kd), s_attn = align_floats(qd), s_h = align_floats(M->H),
                 s_act = align_floats(M->F);
    const size_t per_layer = s_raw + s_attn + 2 * s_h + s_act;
    float* arena = nullptr;
    hipError_t e = dalloc(M, &arena, sizeof(float) * (s_h + per_layer * M->L));
    if (e != hipSuccess) return e;
    M->arena_h0 = arena;
    M->arena_h2.assign(M->L, nullptr);
    std::vector<LayerDev> ld(M->L);
    const float* prev = M->arena_h0;
    for (int l = 0; l < M->L; l++) {
        float* base = arena + s_h + per_layer * l;
        float *raw = base, *att = raw + s_raw, *h1 = att + s_attn, *act = h1 + s_h, *h2 = act + s_act;
        LayerDev& L = ld[l];
        L.qkv = M->mv_qkv[l];
        L.qkv.x = prev;
        L.qkv.seg[0].out = raw; L.qkv.seg[1].out = raw + qd; L.qkv.seg[2].out = raw + qd + kd;
        for (auto& sg : L.qkv.seg) sg.res = nullptr;
        if (layout_grid(L.qkv, n_wg) < 0) return hipSuccess;   // no persistent step for this shape
        L.attn = attn_args(M, l, 1);
        L.attn.raw = raw;
        L.attn.out = att;
        L.o = M->mv_o[l];
        L.o.x = att;
        L.o.seg[0].out = h1;
        L.o.seg[0].res = prev;
        if (layout_grid(L.o, n_wg) < 0) return hipSuccess;   // no persistent step for this shape
        L.gu = M->mv_gu[l];
        L.gu.x = h1;
        L.gu.seg[0].out = act;
        L.gu.seg[0].res = nullptr;
        if (layout_grid(L.gu, n_wg) < 0) return hipSuccess;   // no persistent step for this shape
        L.down = M->mv_down[l];
        L.down.x = act;
        L.down.seg[0].out = h2;
        L.down.seg[0].res = h1;
        if (layout_grid(L.down, n_wg) < 0) return hipSuccess;   // no persistent step for this shape
        M->arena_h2[l] = h2;
        prev = h2;
    }
    e = dalloc(M, &M->d_layers, sizeof(LayerDev) * M->L);
    if (e == hipSuccess) e = hipMemcpy(M->d_layers, ld.data(), sizeof(LayerDev) * M->L, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = dalloc(M, &M->step_bar, kStepBarBytes);
    if (e == hipSuccess) e = hipMemset(M->step_bar, 0, kStepBarBytes);
    if (e != hipSuccess) return e;
    int clock_khz = 0;
    if ((e = hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, M->device)) != hipSuccess) return e;
    StepArgs& a = M->step_args;
    a = StepArgs{};
    a.layers = M->d_layers;
    a.n_layers = M->L;
    a.embed.w = M->embd;
    a.embed.hidden = M->H;
    a.embed.h = M->arena_h0;
    a.embed.ctl = M->d_ctl;
    a.embed.inv_freq = M->inv_freq;
    a.embed.rope = M->rope;
    a.embed.half_rot = M->rot / 2;
    a.head_mv = M->mv_head;
    a.head_mv.x = prev;
    a.head_mv.seg[0].res = nullptr;
    if (layout_grid(a.head_mv, n_wg) < 0) return hipSuccess;
    a.bar = M->step_bar;
    a.timeout_ticks = (uint64_t)(clock_khz > 0 ? clock_khz : 100000) * 1000ull * 2ull;   // 2 s
    a.ctl = M->d_ctl;
    M->step_key = key;
    M->step_lds = lds;
    M->step_wg = n_wg;
    return hipSuccess;
}

GdnArgs gdn_args(ribn_rocm_model* M, int l) {
    const Layer& y = M->layers[l];
    GdnArgs a{};
    a.mixed = M->mixed; a.z = M->zbuf; a.ba = M->ba;
    a.dt_bias = y.dt_bias; a.ssm_a = y.ssm_a; a.conv_w = y.conv_w; a.ssm_norm = y.ssm_norm;
    a.act = M->gdn_act; a.gated = M->gated; a.ctl = M->d_ctl;
    a.state_off = y.state_off; a.conv_off = y.conv_off;
    a.hk = M->ssm_hk; a.hv = M->ssm_hv; a.d = M->ssm_d; a.conv_k = M->conv_k; a.eps = M->eps;
    return a;
}

// One step of the token loop for the active sequence (decode.rs:550-640):
// embedding (+rope table) -> L x [QKV(+norm) -> attention(+q/k norm, rope, KV
// append) -> O(+residual) -> gate/up(+norm,+SwiGLU) -> down(+residual)]
// -> head(+norm,+argmax) or advance.
hipError_t enqueue_step(ribn_rocm_model* M, bool head, int n_splits, float* trace) {
    hipStream_t st = M->stream;
    EmbedArgs ea{};
    ea.w = M->embd;
    ea.hidden = M->H;
    ea.h = M->h;
    ea.ctl = M->d_ctl;
    ea.inv_freq = M->inv_freq;
    ea.rope = M->rope;
    ea.half_rot = M->rot / 2;
    hipError_t e = launch_embed(ea, st);
    if (e != hipSuccess) return e;
    if (trace && (e = hipMemcpyAsync(trace, M->h, sizeof(float) * M->H, hipMemcpyDeviceToDevice, st)) != hipSuccess)
        return e;
    AttnArgs at = attn_args(M, 0, n_splits);
    // At a few splits (short contexts, where the launch is latency-bound) the
    // o projection merges the attention's split partials while it stages its
    // input, which saves the attention launch its arrival count and merge round
    // trips. Gated attention multiplies the merged output first, so hybrids merge
    // in the attention launch.
    const bool defer = !M->hybrid && n_splits > 1 && n_splits <= kDeferMaxSplits;
    // Long contexts (more splits than the projection merges) merge the partials
    // in a launch of their own, one wave per query head: the attention launch's
    // last workgroup per KV head took ~10 us for 32 splits at G = 8.
    const bool merge_apart = merge_apart_for(M, n_splits);
    for (int l = 0; l < M->L; l++) {
        const Layer& y = M->layers[l];
        if ((e = launch_matvec(M->mv_qkv[l], M->wg_qkv[l], st)) != hipSuccess) return e;
        if (y.recurrent) {
            if ((e = launch_gdn(gdn_args(M, l), st)) != hipSuccess) return e;
        } else {
            if (M->hybrid && (e = launch_matvec(M->mv_aux[l], M->wg_aux[l], st)) != hipSuccess) return e;
            at = attn_args(M, l, n_splits);
            at.defer = defer ? 1 : merge_apart ? 2 : 0;
            if ((e = launch_attention(at, st)) != hipSuccess) return e;
            if (merge_apart && (e = launch_attention_merge(at, st)) != hipSuccess) return e;
            if (M->hybrid && (e = launch_gate_mul(M->attn, M->att_gate, M->hq * M->hd, st)) != hipSuccess) return e;
        }
        MvArgs o = M->mv_o[l];
        if (defer && !y.recurrent) {
            o.parts = M->part;
            o.parts_splits = n_splits;
            o.parts_g = M->hq / M->hkv;
            o.parts_hd = M->hd;
        }
        if ((e = launch_matvec(o, M->wg_o[l], st)) != hipSuccess) return e;
        if (M->gu_clk) e = launch_matvec_clocked(M->mv_gu[l], M->wg_gu[l], M->gu_clk + 2 * l, st);
        else e = launch_matvec(M->mv_gu[l], M->wg_gu[l], st);
        if (e != hipSuccess) return e;
        if ((e = launch_matvec(M->mv_down[l], M->wg_down[l], st)) != hipSuccess) return e;
        if (trace &&
            (e = hipMemcpyAsync(trace + (size_t)(l + 1) * M->H, M->h, sizeof(float) * M->H, hipMemcpyDeviceToDevice, st)) !=
                hipSuccess)
            return e;
    }
    if (head) return launch_matvec(M->mv_head, M->head_wgs, st);
    return launch_advance(M->d_ctl, st);
}

// RIBN_ROCM_EAGER=1 launches the chain directly instead of replaying graphs
// (same kernels and arguments). Used for profiler runs: rocprofv3's kernel
// tracer crashes the host process inside HIP graph capture on this image.
bool eager_mode() {
    static const bool eager = [] {
        const char* v = std::getenv("RIBN_ROCM_EAGER");
        return v && v[0] == '1';
    }();
    return eager;
}

hipError_t graph_step(ribn_rocm_model* M, bool head, int ctx) {
    const int ns = splits_for_ctx(ctx);
    if (eager_mode()) return enqueue_step(M, head, ns, nullptr);
    const int key = ns * 2 + (head ? 1 : 0);
    auto it = M->graphs.find(key);
    if (it == M->graphs.end()) {
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return e;
        hipError_t e2 = enqueue_step(M, head, ns, nullptr);
        e = hipStreamEndCapture(M->stream, &g);
        if (e2 != hipSuccess) { if (g) hipGraphDestroy(g); return e2; }
        if (e != hipSuccess) return e;
        hipGraphExec_t ex = nullptr;
        e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (e != hipSuccess) return e;
        it = M->graphs.emplace(key, ex).first;
    }
    return hipGraphLaunch(it->second, M->stream);
}

// A prefill / batched-decode projection: the dequantizing MFMA GEMM, or with
// resident binary16 weights (w16, n output rows, optional concatenated bias) a
// hipBLASLt GEMM followed by the fused step as its own launch.
hipError_t run_gemm(ribn_rocm_model* M, const PrefillGemm& g, const uint16_t* w16, int n, const float* bias,
                    hipStream_t st) {
    if (!M->blas || !w16) return launch_prefill_gemm(g, st);
    hipError_t e = blas_gemm(M->blas, g.x, g.m, g.k, w16, n, g.y, g.ldy, g.mode == MV_ADD, bias, st);
    if (e == hipErrorNotSupported) return launch_prefill_gemm(g, st);   // no library kernel for this shape
    if (e != hipSuccess) return e;
    if (g.post == GEMM_POST_RMS_F16)
        return launch_rows_rms_f16(g.y, g.m, g.ldy, g.post_w, g.post_eps, true, g.post_out, g.ldy, st);
    if (g.post == GEMM_POST_SILU_F16) return launch_silu_mul_f16(g.y, g.ldy / 2, g.m, g.post_out, st);
    return hipSuccess;
}

// One prefill chunk of the sequence in `slot`: rows pos0 .. pos0 + m - 1 of its
// token array through every layer (prefill_chunk, nvidia/src/decode.rs:2124).
// final: the last row's hidden state goes through the head and its greedy
// token is written at pos0 + m (sampled-final, decode.rs:807-840); else the
// position just advances. trace (device, optional): hidden rows after the
// embedding and after every layer, [(L + 1)][m][hidden].
hipError_t prefill_chunk(ribn_rocm_model* M, int slot, int pos0, int m, bool final, float* trace) {
    hipStream_t st = M->stream;
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd, ldq = qd + 2 * kd;
    const uint32_t* toks = M->d_tokens + (size_t)slot * (M->context + 1) + pos0;
    hipError_t e = launch_embed_rows(M->embd, toks, m, M->H, M->p_h, st);
    if (e != hipSuccess) return e;
    auto snap = [&](int i) {
        return trace ? hipMemcpyAsync(trace + (size_t)i * m * M->H, M->p_h, sizeof(float) * m * M->H,
                                      hipMemcpyDeviceToDevice, st)
                     : hipSuccess;
    };
    if ((e = snap(0)) != hipSuccess) return e;
    PrefillRows rows{};
    rows.qkv = M->p_qkv;
    rows.ld_qkv = ldq;
    rows.qout = M->p_q;
    rows.attn16 = M->p_att16;
    rows.m = m;
    rows.pos0 = pos0;
    rows.hq = M->hq; rows.hkv = M->hkv; rows.hd = M->hd; rows.rot = M->rot;
    rows.kv_f16 = M->kv_f16 ? 1 : 0;
    rows.inv_freq = M->inv_freq;
    rows.eps = M->eps;
    rows.pages = M->d_pages + (size_t)slot * M->max_pages;
    // one launch per input: q|k|v, attn_output, gate|up, down
    auto gemm = [&](const uint16_t* x, int k, float* y, int ldy, int mode, std::initializer_list<PrefillSeg> segs,
                    int post = GEMM_POST_NONE, const float* post_w = nullptr, uint16_t* post_out = nullptr,
                    const uint16_t* w16 = nullptr, const float* bias16 = nullptr) {
        PrefillGemm g{};
        g.x = x; g.m = m; g.k = k; g.y = y; g.ldy = ldy; g.res = y; g.mode = mode;
        g.post = post; g.post_w = post_w; g.post_eps = M->eps; g.post_out = post_out;
        int tiles = 0;
        for (const PrefillSeg& sg : segs) {
            g.seg[g.nseg] = sg;
            g.seg[g.nseg].tile0 = tiles;
            tiles += gemm_tiles((int)sg.w.rows);
            g.nseg++;
        }
        g.ksplit = prefill_gemm_splits(m, k, tiles);
        if (g.ksplit > 1 && (size_t)g.ksplit * m * ldy <= M->p_part_floats) g.part = M->p_part;
        else g.ksplit = 1;
        return run_gemm(M, g, w16, ldy, bias16, st);
    };
    for (int l = 0; l < M->L; l++) {
        const Layer& y = M->layers[l];
        // layer l > 0 receives its normed input from the previous down GEMM
        if (l == 0 &&
            (e = launch_rows_rms_f16(M->p_h, m, M->H, y.attn_norm, M->eps, true, M->p_x16, M->H, st)) != hipSuccess)
            return e;
        if ((e = gemm(M->p_x16, M->H, M->p_qkv, ldq, MV_STORE,
                      {PrefillSeg{y.q, 0, 0, y.q_bias}, PrefillSeg{y.k, qd, 0, y.k_bias},
                       PrefillSeg{y.v, qd + kd, 0, y.v_bias}},
                      GEMM_POST_NONE, nullptr, nullptr, y.w16_qkv, y.qkv_bias)) != hipSuccess)
            return e;
        rows.q_norm = y.q_norm;
        rows.k_norm = y.k_norm;
        rows.kcache = y.kc;
        rows.vcache = y.vc;
        if ((e = launch_qk_rope_append(rows, st)) != hipSuccess) return e;
        if ((e = launch_prefill_attention(rows, st)) != hipSuccess) return e;
        if ((e = gemm(M->p_att16, qd, M->p_h, M->H, MV_ADD, {PrefillSeg{y.o, 0, 0, nullptr}}, GEMM_POST_RMS_F16,
                      y.ffn_norm, M->p_x16, y.w16_o)) != hipSuccess)
            return e;
        if ((e = gemm(M->p_x16, M->H, M->p_gu, 2 * M->F, MV_STORE,
                      {PrefillSeg{y.gate, 0, 0, nullptr}, PrefillSeg{y.up, M->F, 0, nullptr}}, GEMM_POST_SILU_F16, nullptr,
                      M->p_act16, y.w16_gu)) != hipSuccess)
            return e;
        const bool more = l + 1 < M->L;
        if ((e = gemm(M->p_act16, M->F, M->p_h, M->H, MV_ADD, {PrefillSeg{y.down, 0, 0, nullptr}},
                      more ? GEMM_POST_RMS_F16 : GEMM_POST_NONE, more ? M->layers[l + 1].attn_norm : nullptr,
                      M->p_x16, y.w16_down)) != hipSuccess)
            return e;
        if ((e = snap(l + 1)) != hipSuccess) return e;
    }
    SeqState* seq = &M->d_slots[slot];
    if (!final) return launch_set_pos(seq, pos0 + m, st);
    e = hipMemcpyAsync(M->h, M->p_h + (size_t)(m - 1) * M->H, sizeof(float) * M->H, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = launch_set_pos(seq, pos0 + m - 1, st);
    if (e == hipSuccess) e = launch_matvec(M->mv_head, M->head_wgs, st);
    return e;
}

int device_cus() {
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    return n;
}

// The layers and head of the decode rows in the integer-dot mode (the
// reference's GemvMode::IntegerDot, nvidia/src/decode.rs:298-312; its batched
// executor gemv_batch, decode.rs:1591-1633, 2250-2520): each projection's input
// rows are packed to Q8_1 (with the RMSNorm before it fused into the packing),
// then the integer-dot matvec reads the weights once for every group of at
// most kIdMaxMembers rows. Attention, rope, the caches and the argmax are those
// of the float rows; the embedding rows are in p_h.
hipError_t intdot_rows(ribn_rocm_model* M, const DecodeRows& dr, int n_splits) {
    hipStream_t st = M->stream;
    const int n = dr.rows;
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd, ldq = qd + 2 * kd;
    const int n_cu = device_cus();
    auto seg = [](const QMat& w, float* out, const float* bias = nullptr, const float* res = nullptr) {
        MvSeg sg{};
        sg.w = w;
        sg.out = out;
        sg.bias = bias;
        sg.res = res;
        return sg;
    };
    auto proj = [&](const float* x, int k, const float* norm_w, int mode, std::initializer_list<MvSeg> segs, int ld) {
        const size_t words = (size_t)(k / 32) * 9;
        hipError_t e = launch_q8_1_rows(x, k, n, k, norm_w, M->eps, M->b_xq, st);
        for (int r0 = 0; e == hipSuccess && r0 < n; r0 += kIdMaxMembers) {
            IdArgs a{};
            a.xq = M->b_xq + (size_t)r0 * words;
            a.k = k;
            a.members = std::min(kIdMaxMembers, n - r0);
            a.ld = ld;
            a.mode = mode;
            for (MvSeg sg : segs) {
                sg.out += (size_t)r0 * ld;
                if (sg.res) sg.res += (size_t)r0 * ld;
                a.seg[a.nseg++] = sg;
            }
            a.type_a = a.seg[0].w.type;
            a.type_b = a.seg[a.nseg - 1].w.type;
            e = launch_intdot(a, intdot_layout(a, n_cu), st);
        }
        return e;
    };
    hipError_t e = hipSuccess;
    for (int l = 0; l < M->L; l++) {
        const Layer& y = M->layers[l];
        if ((e = proj(M->p_h, M->H, y.attn_norm, MV_STORE,
                      {seg(y.q, M->p_qkv, y.q_bias), seg(y.k, M->p_qkv + qd, y.k_bias),
                       seg(y.v, M->p_qkv + qd + kd, y.v_bias)},
                      ldq)) != hipSuccess)
            return e;
        AttnArgs at = attn_args(M, l, n_splits);
        if ((e = launch_attention_rows(at, dr, st)) != hipSuccess) return e;
        if ((e = proj(M->b_att, qd, nullptr, MV_ADD, {seg(y.o, M->p_h, nullptr, M->p_h)}, M->H)) != hipSuccess) return e;
        MvSeg gu = seg(y.gate, M->b_act);
        gu.w2 = y.up;
        if ((e = proj(M->p_h, M->H, y.ffn_norm, MV_SILU, {gu}, M->F)) != hipSuccess) return e;
        if ((e = proj(M->b_act, M->F, nullptr, MV_ADD, {seg(y.down, M->p_h, nullptr, M->p_h)}, M->H)) != hipSuccess)
            return e;
    }
    if ((e = proj(M->p_h, M->H, M->out_norm, MV_STORE, {seg(M->out, M->b_logits)}, M->V)) != hipSuccess) return e;
    return launch_rows_argmax_commit(M->b_logits, M->V, dr, M->d_slots, M->b_argmax, st);
}

// Float decode rows of a few sequences (up to kMatvecRowsMax): the projections
// run as the batch-1 matvec launches with several input rows, each weight
// unit read from HBM once and applied to every row (groups of at most
// matvec_max_rows(k) rows per launch). Each row's arithmetic is the batch-1
// step's own, so a row's logits equal those of the same sequence stepped alone.
constexpr int kMatvecRowsMax = 4;

hipError_t matvec_rows(ribn_rocm_model* M, const DecodeRows& dr, int n_splits) {
    hipStream_t st = M->stream;
    const int n = dr.rows;
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd, ldq = qd + 2 * kd;
    // one projection over rows [0, n): x rows ldx apart; segment outputs (and
    // residuals) moved to row r0 at ldo floats per row
    auto proj = [&](MvArgs a, int n_wg, const float* x, int ldx, const float* norm_w, int ldo, int mode,
                    std::initializer_list<std::pair<float*, const float*>> outs) {
        a.norm_w = norm_w;
        a.mode = mode;
        a.parts = nullptr;
        a.ldx = ldx;
        a.ldo = ldo;
        const int step = matvec_max_rows(a.k);
        hipError_t e = hipSuccess;
        for (int r0 = 0; e == hipSuccess && r0 < n; r0 += step) {
            MvArgs b = a;
            b.rows = std::min(step, n - r0);
            b.x = x + (size_t)r0 * ldx;
            int i = 0;
            for (const auto& o : outs) {
                b.seg[i].out = o.first + (size_t)r0 * ldo;
                b.seg[i].res = o.second ? o.second + (size_t)r0 * ldo : nullptr;
                i++;
            }
            e = launch_matvec(b, n_wg, st);
        }
        return e;
    };
    hipError_t e = hipSuccess;
    for (int l = 0; l < M->L; l++) {
        const Layer& y = M->layers[l];
        if ((e = proj(M->mv_qkv[l], M->wg_qkv[l], M->p_h, M->H, y.attn_norm, ldq, MV_STORE,
                      {{M->p_qkv, nullptr}, {M->p_qkv + qd, nullptr}, {M->p_qkv + qd + kd, nullptr}})) != hipSuccess)
            return e;
        AttnArgs at = attn_args(M, l, n_splits);
        if ((e = launch_attention_rows(at, dr, st)) != hipSuccess) return e;
        if ((e = proj(M->mv_o[l], M->wg_o[l], M->b_att, qd, nullptr, M->H, MV_ADD, {{M->p_h, M->p_h}})) != hipSuccess)
            return e;
        if ((e = proj(M->mv_gu[l], M->wg_gu[l], M->p_h, M->H, y.ffn_norm, M->F, MV_SILU, {{M->b_act, nullptr}})) !=
            hipSuccess)
            return e;
        if ((e = proj(M->mv_down[l], M->wg_down[l], M->b_act, M->F, nullptr, M->H, MV_ADD, {{M->p_h, M->p_h}})) !=
            hipSuccess)
            return e;
    }
    if ((e = proj(M->mv_head, M->head_wgs, M->p_h, M->H, M->out_norm, M->V, MV_STORE, {{M->b_logits, nullptr}})) !=
        hipSuccess)
        return e;
    return launch_rows_argmax_commit(M->b_logits, M->V, dr, M->d_slots, M->b_argmax, st);
}

// The projections of batched decode rows run as the chunked-prefill MFMA GEMMs
// over the rows (or the integer-dot matvec); attention is the split-K decode
// kernel over each row's own cache; the head is one GEMM over the rows followed
// by a per-row argmax.
// The launches of a decode-rows step for n rows and a split dimension of
// n_splits: they read the rows' slots and positions from d_brows only, so one
// captured graph serves every step with the same (n, n_splits).
hipError_t decode_rows_body(ribn_rocm_model* M, int n, int n_splits) {
    hipStream_t st = M->stream;
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd, ldq = qd + 2 * kd;
    hipError_t e = hipSuccess;
    DecodeRows dr{};
    dr.rows = n;
    dr.slot = M->d_brows;
    dr.pos = M->d_brows + n;
    dr.pages = M->d_pages;
    dr.max_pages = M->max_pages;
    dr.raw = M->p_qkv;
    dr.ld_raw = ldq;
    dr.out = M->b_att;
    dr.ld_out = qd;
    dr.rope = M->b_rope;
    dr.part = M->b_part;
    dr.part_stride = M->b_part_stride;
    dr.counters = M->b_counters;
    // splits per row: the rows (x KV heads) already spread the work over the
    // GPU, so a split covers up to kMaxSplitTokens positions (measured on
    // 256-position splits 11.1k aggregate tok/s with the current
    // GEMMs, 512 11.8k, 1024 12.2k, 2048 12.2k)
    dr.split_tokens = kMaxSplitTokens;
    if ((e = launch_gather_row_tokens(M->d_tokens, M->context + 1, dr, M->d_btokens, st)) != hipSuccess) return e;
    if ((e = launch_embed_rows(M->embd, M->d_btokens, n, M->H, M->p_h, st)) != hipSuccess) return e;
    if ((e = launch_rope_rows(M->inv_freq, M->rot, dr, st)) != hipSuccess) return e;
    if (M->int_dot) return intdot_rows(M, dr, n_splits);
    if (n <= kMatvecRowsMax) return matvec_rows(M, dr, n_splits);
    auto gemm = [&](const uint16_t* x, int k, float* y, int ldy, int mode, std::initializer_list<PrefillSeg> segs,
                    int post = GEMM_POST_NONE, const float* post_w = nullptr, uint16_t* post_out = nullptr,
                    const uint16_t* w16 = nullptr, const float* bias16 = nullptr) {
        PrefillGemm g{};
        g.x = x; g.m = n; g.k = k; g.y = y; g.ldy = ldy; g.res = y; g.mode = mode;
        g.post = post; g.post_w = post_w; g.post_eps = M->eps; g.post_out = post_out;
        int tiles = 0;
        for (const PrefillSeg& sg : segs) {
            g.seg[g.nseg] = sg;
            g.seg[g.nseg].tile0 = tiles;
            tiles += gemm_tiles((int)sg.w.rows);
            g.nseg++;
        }
        g.ksplit = prefill_gemm_splits(n, k, tiles);
        if (g.ksplit > 1 && (size_t)g.ksplit * n * ldy <= M->p_part_floats) g.part = M->p_part;
        else g.ksplit = 1;
        return run_gemm(M, g, w16, ldy, bias16, st);
    };
    for (int l = 0; l < M->L; l++) {
        const Layer& y = M->layers[l];
        // layer l > 0 receives its normed input from the previous down GEMM
        if (l == 0 &&
            (e = launch_rows_rms_f16(M->p_h, n, M->H, y.attn_norm, M->eps, true, M->p_x16, M->H, st)) != hipSuccess)
            return e;
        if ((e = gemm(M->p_x16, M->H, M->p_qkv, ldq, MV_STORE,
                      {PrefillSeg{y.q, 0, 0, y.q_bias}, PrefillSeg{y.k, qd, 0, y.k_bias},
                       PrefillSeg{y.v, qd + kd, 0, y.v_bias}},
                      GEMM_POST_NONE, nullptr, nullptr, y.w16_qkv, y.qkv_bias)) != hipSuccess)
            return e;
        AttnArgs at = attn_args(M, l, n_splits);
        if ((e = launch_attention_rows(at, dr, st)) != hipSuccess) return e;
        if ((e = launch_rows_rms_f16(M->b_att, n, qd, nullptr, 0.f, false, M->p_att16, qd, st)) != hipSuccess) return e;
        if ((e = gemm(M->p_att16, qd, M->p_h, M->H, MV_ADD, {PrefillSeg{y.o, 0, 0, nullptr}}, GEMM_POST_RMS_F16,
                      y.ffn_norm, M->p_x16, y.w16_o)) != hipSuccess)
            return e;
        if ((e = gemm(M->p_x16, M->H, M->p_gu, 2 * M->F, MV_STORE,
                      {PrefillSeg{y.gate, 0, 0, nullptr}, PrefillSeg{y.up, M->F, 0, nullptr}}, GEMM_POST_SILU_F16, nullptr,
                      M->p_act16, y.w16_gu)) != hipSuccess)
            return e;
        // the last layer's down GEMM norms the rows for the head
        const float* next_norm = l + 1 < M->L ? M->layers[l + 1].attn_norm : M->out_norm;
        if ((e = gemm(M->p_act16, M->F, M->p_h, M->H, MV_ADD, {PrefillSeg{y.down, 0, 0, nullptr}}, GEMM_POST_RMS_F16,
                      next_norm, M->p_x16, y.w16_down)) != hipSuccess)
            return e;
    }
    if ((e = gemm(M->p_x16, M->H, M->b_logits, M->V, MV_STORE, {PrefillSeg{M->out, 0, 0, nullptr}}, GEMM_POST_NONE,
                  nullptr, nullptr, M->w16_head)) != hipSuccess)
        return e;
    return launch_rows_argmax_commit(M->b_logits, M->V, dr, M->d_slots, M->b_argmax, st);
}

// One decode row per sequence, all in one step (batched decode): row r
// consumes the token at position pos[r] of the sequence in slot[r] and samples
// the next one. The rows go to d_brows, then the step's launches replay from a
// HIP graph keyed by (rows, splits) (captured on first use; eager with
// RIBN_ROCM_EAGER=1 or resident binary16 weights, whose library GEMMs stay out
// of graphs).
hipError_t decode_rows(ribn_rocm_model* M, const std::vector<int>& slots, const std::vector<int>& pos) {
    hipStream_t st = M->stream;
    const int n = (int)slots.size();
    int max_ctx = 0;
    for (int r = 0; r < n; r++) {
        M->h_brows[r] = slots[r];
        M->h_brows[n + r] = pos[r];
        max_ctx = std::max(max_ctx, pos[r] + 1);
    }
    hipError_t e = hipMemcpyAsync(M->d_brows, M->h_brows.data(), sizeof(int32_t) * 2 * n, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return e;
    const int n_splits = rows_splits(max_ctx, kMaxSplitTokens);   // the grid's split dimension
    if (eager_mode() || M->blas) return decode_rows_body(M, n, n_splits);
    const int key = n * 64 + n_splits;
    auto it = M->row_graphs.find(key);
    if (it == M->row_graphs.end()) {
        hipGraph_t g = nullptr;
        e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return e;
        hipError_t e2 = decode_rows_body(M, n, n_splits);
        e = hipStreamEndCapture(st, &g);
        if (e2 != hipSuccess) { if (g) hipGraphDestroy(g); return e2; }
        if (e != hipSuccess) return e;
        hipGraphExec_t ex = nullptr;
        e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (e != hipSuccess) return e;
        it = M->row_graphs.emplace(key, ex).first;
    }
    return hipGraphLaunch(it->second, st);
}

// Prompt rows pos0 .. pos0 + n - 1 of the sequence in `slot` in chunks of at
// most M->chunk rows; the last chunk samples the next token when `final`.
hipError_t run_step(ribn_rocm_model* M, bool head, int ctx, float* trace);

hipError_t prefill_rows(ribn_rocm_model* M, int slot, int pos0, int n, bool final) {
    if (M->hybrid) {
        // the recurrent layers advance one token at a time: prompt rows run as decode
        // steps (the reference's default prefill lane; its chunk scan is opt-in,
        // decode.rs gdn_chunk_scan), the last one sampling when `final`
        for (int p = 0; p < n; p++) {
            hipError_t e = run_step(M, final && p + 1 == n, pos0 + p + 1, nullptr);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    for (int p = 0; p < n; p += M->chunk) {
        const int m = std::min(M->chunk, n - p);
        hipError_t e = prefill_chunk(M, slot, pos0 + p, m, final && p + m == n, nullptr);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// One token step of the active sequence: the persistent step kernel when the
// model has one, else the launch chain (graph replay; eager when tracing).
// trace (device, (L+1) x hidden): residual stream after the embedding and
// after every layer.
hipError_t run_step(ribn_rocm_model* M, bool head, int ctx, float* trace) {
    // integer-dot mode: a sampled step of the active sequence is a decode row
    if (M->int_dot && head && !trace) return decode_rows(M, {M->cur_slot}, {ctx - 1});
    if (M->step_wg > 0) {
        StepArgs a = M->step_args;
        a.head = head ? 1 : 0;
        hipError_t e = launch_step(a, M->step_key, M->step_wg, M->step_lds, M->stream);
        if (e != hipSuccess || !trace) return e;
        e = hipMemcpyAsync(trace, M->arena_h0, sizeof(float) * M->H, hipMemcpyDeviceToDevice, M->stream);
        for (int l = 0; e == hipSuccess && l < M->L; l++)
            e = hipMemcpyAsync(trace + (size_t)(l + 1) * M->H, M->arena_h2[l], sizeof(float) * M->H,
                               hipMemcpyDeviceToDevice, M->stream);
        return e;
    }
    if (trace) return enqueue_step(M, head, splits_for_ctx(ctx), trace);
    return graph_step(M, head, ctx);
}

// A persistent step whose grid barrier gave up (see step.h) sets a flag on the
// device; checked after the stream is synchronized.
hipError_t step_failed(ribn_rocm_model* M, bool* failed) {
    *failed = false;
    if (M->step_wg == 0) return hipSuccess;
    uint32_t flag = 0;
    hipError_t e = hipMemcpy(&flag, M->step_bar + 64, 4, hipMemcpyDeviceToHost);
    *failed = flag != 0;
    return e;
}

// Point the graphs at `slot` and (re)write its device state from the pinned mirror.
hipError_t select_slot(ribn_rocm_model* M, int slot) {
    M->cur_slot = slot;
    return hipMemcpyAsync(M->d_ctl, &M->h_ctl[slot], sizeof(StepCtl), hipMemcpyHostToDevice, M->stream);
}

hipError_t reset_slot(ribn_rocm_model* M, int slot, const std::vector<int32_t>& pages, const uint32_t* toks,
                      uint32_t n_toks) {
    SeqState& s = M->h_state[slot];
    s.pos = 0;
    s.last_token = 0;
    int32_t* hp = M->h_pages + (size_t)slot * M->max_pages;
    for (int i = 0; i < M->max_pages; i++) hp[i] = i < (int)pages.size() ? pages[i] : pages.empty() ? 0 : pages[0];
    uint32_t* ht = M->h_tokens + (size_t)slot * (M->context + 1);
    std::memcpy(ht, toks, sizeof(uint32_t) * n_toks);
    hipError_t e = hipMemcpyAsync(M->d_pages + (size_t)slot * M->max_pages, hp, sizeof(int32_t) * M->max_pages,
                                  hipMemcpyHostToDevice, M->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(M->d_tokens + (size_t)slot * (M->context + 1), ht, sizeof(uint32_t) * n_toks,
                           hipMemcpyHostToDevice, M->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(&M->d_slots[slot], &s, sizeof(SeqState), hipMemcpyHostToDevice, M->stream);
    // a new sequence starts from a zero recurrent state (qwen35 hybrids)
    if (e == hipSuccess && M->hybrid && M->rec_floats)
        e = hipMemsetAsync(M->h_ctl[slot].rec, 0, sizeof(float) * M->rec_floats, M->stream);
    return e;
}

bool take_pages(ribn_rocm_model* M, uint32_t tokens, std::vector<int32_t>* out) {
    const size_t need = (tokens + kPageTokens - 1) / kPageTokens;
    if (M->free_pages.size() < need) return false;
    out->assign(M->free_pages.end() - need, M->free_pages.end());
    M->free_pages.resize(M->free_pages.size() - need);
    return true;
}
void give_pages(ribn_rocm_model* M, std::vector<int32_t>& pages) {
    M->free_pages.insert(M->free_pages.end(), pages.begin(), pages.end());
    pages.clear();
}

// RIBN_LOAD_RESIDENT_F16: binary16 copies of every layer matrix and the head,
// and the hipBLASLt state that multiplies with them.
hipError_t make_resident(ribn_rocm_model* M) {
    hipStream_t st = M->stream;
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd;
    auto copy = [&](uint16_t* dst, const QMat& w) { return launch_dequant_f16(w, dst, st); };
    for (Layer& y : M->layers) {
        hipError_t e;
        if ((e = dalloc(M, &y.w16_qkv, 2ull * (qd + 2 * kd) * M->H)) != hipSuccess) return e;
        if ((e = dalloc(M, &y.w16_o, 2ull * M->H * qd)) != hipSuccess) return e;
        if ((e = dalloc(M, &y.w16_gu, 2ull * 2 * M->F * M->H)) != hipSuccess) return e;
        if ((e = dalloc(M, &y.w16_down, 2ull * M->H * M->F)) != hipSuccess) return e;
        if ((e = copy(y.w16_qkv, y.q)) != hipSuccess) return e;
        if ((e = copy(y.w16_qkv + (size_t)qd * M->H, y.k)) != hipSuccess) return e;
        if ((e = copy(y.w16_qkv + (size_t)(qd + kd) * M->H, y.v)) != hipSuccess) return e;
        if ((e = copy(y.w16_o, y.o)) != hipSuccess) return e;
        if ((e = copy(y.w16_gu, y.gate)) != hipSuccess) return e;
        if ((e = copy(y.w16_gu + (size_t)M->F * M->H, y.up)) != hipSuccess) return e;
        if ((e = copy(y.w16_down, y.down)) != hipSuccess) return e;
        if (y.q_bias) {
            if ((e = dalloc(M, &y.qkv_bias, sizeof(float) * (qd + 2 * kd))) != hipSuccess) return e;
            const float* parts[3] = {y.q_bias, y.k_bias, y.v_bias};
            const int off[3] = {0, qd, qd + kd}, len[3] = {qd, kd, kd};
            for (int i = 0; i < 3; i++) {
                if (parts[i]) e = hipMemcpyAsync(y.qkv_bias + off[i], parts[i], sizeof(float) * len[i], hipMemcpyDeviceToDevice, st);
                else e = hipMemsetAsync(y.qkv_bias + off[i], 0, sizeof(float) * len[i], st);
                if (e != hipSuccess) return e;
            }
        }
    }
    hipError_t e = dalloc(M, &M->w16_head, 2ull * M->V * M->H);
    if (e == hipSuccess) e = copy(M->w16_head, M->out);
    if (e == hipSuccess) e = blas_create(&M->blas, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e;
}

std::string validate_type(const GgufTensor* t, const char* what, bool matrix) {
    if (!t) return std::string("missing tensor ") + what;
    if (matrix) {
        if (t->type != GGML_Q4_K && t->type != GGML_Q6_K && t->type != GGML_Q8_0)
            return "tensor " + t->name + " has unsupported value type " + std::to_string(t->type) + " (" +
                   type_name(t->type) + "); supported: Q4_K, Q6_K, Q8_0";
    } else if (t->type != GGML_F32) {
        return "tensor " + t->name + " has value type " + std::to_string(t->type) + "; expected F32";
    }
    return {};
}

}  // namespace

// ===========================================================================
extern "C" int ribn_rocm_load_gguf(const char* path, const ribn_rocm_load_options* opts, ribn_rocm_model** out,
                                   char* err, size_t err_len) {
    if (!path || !out) { set_err(err, err_len, "null argument"); return RIBN_ERR_INVALID; }
    *out = nullptr;
    GgufFile g;
    std::string msg = g.open(path);
    if (!msg.empty()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }
    std::string arch;
    if (!g.get_str("general.architecture", &arch)) { set_err(err, err_len, "missing general.architecture"); return RIBN_ERR_FORMAT; }
    if (arch != "qwen2" && arch != "qwen3" && arch != "qwen35") {
        set_err(err, err_len, "general.architecture `" + arch + "` is not supported (expected qwen2, qwen3 or qwen35)");
        return RIBN_ERR_FORMAT;
    }
    std::unique_ptr<ribn_rocm_model, void (*)(ribn_rocm_model*)> Mp(new ribn_rocm_model(), ribn_rocm_free);
    ribn_rocm_model* M = Mp.get();
    M->qwen3 = arch != "qwen2";
    M->hybrid = arch == "qwen35";
    auto need_u = [&](const char* suffix, int* dst) -> bool {
        uint64_t v;
        if (!g.get_u64(arch + "." + suffix, &v) || v == 0 || v > (1u << 30)) {
            set_err(err, err_len, "missing or invalid " + arch + "." + suffix);
            return false;
        }
        *dst = (int)v;
        return true;
    };
    if (!need_u("embedding_length", &M->H) || !need_u("block_count", &M->L) || !need_u("attention.head_count", &M->hq) ||
        !need_u("attention.head_count_kv", &M->hkv) || !need_u("feed_forward_length", &M->F))
        return RIBN_ERR_FORMAT;
    uint64_t v;
    M->hd = g.get_u64(arch + ".attention.key_length", &v) ? (int)v : M->H / M->hq;
    M->rot = g.get_u64(arch + ".rope.dimension_count", &v) ? (int)v : M->hd;
    if (!g.get_f32(arch + ".attention.layer_norm_rms_epsilon", &M->eps)) M->eps = 1e-6f;
    if (!g.get_f32(arch + ".rope.freq_base", &M->base)) M->base = 10000.f;
    uint64_t vlen;
    if (g.get_u64(arch + ".attention.value_length", &vlen) && (int)vlen != M->hd) {
        set_err(err, err_len, arch + ".attention.value_length must equal key_length"); return RIBN_ERR_FORMAT;
    }
    // head_dim 256 (the qwen35 27B's attention) runs the decode attention kernel only: hybrids have no
    // chunked-prefill or batched-row attention
    if ((M->hd != 64 && M->hd != 128 && !(M->hybrid && M->hd == 256)) || M->rot > M->hd || M->rot % 2) {
        set_err(err, err_len, arch + ".attention.key_length " + std::to_string(M->hd) +
                                  " is not supported (64 or 128; 256 for qwen35)");
        return RIBN_ERR_FORMAT;
    }
    if (M->hq % M->hkv || M->hq / M->hkv > 8) {
        set_err(err, err_len, arch + ".attention.head_count / head_count_kv must be an integer <= 8");
        return RIBN_ERR_FORMAT;
    }
    if (M->hybrid) {
        // crates/qwen/src/gguf/config.rs:17-37 (keys) and :93-128 (periodic layer schedule)
        if (!need_u("ssm.group_count", &M->ssm_hk) || !need_u("ssm.time_step_rank", &M->ssm_hv) ||
            !need_u("ssm.state_size", &M->ssm_d) || !need_u("ssm.inner_size", &M->inner) ||
            !need_u("ssm.conv_kernel", &M->conv_k))
            return RIBN_ERR_FORMAT;
        uint64_t nextn = 0;
        if (g.get_u64("qwen35.nextn_predict_layers", &nextn) && nextn != 0) {
            set_err(err, err_len, "qwen35.nextn_predict_layers: multi-token-prediction layers are not supported");
            return RIBN_ERR_FORMAT;
        }
        if (g.get("qwen35.attention.recurrent_layers")) {
            set_err(err, err_len, "qwen35.attention.recurrent_layers: only the periodic full_attention_interval "
                                  "schedule is supported");
            return RIBN_ERR_FORMAT;
        }
        uint64_t iv = 4;
        g.get_u64("qwen35.full_attention_interval", &iv);
        M->interval = (int)iv;
        if (M->interval < 1 || M->interval > M->L) {
            set_err(err, err_len, "qwen35.full_attention_interval must be in [1, block_count]"); return RIBN_ERR_FORMAT;
        }
        if ((M->ssm_d != 64 && M->ssm_d != 128) || M->ssm_hv % M->ssm_hk || M->inner != M->ssm_hv * M->ssm_d ||
            M->conv_k < 2 || M->conv_k > 8) {
            set_err(err, err_len, "qwen35.ssm: state_size must be 64 or 128, time_step_rank a multiple of group_count, "
                                  "inner_size = time_step_rank * state_size, conv_kernel in [2, 8]");
            return RIBN_ERR_FORMAT;
        }
        M->channels = 2 * M->ssm_hk * M->ssm_d + M->inner;
        if (opts && (opts->flags & (RIBN_LOAD_RESIDENT_F16 | RIBN_LOAD_PERSISTENT_STEP | RIBN_LOAD_INT_DOT))) {
            set_err(err, err_len, "qwen35 hybrids run the default launch chain (no resident, persistent or "
                                  "integer-dot mode)");
            return RIBN_ERR_INVALID;
        }
    }
    if (M->H % 32 || M->F % 32 || M->H > 16384 || M->F > 28672) {
        set_err(err, err_len, arch + ".embedding_length and feed_forward_length must be multiples of 32 "
                                     "(<= 16384 / 28672)");
        return RIBN_ERR_FORMAT;
    }
    const GgufTensor* te = g.tensor("token_embd.weight");
    if ((msg = validate_type(te, "token_embd.weight", true)).size()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }
    if (te->dims.size() != 2 || (int)te->dims[0] != M->H) {
        set_err(err, err_len, "token_embd.weight must be [embedding_length, vocab]"); return RIBN_ERR_FORMAT;
    }
    M->V = (int)te->dims[1];
    const GgufTensor* to = g.tensor("output.weight");
    if (!to) to = te;   // tied head
    if ((msg = validate_type(to, "output.weight", true)).size()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }
    const GgufTensor* ton = g.tensor("output_norm.weight");
    if ((msg = validate_type(ton, "output_norm.weight", false)).size()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }

    uint64_t ctx_meta = 0;
    g.get_u64(arch + ".context_length", &ctx_meta);
    ribn_rocm_load_options o{};
    if (opts) o = *opts;
    M->context = o.context_tokens ? o.context_tokens : (uint32_t)std::min<uint64_t>(ctx_meta ? ctx_meta : 4096, 4096);
    M->max_seqs = o.max_sequences ? o.max_sequences : 8;
    M->max_batch_tokens = o.max_batch_tokens ? o.max_batch_tokens : 2048;
    if (M->context > (uint32_t)(kMaxSplits * kMaxSplitTokens)) {
        set_err(err, err_len, "context_tokens above " + std::to_string(kMaxSplits * kMaxSplitTokens));
        return RIBN_ERR_INVALID;
    }
    M->max_pages = (int)((M->context + kPageTokens - 1) / kPageTokens);
    M->kv_pages = o.kv_pages ? o.kv_pages : (uint32_t)(M->max_seqs * M->max_pages);
    if ((int)M->kv_pages < M->max_pages) M->kv_pages = M->max_pages;
    M->device = o.device;
    M->kv_f16 = (o.flags & RIBN_LOAD_KV_BF16) == 0;
    M->int_dot = (o.flags & RIBN_LOAD_INT_DOT) != 0;
    if (M->int_dot && (o.flags & RIBN_LOAD_PERSISTENT_STEP)) {
        set_err(err, err_len, "the integer-dot mode runs decode rows, not the persistent step");
        return RIBN_ERR_INVALID;
    }
    M->name = "ribn-rocm " + arch + " " + std::to_string(M->L) + "x" + std::to_string(M->H);

    HIPCHK(hipSetDevice(M->device));
    HIPCHK(hipStreamCreateWithFlags(&M->stream, hipStreamNonBlocking));
    std::vector<uint8_t> staging;
    const int qd = M->hq * M->hd, kd = M->hkv * M->hd;
    // matrices the GEMMs read also get the GEMM-ordered copy (not the embedding table)
    const bool gemm_copy = !(o.flags & RIBN_LOAD_GEMM_FROM_PLANES);
    M->merge_in_launch = (o.flags & RIBN_LOAD_ATTN_MERGE_IN_LAUNCH) != 0;
    auto upload_mat = [&](const GgufTensor* t, uint64_t rows, uint64_t k, QMat* q) -> int {
        if (t->dims.size() != 2 || t->dims[0] != k || t->dims[1] != rows) {
            return fail(nullptr, err, err_len,
                        "tensor " + t->name + " has shape [" + std::to_string(t->dims[0]) + ", " +
                            std::to_string(t->dims.size() > 1 ? t->dims[1] : 0) + "], expected [" + std::to_string(k) +
                            ", " + std::to_string(rows) + "]",
                        RIBN_ERR_FORMAT);
        }
        uint64_t be, bb;
        type_layout(t->type, &be, &bb);
        if (k % be)
            return fail(nullptr, err, err_len,
                        "tensor " + t->name + ": input length " + std::to_string(k) + " is not a multiple of the " +
                            type_name(t->type) + " block (" + std::to_string(be) + ")",
                        RIBN_ERR_FORMAT);
        HIPCHK(upload_qmat(M, t->type, rows, k, g.data(*t), q, staging, gemm_copy && q != &M->embd));
        return RIBN_OK;
    };
    auto upload_f32 = [&](const GgufTensor* t, uint64_t n, float** dst) -> int {
        if (t->type != GGML_F32 || t->dims.empty() || t->dims[0] != n)
            return fail(nullptr, err, err_len, "tensor " + t->name + " must be F32 [" + std::to_string(n) + "]", RIBN_ERR_FORMAT);
        HIPCHK(dalloc(M, dst, n * 4));
        HIPCHK(hipMemcpy(*dst, g.data(*t), n * 4, hipMemcpyHostToDevice));
        return RIBN_OK;
    };
    int rc;
    if ((rc = upload_mat(te, M->V, M->H, &M->embd)) != RIBN_OK) return rc;
    if (to == te) M->out = M->embd;
    else if ((rc = upload_mat(to, M->V, M->H, &M->out)) != RIBN_OK) return rc;
    if ((rc = upload_f32(ton, M->H, &M->out_norm)) != RIBN_OK) return rc;
    M->layers.resize(M->L);
    size_t rec_off = 0;
    for (int l = 0; l < M->L; l++) {
        Layer& y = M->layers[l];
        auto T = [&](const char* nm) { return g.tensor("blk." + std::to_string(l) + "." + nm); };
        auto lname = [&](const char* nm) { return "blk." + std::to_string(l) + "." + nm; };
        auto mat = [&](const char* nm, uint64_t rows, uint64_t k, QMat* q) -> int {
            const GgufTensor* t = T(nm);
            const std::string full = lname(nm);
            if ((msg = validate_type(t, full.c_str(), true)).size()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }
            return upload_mat(t, rows, k, q);
        };
        auto vec = [&](const char* nm, uint64_t n, float** dst) -> int {
            const GgufTensor* t = T(nm);
            if (!t) { set_err(err, err_len, "missing tensor " + lname(nm)); return RIBN_ERR_FORMAT; }
            return upload_f32(t, n, dst);
        };
        if (!M->hybrid) {
        struct { const char* n; uint64_t rows, k; QMat* q; } mats[] = {
            {"attn_q.weight", (uint64_t)qd, (uint64_t)M->H, &y.q},     {"attn_k.weight", (uint64_t)kd, (uint64_t)M->H, &y.k},
            {"attn_v.weight", (uint64_t)kd, (uint64_t)M->H, &y.v},     {"attn_output.weight", (uint64_t)M->H, (uint64_t)qd, &y.o},
            {"ffn_gate.weight", (uint64_t)M->F, (uint64_t)M->H, &y.gate}, {"ffn_up.weight", (uint64_t)M->F, (uint64_t)M->H, &y.up},
            {"ffn_down.weight", (uint64_t)M->H, (uint64_t)M->F, &y.down},
        };
        for (auto& m : mats) {
            const GgufTensor* t = T(m.n);
            std::string nm = "blk." + std::to_string(l) + "." + m.n;
            if ((msg = validate_type(t, nm.c_str(), true)).size()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }
            if ((rc = upload_mat(t, m.rows, m.k, m.q)) != RIBN_OK) return rc;
        }
        if (y.q.type != y.k.type) {
            set_err(err, err_len, "attn_q and attn_k must share a value type"); return RIBN_ERR_FORMAT;
        }
        if (y.gate.type != y.up.type) {
            set_err(err, err_len, "ffn_gate and ffn_up must share a value type"); return RIBN_ERR_FORMAT;
        }
        struct { const char* n; uint64_t len; float** dst; bool req; } vecs[] = {
            {"attn_norm.weight", (uint64_t)M->H, &y.attn_norm, true}, {"ffn_norm.weight", (uint64_t)M->H, &y.ffn_norm, true},
            {"attn_q_norm.weight", (uint64_t)M->hd, &y.q_norm, false}, {"attn_k_norm.weight", (uint64_t)M->hd, &y.k_norm, false},
            {"attn_q.bias", (uint64_t)qd, &y.q_bias, false},          {"attn_k.bias", (uint64_t)kd, &y.k_bias, false},
            {"attn_v.bias", (uint64_t)kd, &y.v_bias, false},
        };
        for (auto& vv : vecs) {
            const GgufTensor* t = T(vv.n);
            if (!t) {
                if (vv.req) { set_err(err, err_len, "missing tensor blk." + std::to_string(l) + "." + vv.n); return RIBN_ERR_FORMAT; }
                continue;
            }
            if ((rc = upload_f32(t, vv.len, vv.dst)) != RIBN_OK) return rc;
        }
        } else {
            // qwen35 (decode.rs:52-82 tensor sets; config.rs:93-128 schedule)
            y.recurrent = (l + 1) % M->interval != 0;
            if ((rc = mat("ffn_gate.weight", M->F, M->H, &y.gate)) || (rc = mat("ffn_up.weight", M->F, M->H, &y.up)) ||
                (rc = mat("ffn_down.weight", M->H, M->F, &y.down)) || (rc = vec("attn_norm.weight", M->H, &y.attn_norm)) ||
                (rc = vec("post_attention_norm.weight", M->H, &y.ffn_norm)))
                return rc;
            if (y.gate.type != y.up.type) { set_err(err, err_len, "ffn_gate and ffn_up must share a value type"); return RIBN_ERR_FORMAT; }
            if (y.recurrent) {
                if ((rc = mat("attn_qkv.weight", M->channels, M->H, &y.gdn_mix)) ||
                    (rc = mat("attn_gate.weight", M->inner, M->H, &y.gdn_z)) ||
                    (rc = mat("ssm_out.weight", M->H, M->inner, &y.o)) || (rc = vec("ssm_dt.bias", M->ssm_hv, &y.dt_bias)) ||
                    (rc = vec("ssm_a", M->ssm_hv, &y.ssm_a)) || (rc = vec("ssm_norm.weight", M->ssm_d, &y.ssm_norm)))
                    return rc;
                if (y.gdn_mix.type != y.gdn_z.type) {
                    set_err(err, err_len, lname("attn_qkv.weight") + " and attn_gate.weight must share a value type");
                    return RIBN_ERR_FORMAT;
                }
                // beta and alpha share one matrix of 2 * time_step_rank rows (beta first)
                const GgufTensor* tb = T("ssm_beta.weight");
                const GgufTensor* ta = T("ssm_alpha.weight");
                const std::string nb = lname("ssm_beta.weight"), na = lname("ssm_alpha.weight");
                if ((msg = validate_type(tb, nb.c_str(), true)).size() || (msg = validate_type(ta, na.c_str(), true)).size()) {
                    set_err(err, err_len, msg); return RIBN_ERR_FORMAT;
                }
                if (tb->type != ta->type || tb->dims.size() != 2 || ta->dims.size() != 2 || tb->dims[0] != (uint64_t)M->H ||
                    ta->dims[0] != (uint64_t)M->H || tb->dims[1] != (uint64_t)M->ssm_hv || ta->dims[1] != (uint64_t)M->ssm_hv) {
                    set_err(err, err_len, nb + " and ssm_alpha.weight must be [embedding_length, time_step_rank] of one type");
                    return RIBN_ERR_FORMAT;
                }
                {
                    std::vector<uint8_t> cat(tb->bytes + ta->bytes);
                    std::memcpy(cat.data(), g.data(*tb), tb->bytes);
                    std::memcpy(cat.data() + tb->bytes, g.data(*ta), ta->bytes);
                    HIPCHK(upload_qmat(M, tb->type, 2ull * M->ssm_hv, M->H, cat.data(), &y.gdn_ba, staging));
                }
                const GgufTensor* tc = T("ssm_conv1d.weight");
                if (!tc || tc->type != GGML_F32 || tc->dims.size() != 2 || tc->dims[0] != (uint64_t)M->conv_k ||
                    tc->dims[1] != (uint64_t)M->channels) {
                    set_err(err, err_len, lname("ssm_conv1d.weight") + " must be F32 [conv_kernel, channels]");
                    return RIBN_ERR_FORMAT;
                }
                HIPCHK(dalloc(M, &y.conv_w, tc->bytes));
                HIPCHK(hipMemcpy(y.conv_w, g.data(*tc), tc->bytes, hipMemcpyHostToDevice));
                y.state_off = rec_off;
                rec_off += (size_t)M->ssm_hv * M->ssm_d * M->ssm_d;
                y.conv_off = rec_off;
                rec_off += (size_t)M->channels * (M->conv_k - 1);
            } else {
                // attn_q holds [q | gate] per head (2 head_dim rows each, qwen_reference.rs:379-385): split
                // into a q matrix and a gate matrix so q|k|v feed the attention kernel as in dense layers
                const GgufTensor* tq = T("attn_q.weight");
                const std::string nq = lname("attn_q.weight");
                if ((msg = validate_type(tq, nq.c_str(), true)).size()) { set_err(err, err_len, msg); return RIBN_ERR_FORMAT; }
                if (tq->dims.size() != 2 || tq->dims[0] != (uint64_t)M->H || tq->dims[1] != 2ull * qd) {
                    set_err(err, err_len, nq + " must be [embedding_length, 2 * head_count * key_length]");
                    return RIBN_ERR_FORMAT;
                }
                uint64_t be, bb;
                type_layout(tq->type, &be, &bb);
                const size_t rb = (size_t)(M->H / be * bb), hb = rb * M->hd;
                std::vector<uint8_t> qh((size_t)qd * rb), gh((size_t)qd * rb);
                const uint8_t* src = g.data(*tq);
                for (int h = 0; h < M->hq; h++) {
                    std::memcpy(qh.data() + h * hb, src + (2 * h) * hb, hb);
                    std::memcpy(gh.data() + h * hb, src + (2 * h + 1) * hb, hb);
                }
                HIPCHK(upload_qmat(M, tq->type, qd, M->H, qh.data(), &y.q, staging));
                HIPCHK(upload_qmat(M, tq->type, qd, M->H, gh.data(), &y.q_gate, staging));
                if ((rc = mat("attn_k.weight", kd, M->H, &y.k)) || (rc = mat("attn_v.weight", kd, M->H, &y.v)) ||
                    (rc = mat("attn_output.weight", M->H, qd, &y.o)) || (rc = vec("attn_q_norm.weight", M->hd, &y.q_norm)) ||
                    (rc = vec("attn_k_norm.weight", M->hd, &y.k_norm)))
                    return rc;
                if (y.q.type != y.k.type) { set_err(err, err_len, "attn_q and attn_k must share a value type"); return RIBN_ERR_FORMAT; }
            }
        }
        if (y.recurrent) continue;
        const size_t kv_layer = (size_t)M->kv_pages * M->hkv * kPageTokens * M->hd;
        HIPCHK(dalloc(M, &y.kc, kv_layer * 2));
        HIPCHK(dalloc(M, &y.vc, kv_layer * 2));
        HIPCHK(hipMemsetAsync(y.kc, 0, kv_layer * 2, M->stream));
        HIPCHK(hipMemsetAsync(y.vc, 0, kv_layer * 2, M->stream));
        M->kv_bytes += kv_layer * 4;
    }
    staging.clear();
    staging.shrink_to_fit();
    M->rec_floats = rec_off;
    if (M->hybrid) {
        HIPCHK(dalloc(M, &M->mixed, sizeof(float) * M->channels));
        HIPCHK(dalloc(M, &M->gdn_act, sizeof(float) * M->channels));
        HIPCHK(dalloc(M, &M->zbuf, sizeof(float) * M->inner));
        HIPCHK(dalloc(M, &M->gated, sizeof(float) * M->inner));
        HIPCHK(dalloc(M, &M->ba, sizeof(float) * 2 * M->ssm_hv));
        HIPCHK(dalloc(M, &M->att_gate, sizeof(float) * qd));
        const size_t slots_rec = (size_t)M->max_seqs + 1;
        HIPCHK(dalloc(M, &M->d_rec, sizeof(float) * std::max<size_t>(1, slots_rec * M->rec_floats)));
        HIPCHK(hipMemsetAsync(M->d_rec, 0, sizeof(float) * std::max<size_t>(1, slots_rec * M->rec_floats), M->stream));
    }

    HIPCHK(dalloc(M, &M->h, sizeof(float) * M->H));
    HIPCHK(dalloc(M, &M->raw, sizeof(float) * (qd + 2 * kd)));
    HIPCHK(dalloc(M, &M->qbuf, sizeof(float) * qd));
    HIPCHK(dalloc(M, &M->attn, sizeof(float) * qd));
    HIPCHK(dalloc(M, &M->act, sizeof(float) * M->F));
    HIPCHK(dalloc(M, &M->logits, sizeof(float) * M->V));
    HIPCHK(dalloc(M, &M->part, sizeof(float) * (size_t)kMaxSplits * (qd + 2 * M->hq)));
    const int n_counters = M->hkv + 1;
    {
        std::vector<float> inv(M->rot / 2);
        for (int p = 0; p < M->rot / 2; p++) inv[p] = std::pow(M->base, -(2.0f * (float)p) / (float)M->rot);
        HIPCHK(dalloc(M, &M->inv_freq, sizeof(float) * inv.size()));
        HIPCHK(dalloc(M, &M->rope, sizeof(float) * M->rot));
        HIPCHK(hipMemcpy(M->inv_freq, inv.data(), sizeof(float) * inv.size(), hipMemcpyHostToDevice));
    }
    HIPCHK(dalloc(M, &M->counters, sizeof(uint32_t) * n_counters));
    HIPCHK(hipMemsetAsync(M->counters, 0, sizeof(uint32_t) * n_counters, M->stream));
    HIPCHK(dalloc(M, &M->head_partial, sizeof(uint64_t) * std::max<size_t>((size_t)M->V / 2 + 64, 8192)));
    {
        M->chunk = (int)std::min<uint32_t>(M->max_batch_tokens, 2048);
        const size_t c = (size_t)M->chunk;
        const size_t kmax = (size_t)std::max(std::max(M->H, M->F), qd);
        HIPCHK(dalloc(M, &M->p_h, sizeof(float) * c * M->H));
        HIPCHK(dalloc(M, &M->p_qkv, sizeof(float) * c * (qd + 2 * kd)));
        HIPCHK(dalloc(M, &M->p_q, sizeof(float) * c * qd));
        HIPCHK(dalloc(M, &M->p_gu, sizeof(float) * c * 2 * M->F));
        HIPCHK(dalloc(M, &M->p_x16, 2 * c * kmax));
        HIPCHK(dalloc(M, &M->p_att16, 2 * c * qd));
        HIPCHK(dalloc(M, &M->p_act16, 2 * c * M->F));
        // split-K partials: the largest split x ldy over the chunk's GEMMs
        const int ldq = qd + 2 * kd;
        auto need = [&](int k, int ldy, int tiles) { return (size_t)prefill_gemm_splits(M->chunk, k, tiles) * ldy; };
        const int t_qkv = gemm_tiles(qd) + 2 * gemm_tiles(kd), t_h = gemm_tiles(M->H), t_gu = 2 * gemm_tiles(M->F);
        size_t per_row = std::max(std::max(need(M->H, ldq, t_qkv), need(qd, M->H, t_h)),
                                  std::max(need(M->H, 2 * M->F, t_gu), need(M->F, M->H, t_h)));
        M->p_part_floats = per_row * c;
        HIPCHK(dalloc(M, &M->p_part, sizeof(float) * M->p_part_floats));
        // batched decode rows: one per sequence, at most the chunk's rows
        // (hybrids decode one sequence per step: the recurrent blocks have no batched form here)
        M->b_rows = M->hybrid ? 0 : (int)std::min<size_t>(c, M->max_seqs);
        // the integer-dot mode runs every sampled decode row here, also one at a time
        if (M->int_dot) M->b_rows = std::max(M->b_rows, 1);
        if (M->b_rows >= 2 || M->int_dot) {
            const size_t R = (size_t)M->b_rows;
            M->b_part_stride = (size_t)M->hkv * kMaxSplits * ((size_t)(M->hq / M->hkv) * M->hd + 2 * (M->hq / M->hkv));
            HIPCHK(dalloc(M, &M->d_brows, sizeof(int32_t) * 2 * R));
            HIPCHK(dalloc(M, &M->d_btokens, sizeof(uint32_t) * R));
            HIPCHK(dalloc(M, &M->b_att, sizeof(float) * R * qd));
            HIPCHK(dalloc(M, &M->b_rope, sizeof(float) * R * M->rot));
            HIPCHK(dalloc(M, &M->b_part, sizeof(float) * R * M->b_part_stride));
            HIPCHK(dalloc(M, &M->b_logits, sizeof(float) * R * M->V));
            HIPCHK(dalloc(M, &M->b_argmax, sizeof(uint64_t) * R * 64));
            HIPCHK(dalloc(M, &M->b_counters, sizeof(uint32_t) * R * M->hkv));
            HIPCHK(hipMemsetAsync(M->b_counters, 0, sizeof(uint32_t) * R * M->hkv, M->stream));
            M->h_brows.assign(2 * R, 0);
            HIPCHK(dalloc(M, &M->b_act, sizeof(float) * R * M->F));
            if (M->int_dot) HIPCHK(dalloc(M, &M->b_xq, sizeof(uint32_t) * R * (kmax / 32) * 9));
        }
    }

    const int slots = (int)M->max_seqs + 1;
    HIPCHK(dalloc(M, &M->d_slots, sizeof(SeqState) * slots));
    HIPCHK(dalloc(M, &M->d_pages, sizeof(int32_t) * (size_t)slots * M->max_pages));
    HIPCHK(dalloc(M, &M->d_tokens, sizeof(uint32_t) * (size_t)slots * (M->context + 1)));
    HIPCHK(dalloc(M, &M->d_ctl, sizeof(StepCtl)));
    HIPCHK(hipMemsetAsync(M->d_pages, 0, sizeof(int32_t) * (size_t)slots * M->max_pages, M->stream));
    HIPCHK(hipMemsetAsync(M->d_tokens, 0, sizeof(uint32_t) * (size_t)slots * (M->context + 1), M->stream));
    HIPCHK(halloc(M, &M->h_ctl, sizeof(StepCtl) * slots));
    HIPCHK(halloc(M, &M->h_state, sizeof(SeqState) * slots));
    HIPCHK(halloc(M, &M->h_pages, sizeof(int32_t) * (size_t)slots * M->max_pages));
    HIPCHK(halloc(M, &M->h_tokens, sizeof(uint32_t) * (size_t)slots * (M->context + 1)));
    HIPCHK(halloc(M, &M->h_out, sizeof(uint32_t) * (M->max_seqs + 8)));
    for (int s = 0; s < slots; s++) {
        M->h_ctl[s].seq = &M->d_slots[s];
        M->h_ctl[s].pos = 0;
        M->h_ctl[s].pages = M->d_pages + (size_t)s * M->max_pages;
        M->h_ctl[s].rec = M->hybrid ? M->d_rec + (size_t)s * M->rec_floats : nullptr;
        SeqState& st = M->h_state[s];
        st.pos = 0;
        st.last_token = 0;
        st.max_pages = M->max_pages;
        st.max_ctx = (int)M->context;
        st.pages = M->d_pages + (size_t)s * M->max_pages;
        st.tokens = M->d_tokens + (size_t)s * (M->context + 1);
    }
    HIPCHK(hipMemcpyAsync(M->d_slots, M->h_state, sizeof(SeqState) * slots, hipMemcpyHostToDevice, M->stream));
    HIPCHK(hipMemcpyAsync(M->d_ctl, &M->h_ctl[slots - 1], sizeof(StepCtl), hipMemcpyHostToDevice, M->stream));
    M->cur_slot = slots - 1;
    HIPCHK(hipStreamSynchronize(M->stream));
    for (int s = (int)M->max_seqs - 1; s >= 0; s--) M->free_slots.push_back(s);
    for (int p = (int)M->kv_pages - 1; p >= 0; p--) M->free_pages.push_back(p);
    build_launches(M);
    HIPCHK(build_step(M, (o.flags & RIBN_LOAD_PERSISTENT_STEP) != 0));
    if (o.flags & RIBN_LOAD_RESIDENT_F16) HIPCHK(make_resident(M));
    *out = Mp.release();
    return RIBN_OK;
}

extern "C" void ribn_rocm_free(ribn_rocm_model* M) {
    if (!M) return;
    if (M->stream) hipStreamSynchronize(M->stream);
    for (auto& kv : M->graphs) hipGraphExecDestroy(kv.second);
    for (auto& kv : M->row_graphs) hipGraphExecDestroy(kv.second);
    if (M->pending.done) hipEventDestroy(M->pending.done);
    blas_destroy(M->blas);
    for (void* p : M->dev_allocs) hipFree(p);
    for (void* p : M->host_allocs) hipHostFree(p);
    if (M->stream) hipStreamDestroy(M->stream);
    delete M;
}

extern "C" int ribn_rocm_info(const ribn_rocm_model* M, ribn_rocm_info_t* o) {
    if (!M || !o) return RIBN_ERR_INVALID;
    std::memset(o, 0, sizeof(*o));
    std::snprintf(o->name, sizeof(o->name), "%s", M->name.c_str());
    o->context_tokens = M->context;
    o->max_sequences = M->max_seqs;
    o->max_batch_tokens = M->max_batch_tokens;
    o->max_decode_tokens = 1;
    o->hidden = M->H; o->layers = M->L; o->q_heads = M->hq; o->kv_heads = M->hkv;
    o->head_dim = M->hd; o->ffn = M->F; o->vocab = M->V; o->rope_dims = M->rot;
    o->weight_bytes = M->weight_bytes;
    o->kv_bytes = M->kv_bytes;
    o->kv_f16 = M->kv_f16 ? 1 : 0;
    o->persistent_step = M->step_wg > 0 ? 1 : 0;
    o->step_workgroups = (uint32_t)M->step_wg;
    return RIBN_OK;
}

// ---------------------------------------------------------------------------
extern "C" int ribn_rocm_generate(ribn_rocm_model* M, const uint32_t* prompt, uint32_t n_prompt, uint32_t n_new,
                                  uint32_t* out_tokens, ribn_rocm_timing* timing, char* err, size_t err_len) {
    if (!M || !prompt || !out_tokens) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->faulted) return fail(nullptr, err, err_len, "ROCm execution is faulted", RIBN_ERR_FAULTED);
    if (M->has_pending) return fail(nullptr, err, err_len, "a submission is in flight", RIBN_ERR_BUSY);
    if (n_prompt == 0 || n_new == 0 || (uint64_t)n_prompt + n_new > M->context)
        return fail(nullptr, err, err_len, "prompt/output length outside the prepared context", RIBN_ERR_INVALID);
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= (uint32_t)M->V) return fail(nullptr, err, err_len, "token id out of range", RIBN_ERR_INVALID);
    std::vector<int32_t> pages;
    if (!take_pages(M, n_prompt + n_new, &pages))
        return fail(nullptr, err, err_len, "not enough free KV pages", RIBN_ERR_CAPACITY);
    const int slot = (int)M->max_seqs;
    hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr;
    auto cleanup = [&]() {
        if (e0) hipEventDestroy(e0);
        if (e1) hipEventDestroy(e1);
        if (e2) hipEventDestroy(e2);
        give_pages(M, pages);
    };
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventCreate(&e2);
    if (e == hipSuccess) e = reset_slot(M, slot, pages, prompt, n_prompt);
    if (e == hipSuccess) e = select_slot(M, slot);
    if (e == hipSuccess) e = hipEventRecord(e0, M->stream);
    if (e == hipSuccess) e = prefill_rows(M, slot, 0, (int)n_prompt, true);
    if (e == hipSuccess) e = hipEventRecord(e1, M->stream);
    for (uint32_t t = 1; e == hipSuccess && t < n_new; t++) e = run_step(M, true, (int)(n_prompt + t), nullptr);
    if (e == hipSuccess) e = hipEventRecord(e2, M->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(out_tokens, M->d_tokens + (size_t)slot * (M->context + 1) + n_prompt, sizeof(uint32_t) * n_new,
                           hipMemcpyDeviceToHost, M->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(M->stream);
    if (e == hipSuccess && timing) {
        float a = 0.f, b = 0.f;
        hipEventElapsedTime(&a, e0, e1);
        hipEventElapsedTime(&b, e1, e2);
        timing->prefill_ms = a;
        timing->decode_ms = b;
        timing->prefill_tokens = n_prompt;
        timing->decode_tokens = n_new - 1;
    }
    bool barrier_failed = false;
    if (e == hipSuccess) e = step_failed(M, &barrier_failed);
    cleanup();
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("generate", e));
    if (barrier_failed) return fail(M, err, err_len, "decode step: a grid barrier wait exceeded its limit");
    return RIBN_OK;
}

extern "C" int ribn_rocm_trace(ribn_rocm_model* M, const uint32_t* tokens, uint32_t n, uint32_t* argmax_out,
                               float* logits_out, float* hidden_out, char* err, size_t err_len) {
    if (!M || !tokens || !argmax_out) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->faulted) return fail(nullptr, err, err_len, "ROCm execution is faulted", RIBN_ERR_FAULTED);
    if (M->has_pending) return fail(nullptr, err, err_len, "a submission is in flight", RIBN_ERR_BUSY);
    if (M->int_dot)
        return fail(nullptr, err, err_len, "traces run the float projections: not in the integer-dot mode", RIBN_ERR_INVALID);
    if (n == 0 || n + 1 > M->context) return fail(nullptr, err, err_len, "trace length outside the context", RIBN_ERR_INVALID);
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)M->V) return fail(nullptr, err, err_len, "token id out of range", RIBN_ERR_INVALID);
    std::vector<int32_t> pages;
    if (!take_pages(M, n + 1, &pages)) return fail(nullptr, err, err_len, "not enough free KV pages", RIBN_ERR_CAPACITY);
    const int slot = (int)M->max_seqs;
    float* dtrace = nullptr;
    hipError_t e = hipSuccess;
    if (hidden_out) e = hipMalloc(&dtrace, sizeof(float) * (size_t)(M->L + 1) * M->H);
    if (e == hipSuccess) e = reset_slot(M, slot, pages, tokens, n);
    if (e == hipSuccess) e = select_slot(M, slot);
    uint32_t* dtok = M->d_tokens + (size_t)slot * (M->context + 1);
    for (uint32_t p = 0; e == hipSuccess && p < n; p++) {
        e = run_step(M, true, (int)p + 1, dtrace);
        if (e == hipSuccess)
            e = hipMemcpyAsync(&M->h_out[0], &M->d_slots[slot].last_token, 4, hipMemcpyDeviceToHost, M->stream);
        if (e == hipSuccess && logits_out)
            e = hipMemcpyAsync(logits_out + (size_t)p * M->V, M->logits, sizeof(float) * M->V, hipMemcpyDeviceToHost, M->stream);
        if (e == hipSuccess && hidden_out)
            e = hipMemcpyAsync(hidden_out + (size_t)p * (M->L + 1) * M->H, dtrace, sizeof(float) * (M->L + 1) * M->H,
                               hipMemcpyDeviceToHost, M->stream);
        // teacher forcing: restore the given next token over the sampled one
        if (e == hipSuccess && p + 1 < n)
            e = hipMemcpyAsync(dtok + p + 1, M->h_tokens + (size_t)slot * (M->context + 1) + p + 1, 4,
                               hipMemcpyHostToDevice, M->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(M->stream);
        if (e == hipSuccess) argmax_out[p] = M->h_out[0];
    }
    if (dtrace) hipFree(dtrace);
    give_pages(M, pages);
    bool barrier_failed = false;
    if (e == hipSuccess) e = step_failed(M, &barrier_failed);
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("trace", e));
    if (barrier_failed) return fail(M, err, err_len, "decode step: a grid barrier wait exceeded its limit");
    return RIBN_OK;
}

// ---------------------------------------------------------------------------
// GenerationExecutor (executor.rs:171-254) with the Qwen adapter's rules
// (crates/qwen/src/execution.rs:80-414).
extern "C" int ribn_rocm_admit(ribn_rocm_model* M, uint64_t request_id, uint64_t sequence, const uint32_t* tokens,
                               uint32_t n_tokens, const ribn_rocm_token_options* opt, int32_t* admission, char* err,
                               size_t err_len) {
    (void)request_id;
    if (!M || !admission || !opt) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->faulted) return fail(nullptr, err, err_len, "ROCm execution is faulted", RIBN_ERR_FAULTED);
    if (M->seqs.count(sequence)) return fail(nullptr, err, err_len, "duplicate sequence", RIBN_ERR_INVALID);
    const uint64_t total = (uint64_t)n_tokens + opt->max_output_tokens;
    bool bad = n_tokens == 0 || !tokens || opt->max_output_tokens == 0 || total > M->context;
    for (uint32_t i = 0; !bad && i < n_tokens; i++) bad = tokens[i] >= (uint32_t)M->V;
    for (uint32_t i = 0; !bad && i < opt->n_stop_tokens; i++) bad = opt->stop_tokens[i] >= (uint32_t)M->V;
    if (bad) {
        *admission = RIBN_ADMIT_REJECTED;
        set_err(err, err_len, "Qwen input/output limits or token IDs are invalid");
        return RIBN_OK;
    }
    if (opt->temperature != 0.0f) {
        *admission = RIBN_ADMIT_REJECTED;
        set_err(err, err_len, "the ROCm Qwen executor currently supports greedy sampling only");
        return RIBN_OK;
    }
    const uint64_t need = (total + kPageTokens - 1) / kPageTokens;
    if (need > M->kv_pages) {
        *admission = RIBN_ADMIT_REJECTED;
        set_err(err, err_len, "Qwen needs " + std::to_string(need) + " KV pages, above the " +
                                  std::to_string(M->kv_pages) + "-page pool");
        return RIBN_OK;
    }
    if (M->free_slots.empty() || M->free_pages.size() < need) {
        *admission = RIBN_ADMIT_DEFERRED;
        set_err(err, err_len, "waiting for sequence capacity");
        return RIBN_OK;
    }
    Sequence s;
    s.slot = M->free_slots.back();
    take_pages(M, (uint32_t)total, &s.pages);
    s.prompt_len = n_tokens;
    hipError_t e = reset_slot(M, s.slot, s.pages, tokens, n_tokens);
    if (e != hipSuccess) {
        give_pages(M, s.pages);
        return fail(M, err, err_len, hip_msg("admit", e));
    }
    M->free_slots.pop_back();
    M->seqs.emplace(sequence, std::move(s));
    *admission = RIBN_ADMIT_READY;
    if (err && err_len) err[0] = 0;
    return RIBN_OK;
}

namespace {
int check_item(ribn_rocm_model* M, const ribn_rocm_batch_item& it, char* err, size_t err_len) {
    auto s = M->seqs.find(it.sequence);
    if (s == M->seqs.end()) return fail(nullptr, err, err_len, "unknown Qwen sequence", RIBN_ERR_INVALID);
    if (s->second.in_flight) return fail(nullptr, err, err_len, "Qwen sequence is in flight", RIBN_ERR_INVALID);
    const uint64_t end = (uint64_t)it.prefix + it.token_budget;
    if (it.token_budget == 0 || s->second.committed != it.prefix || end > M->context)
        return fail(nullptr, err, err_len, "Qwen work does not match the sequence prefix/capacity", RIBN_ERR_INVALID);
    if (it.kind == RIBN_STEP_PREFILL) {
        if (end > s->second.prompt_len || it.output_budget != (end == s->second.prompt_len ? 1u : 0u))
            return fail(nullptr, err, err_len, "Qwen prefill boundary/output mismatch", RIBN_ERR_INVALID);
    } else if (it.kind == RIBN_STEP_DECODE) {
        if (it.token_budget != 1 || it.output_budget != 1 || it.prefix < s->second.prompt_len)
            return fail(nullptr, err, err_len, "Qwen adapter only supports one-token ordinary decode", RIBN_ERR_INVALID);
        if (!s->second.has_next) return fail(nullptr, err, err_len, "Qwen decode has no next token", RIBN_ERR_INVALID);
    } else {
        return fail(nullptr, err, err_len, "unknown step kind", RIBN_ERR_INVALID);
    }
    return RIBN_OK;
}
bool same_items(const std::vector<ribn_rocm_batch_item>& a, const ribn_rocm_batch_item* b, size_t n) {
    if (a.size() != n) return false;
    for (size_t i = 0; i < n; i++)
        if (a[i].sequence != b[i].sequence || a[i].kind != b[i].kind || a[i].prefix != b[i].prefix ||
            a[i].token_budget != b[i].token_budget || a[i].output_budget != b[i].output_budget)
            return false;
    return true;
}
}  // namespace

extern "C" int ribn_rocm_prepare(ribn_rocm_model* M, const ribn_rocm_batch_item* items, size_t n, char* err,
                                 size_t err_len) {
    if (!M || (!items && n)) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->faulted || M->has_pending || M->has_prepared)
        return fail(nullptr, err, err_len, "Qwen execution is faulted or busy", M->faulted ? RIBN_ERR_FAULTED : RIBN_ERR_BUSY);
    uint64_t tokens = 0;
    for (size_t i = 0; i < n; i++) tokens += items[i].token_budget;
    if (n > M->max_seqs || tokens > M->max_batch_tokens)
        return fail(nullptr, err, err_len, "Qwen batch exceeds prepared limits", RIBN_ERR_CAPACITY);
    for (size_t i = 0; i < n; i++) {
        int rc = check_item(M, items[i], err, err_len);
        if (rc) return rc;
        for (size_t j = 0; j < i; j++)
            if (items[j].sequence == items[i].sequence)
                return fail(nullptr, err, err_len, "duplicate sequence in batch", RIBN_ERR_INVALID);
    }
    M->prepared.assign(items, items + n);
    M->has_prepared = true;
    return RIBN_OK;
}

extern "C" int ribn_rocm_abandon(ribn_rocm_model* M, char* err, size_t err_len) {
    if (!M) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    M->has_prepared = false;
    M->prepared.clear();
    return RIBN_OK;
}

extern "C" int ribn_rocm_submit(ribn_rocm_model* M, const ribn_rocm_batch_item* items, size_t n, uint64_t* submission,
                                char* err, size_t err_len) {
    if (!M || !submission || (!items && n)) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->faulted || M->has_pending)
        return fail(nullptr, err, err_len, "Qwen execution is faulted or busy", M->faulted ? RIBN_ERR_FAULTED : RIBN_ERR_BUSY);
    if (!M->has_prepared) return fail(nullptr, err, err_len, "Qwen batch was not prepared", RIBN_ERR_INVALID);
    if (!same_items(M->prepared, items, n))
        return fail(nullptr, err, err_len, "Qwen submission differs from its preparation", RIBN_ERR_INVALID);
    M->has_prepared = false;
    M->prepared.clear();
    hipError_t e = hipSuccess;
    if (!M->pending.done) e = hipEventCreateWithFlags(&M->pending.done, hipEventDisableTiming);
    // decode rows (one token, sampled) of two or more sequences run as one batched step
    std::vector<char> batched(n, 0);
    M->last_batch_seqs.clear();
    // (in the integer-dot mode every sampled decode row, also a single one)
    const size_t min_rows = M->int_dot ? 1 : 2;
    if (M->b_rows >= (int)min_rows && M->step_wg == 0) {
        std::vector<int> bslots, bpos;
        std::vector<size_t> brow;
        for (size_t r = 0; r < n; r++) {
            const ribn_rocm_batch_item& it = items[r];
            // a one-token prompt row that samples is a decode row too (integer-dot mode)
            const bool row = it.kind == RIBN_STEP_DECODE || M->int_dot;
            if (row && it.token_budget == 1 && it.output_budget == 1 && (int)bslots.size() < M->b_rows) {
                bslots.push_back(M->seqs[it.sequence].slot);
                bpos.push_back((int)it.prefix);
                brow.push_back(r);
            }
        }
        if (bslots.size() >= min_rows) {
            for (size_t i = 0; i < brow.size(); i++) {
                batched[brow[i]] = 1;
                M->seqs[items[brow[i]].sequence].in_flight = true;
            }
            M->last_batch_seqs.clear();
            for (size_t i = 0; i < brow.size(); i++) M->last_batch_seqs.push_back(items[brow[i]].sequence);
            e = decode_rows(M, bslots, bpos);
            for (size_t i = 0; e == hipSuccess && i < brow.size(); i++)
                e = hipMemcpyAsync(&M->h_out[brow[i]], &M->d_slots[bslots[i]].last_token, 4, hipMemcpyDeviceToHost,
                                   M->stream);
        }
    }
    for (size_t r = 0; e == hipSuccess && r < n; r++) {
        if (batched[r]) continue;
        const ribn_rocm_batch_item& it = items[r];
        Sequence& s = M->seqs[it.sequence];
        s.in_flight = true;
        e = select_slot(M, s.slot);
        const uint32_t end = it.prefix + it.token_budget;
        if (it.token_budget >= 2) {
            // prompt rows: chunked prefill (the last chunk samples when the row has an output)
            if (e == hipSuccess) e = prefill_rows(M, s.slot, (int)it.prefix, (int)it.token_budget, it.output_budget > 0);
        } else {
            for (uint32_t p = it.prefix; e == hipSuccess && p < end; p++) {
                const bool head = (p + 1 == end) && it.output_budget > 0;
                e = run_step(M, head, (int)p + 1, nullptr);
            }
        }
        if (e == hipSuccess && it.output_budget > 0)
            e = hipMemcpyAsync(&M->h_out[r], &M->d_slots[s.slot].last_token, 4, hipMemcpyDeviceToHost, M->stream);
    }
    if (e == hipSuccess) e = hipEventRecord(M->pending.done, M->stream);
    M->pending.items.assign(items, items + n);
    M->pending.id = M->next_submission++;
    M->has_pending = true;
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("submit", e));
    *submission = M->pending.id;
    return RIBN_OK;
}

extern "C" int ribn_rocm_batch_logits(ribn_rocm_model* M, uint64_t* sequences, float* out, size_t cap_rows,
                                      size_t* n_rows, char* err, size_t err_len) {
    if (!M || !n_rows) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->has_pending) return fail(nullptr, err, err_len, "a submission is in flight", RIBN_ERR_BUSY);
    const size_t n = M->last_batch_seqs.size();
    *n_rows = n;
    if (n == 0) return RIBN_OK;
    if (cap_rows < n || !out || !sequences) return fail(nullptr, err, err_len, "output too small", RIBN_ERR_INVALID);
    for (size_t i = 0; i < n; i++) sequences[i] = M->last_batch_seqs[i];
    hipError_t e = hipMemcpyAsync(out, M->b_logits, sizeof(float) * n * M->V, hipMemcpyDeviceToHost, M->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(M->stream);
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("batch_logits", e));
    return RIBN_OK;
}

extern "C" int ribn_rocm_poll(ribn_rocm_model* M, uint64_t submission, ribn_rocm_step_completion* out, size_t cap,
                              size_t* n_out, char* err, size_t err_len) {
    if (!M || !n_out) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (!M->has_pending) return fail(nullptr, err, err_len, "unknown Qwen submission", RIBN_ERR_INVALID);
    if (M->pending.id != submission) return fail(nullptr, err, err_len, "Qwen submission identity mismatch", RIBN_ERR_INVALID);
    if (cap < M->pending.items.size()) return fail(nullptr, err, err_len, "completion array too small", RIBN_ERR_INVALID);
    hipError_t e = hipEventQuery(M->pending.done);
    if (e == hipErrorNotReady) return RIBN_PENDING;
    const std::vector<ribn_rocm_batch_item> items = M->pending.items;
    M->has_pending = false;
    for (auto& it : items) M->seqs[it.sequence].in_flight = false;
    bool barrier_failed = false;
    if (e == hipSuccess) e = step_failed(M, &barrier_failed);
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("poll", e));
    if (barrier_failed) return fail(M, err, err_len, "decode step: a grid barrier wait exceeded its limit");
    for (size_t r = 0; r < items.size(); r++) {
        const auto& it = items[r];
        Sequence& s = M->seqs[it.sequence];
        const uint32_t prefix = it.prefix + it.token_budget;
        ribn_rocm_step_completion c{};
        c.sequence = it.sequence;
        c.prefix = prefix;
        if (it.output_budget > 0) {
            const uint32_t tok = M->h_out[r];
            if (tok >= (uint32_t)M->V) return fail(M, err, err_len, "Qwen completion does not match submitted work");
            c.n_tokens = 1;
            c.token = tok;
            s.next = tok;
            s.has_next = true;
        }
        s.committed = prefix;
        out[r] = c;
    }
    *n_out = items.size();
    return RIBN_OK;
}

extern "C" int ribn_rocm_release(ribn_rocm_model* M, uint64_t sequence, char* err, size_t err_len) {
    if (!M) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    auto it = M->seqs.find(sequence);
    if (it == M->seqs.end()) return RIBN_OK;
    if (it->second.in_flight) return fail(nullptr, err, err_len, "Qwen sequence is in flight", RIBN_ERR_BUSY);
    give_pages(M, it->second.pages);
    M->free_slots.push_back(it->second.slot);
    M->seqs.erase(it);
    return RIBN_OK;
}

extern "C" int ribn_rocm_synchronize(ribn_rocm_model* M, char* err, size_t err_len) {
    if (!M) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    M->has_prepared = false;
    M->prepared.clear();
    hipError_t e = hipStreamSynchronize(M->stream);
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("synchronize", e));
    return RIBN_OK;
}

// ---------------------------------------------------------------------------
// Kernel-level entry points.
namespace {
struct Scoped {
    std::vector<void*> p;
    ~Scoped() { for (void* x : p) hipFree(x); }
    template <typename T>
    hipError_t alloc(T** out, size_t bytes) {
        void* v = nullptr;
        hipError_t e = hipMalloc(&v, bytes ? bytes : 256);
        if (e == hipSuccess) { p.push_back(v); *out = static_cast<T*>(v); }
        return e;
    }
};

hipError_t upload_plain(Scoped& S, uint32_t type, uint64_t rows, uint64_t k, const uint8_t* blocks, QMat* q) {
    uint64_t be, bb;
    type_layout(type, &be, &bb);
    const uint64_t nblocks = rows * (k / be);
    size_t sa, sb, sc, sd;
    plane_sizes(type, nblocks, &sa, &sb, &sc, &sd);
    const size_t total = align256(sa) + align256(sb) + align256(sc) + align256(sd);
    std::vector<uint8_t> host(total);
    uint8_t* ha = host.data();
    uint8_t *hb = ha + align256(sa), *hc = hb + align256(sb), *hd = hc + align256(sc);
    if (blocks) retile(type, blocks, nblocks, ha, hb, hc, hd);
    else {
        // benchmark fill: random quants with finite unit-range scales
        uint64_t x = 0x9e3779b97f4a7c15ull;
        for (size_t i = 0; i < total; i++) { x ^= x << 13; x ^= x >> 7; x ^= x << 17; host[i] = (uint8_t)x; }
        auto put_half = [](uint8_t* p, uint16_t h) { p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); };
        for (uint64_t i = 0; i < nblocks; i++) {
            if (type == GGML_Q4_K) { put_half(hc + i * 4, 0x2000); put_half(hc + i * 4 + 2, 0x2000); }
            else if (type == GGML_Q6_K) put_half(hd + i * 2, 0x2000);
            else put_half(hb + i * 2, 0x2000);
        }
    }
    uint8_t* dev = nullptr;
    hipError_t e = S.alloc(&dev, total);
    if (e != hipSuccess) return e;
    if ((e = hipMemcpy(dev, host.data(), total, hipMemcpyHostToDevice)) != hipSuccess) return e;
    QMat m{};
    m.type = type; m.rows = (uint32_t)rows; m.k = (uint32_t)k; m.nb = (uint32_t)(k / be);
    m.a = dev; m.b = dev + (hb - ha); m.c = dev + (hc - ha); m.d = dev + (hd - ha);
    *q = m;
    return hipSuccess;
}

std::string check_shape(uint32_t type, uint64_t rows, uint64_t k) {
    if (type != GGML_Q4_K && type != GGML_Q6_K && type != GGML_Q8_0) return "unsupported value type " + std::to_string(type);
    uint64_t be, bb;
    type_layout(type, &be, &bb);
    if (rows == 0 || k == 0 || k % be || k % 16) return "k must be a positive multiple of the block size";
    if (rows > (1u << 30) || k > 28672) return "matrix too large for the matvec kernel (k <= 28672)";
    return {};
}
}  // namespace

extern "C" int ribn_rocm_dequantize(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t k, float* out,
                                    char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    std::string m = check_shape(type, rows, k);
    if (!m.empty() || !blocks || !out) return fail(nullptr, err, err_len, m.empty() ? "null argument" : m, RIBN_ERR_INVALID);
    Scoped S;
    QMat q;
    float* dout = nullptr;
    HIPCHK(upload_plain(S, type, rows, k, blocks, &q));
    HIPCHK(S.alloc(&dout, sizeof(float) * rows * k));
    HIPCHK(launch_dequant(q, dout, nullptr));
    HIPCHK(hipMemcpy(out, dout, sizeof(float) * rows * k, hipMemcpyDeviceToHost));
    return RIBN_OK;
}

extern "C" int ribn_rocm_gemv(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t k, const float* x,
                              const float* rms_weight, float eps, float* y, char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    std::string m = check_shape(type, rows, k);
    if (!m.empty() || !blocks || !x || !y) return fail(nullptr, err, err_len, m.empty() ? "null argument" : m, RIBN_ERR_INVALID);
    Scoped S;
    QMat q;
    float *dx = nullptr, *dw = nullptr, *dy = nullptr;
    HIPCHK(upload_plain(S, type, rows, k, blocks, &q));
    HIPCHK(S.alloc(&dx, sizeof(float) * k));
    HIPCHK(S.alloc(&dy, sizeof(float) * rows));
    HIPCHK(hipMemcpy(dx, x, sizeof(float) * k, hipMemcpyHostToDevice));
    if (rms_weight) {
        HIPCHK(S.alloc(&dw, sizeof(float) * k));
        HIPCHK(hipMemcpy(dw, rms_weight, sizeof(float) * k, hipMemcpyHostToDevice));
    }
    MvArgs a = mv_base(dx, dw, eps, (int)k, MV_STORE, nullptr);
    a.nseg = 1;
    a.type_a = a.type_b = type;
    a.seg[0].w = q;
    a.seg[0].out = dy;
    a.items_per_wave = choose_ipw((int)(rows / 2), 4);
    const int nwg = layout_segments(a);
    HIPCHK(launch_matvec(a, nwg, nullptr));
    HIPCHK(hipMemcpy(y, dy, sizeof(float) * rows, hipMemcpyDeviceToHost));
    return RIBN_OK;
}

extern "C" int ribn_rocm_bench_gemv(uint32_t type, uint64_t rows, uint64_t k, uint32_t iters, double* avg_ms, char* err,
                                    size_t err_len) {
    ribn_rocm_model* M = nullptr;
    std::string m = check_shape(type, rows, k);
    if (!m.empty() || !avg_ms || iters == 0) return fail(nullptr, err, err_len, m.empty() ? "bad argument" : m, RIBN_ERR_INVALID);
    Scoped S;
    QMat q;
    float *dx = nullptr, *dy = nullptr;
    HIPCHK(upload_plain(S, type, rows, k, nullptr, &q));
    HIPCHK(S.alloc(&dx, sizeof(float) * k));
    HIPCHK(S.alloc(&dy, sizeof(float) * rows));
    std::vector<float> hx(k, 0.5f);
    HIPCHK(hipMemcpy(dx, hx.data(), sizeof(float) * k, hipMemcpyHostToDevice));
    MvArgs a = mv_base(dx, nullptr, 0.f, (int)k, MV_STORE, nullptr);
    a.nseg = 1;
    a.type_a = a.type_b = type;
    a.seg[0].w = q;
    a.seg[0].out = dy;
    a.items_per_wave = choose_ipw((int)(rows / 2), 4);
    const int nwg = layout_segments(a);
    hipStream_t st;
    HIPCHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    for (int i = 0; i < 3; i++) HIPCHK(launch_matvec(a, nwg, st));
    HIPCHK(hipEventRecord(e0, st));
    for (uint32_t i = 0; i < iters; i++) HIPCHK(launch_matvec(a, nwg, st));
    HIPCHK(hipEventRecord(e1, st));
    HIPCHK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, e0, e1));
    *avg_ms = ms / iters;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipStreamDestroy(st);
    return RIBN_OK;
}

extern "C" int ribn_rocm_quantize_q8_1(const float* x, uint64_t n, uint32_t* out, char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    if (!x || !out) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (n == 0 || n % 32)
        return fail(nullptr, err, err_len, "Q8_1 input length must be a positive multiple of 32", RIBN_ERR_INVALID);
    Scoped S;
    float* dx = nullptr;
    uint32_t* dq = nullptr;
    HIPCHK(S.alloc(&dx, sizeof(float) * n));
    HIPCHK(S.alloc(&dq, sizeof(uint32_t) * (n / 32) * 9));
    HIPCHK(hipMemcpy(dx, x, sizeof(float) * n, hipMemcpyHostToDevice));
    HIPCHK(launch_quantize_q8_1(dx, n, dq, nullptr));
    HIPCHK(hipMemcpy(out, dq, sizeof(uint32_t) * (n / 32) * 9, hipMemcpyDeviceToHost));
    return RIBN_OK;
}

std::string check_intdot(uint32_t type, uint64_t rows, uint64_t k, uint32_t members) {
    std::string m = check_shape(type, rows, k);
    if (!m.empty()) return m;
    if (type != 8 && type != 12 && type != 14) return "no integer-dot kernel for this value type";
    if (members < 1 || members > (uint32_t)kIdMaxMembers) return "members must be 1 .. 8";
    if (rows > 0x7fffffffu / members) return "output too large";
    return "";
}

extern "C" int ribn_rocm_gemv_q8_1(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t k,
                                   const uint32_t* packed, uint32_t members, float* y, char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    std::string m = check_intdot(type, rows, k, members);
    if (!m.empty() || !blocks || !packed || !y)
        return fail(nullptr, err, err_len, m.empty() ? "null argument" : m, RIBN_ERR_INVALID);
    Scoped S;
    QMat q;
    uint32_t* dq = nullptr;
    float* dy = nullptr;
    const size_t words = (size_t)members * (k / 32) * 9;
    HIPCHK(upload_plain(S, type, rows, k, blocks, &q));
    HIPCHK(S.alloc(&dq, sizeof(uint32_t) * words));
    HIPCHK(S.alloc(&dy, sizeof(float) * rows * members));
    HIPCHK(hipMemcpy(dq, packed, sizeof(uint32_t) * words, hipMemcpyHostToDevice));
    IdArgs a{};
    a.xq = dq;
    a.k = (int)k;
    a.members = (int)members;
    a.ld = (int)rows;
    a.mode = MV_STORE;
    a.nseg = 1;
    a.type_a = a.type_b = type;
    a.seg[0].w = q;
    a.seg[0].out = dy;
    const int nwg = intdot_layout(a, device_cus());
    HIPCHK(launch_intdot(a, nwg, nullptr));
    HIPCHK(hipMemcpy(y, dy, sizeof(float) * rows * members, hipMemcpyDeviceToHost));
    return RIBN_OK;
}

extern "C" int ribn_rocm_bench_gemv_q8_1(uint32_t type, uint64_t rows, uint64_t k, uint32_t members, uint32_t iters,
                                         double* avg_ms, char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    std::string m = check_intdot(type, rows, k, members);
    if (!m.empty() || !avg_ms || iters == 0)
        return fail(nullptr, err, err_len, m.empty() ? "bad argument" : m, RIBN_ERR_INVALID);
    Scoped S;
    QMat q;
    float *dx = nullptr, *dy = nullptr;
    uint32_t* dq = nullptr;
    HIPCHK(upload_plain(S, type, rows, k, nullptr, &q));
    HIPCHK(S.alloc(&dx, sizeof(float) * k * members));
    HIPCHK(S.alloc(&dq, sizeof(uint32_t) * members * (k / 32) * 9));
    HIPCHK(S.alloc(&dy, sizeof(float) * rows * members));
    std::vector<float> hx(k * members);
    for (size_t i = 0; i < hx.size(); i++) hx[i] = (float)((int)(i * 37 % 101) - 50) * 0.01f;
    HIPCHK(hipMemcpy(dx, hx.data(), sizeof(float) * hx.size(), hipMemcpyHostToDevice));
    HIPCHK(launch_quantize_q8_1(dx, hx.size(), dq, nullptr));
    IdArgs a{};
    a.xq = dq;
    a.k = (int)k;
    a.members = (int)members;
    a.ld = (int)rows;
    a.mode = MV_STORE;
    a.nseg = 1;
    a.type_a = a.type_b = type;
    a.seg[0].w = q;
    a.seg[0].out = dy;
    const int nwg = intdot_layout(a, device_cus());
    hipStream_t st;
    HIPCHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    for (int i = 0; i < 3; i++) HIPCHK(launch_intdot(a, nwg, st));
    HIPCHK(hipEventRecord(e0, st));
    for (uint32_t i = 0; i < iters; i++) HIPCHK(launch_intdot(a, nwg, st));
    HIPCHK(hipEventRecord(e1, st));
    HIPCHK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, e0, e1));
    *avg_ms = ms / iters;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipStreamDestroy(st);
    return RIBN_OK;
}

extern "C" int ribn_rocm_bench_model_kernel(ribn_rocm_model* M, uint32_t which, uint32_t iters, double* avg_ms,
                                            uint64_t* bytes, char* err, size_t err_len) {
    if (!M || !avg_ms || !bytes || iters == 0) return fail(nullptr, err, err_len, "bad argument", RIBN_ERR_INVALID);
    if (M->faulted) return fail(nullptr, err, err_len, "ROCm execution is faulted", RIBN_ERR_FAULTED);
    MvArgs a;
    int nwg;
    auto qbytes = [](const QMat& q) {
        uint64_t be, bb;
        type_layout(q.type, &be, &bb);
        return (uint64_t)q.rows * q.nb * bb;
    };
    bool attn = false;
    AttnArgs at{};
    std::vector<int32_t> bench_pages;
    struct PageReturn {
        ribn_rocm_model* M;
        std::vector<int32_t>* p;
        ~PageReturn() {
            if (!p->empty()) {
                hipStreamSynchronize(M->stream);
                give_pages(M, *p);
            }
        }
    } page_return{M, &bench_pages};
    switch (which) {
    case 0: a = M->mv_gu[0]; nwg = M->wg_gu[0]; *bytes = qbytes(a.seg[0].w) + qbytes(a.seg[0].w2); break;
    case 1: a = M->mv_down[0]; nwg = M->wg_down[0]; a.mode = MV_STORE; a.seg[0].out = M->act; *bytes = qbytes(a.seg[0].w); break;
    case 2: a = M->mv_head; nwg = M->head_wgs; a.mode = MV_STORE; *bytes = qbytes(a.seg[0].w); break;
    case 3: case 4:
        a = M->mv_qkv[0]; nwg = M->wg_qkv[0];
        *bytes = qbytes(a.seg[0].w) + qbytes(a.seg[1].w) + qbytes(a.seg[2].w);
        break;
    case 5: a = M->mv_o[0]; nwg = M->wg_o[0]; a.mode = MV_STORE; a.seg[0].out = M->act; *bytes = qbytes(a.seg[0].w); break;
    case 6: {
        // decode attention of layer 0 for a scratch sequence holding exactly
        // `ctx` positions (the current token is position ctx-1)
        const int ctx = (int)(*bytes & 0xffffffffu), force = (int)(*bytes >> 32);
        if (force && (force > kMaxSplits || (force & (force - 1)) ||
                      (ctx + force - 1) / force > kMaxSplitTokens - kPageTokens))
            return fail(nullptr, err, err_len, "attention bench split count unusable for this context", RIBN_ERR_INVALID);
        if (ctx < 1 || (uint32_t)ctx > M->context)
            return fail(nullptr, err, err_len, "attention bench context outside the prepared context", RIBN_ERR_INVALID);
        if (!take_pages(M, (uint32_t)ctx, &bench_pages))
            return fail(nullptr, err, err_len, "not enough free KV pages", RIBN_ERR_CAPACITY);
        const int slot = (int)M->max_seqs;
        const uint32_t tok0 = 0;
        HIPCHK(reset_slot(M, slot, bench_pages, &tok0, 1));
        M->h_state[slot].pos = ctx - 1;
        M->h_ctl[slot].pos = ctx - 1;   // no embedding kernel runs here to publish it
        HIPCHK(hipMemcpyAsync(&M->d_slots[slot], &M->h_state[slot], sizeof(SeqState), hipMemcpyHostToDevice, M->stream));
        HIPCHK(select_slot(M, slot));
        attn = true;
        at = attn_args(M, 0, force ? force : splits_for_ctx(ctx));
        *bytes = 0;
        break;
    }
    case 7: {
        // every layer's gate/up launch inside graph-replayed decode steps of a
        // scratch sequence holding `ctx` positions (weights streamed from HBM by
        // the other launches in between, as in the decode loop)
        const int ctx = (int)(*bytes & 0xffffffffu);
        if (M->hybrid || M->step_wg) return fail(nullptr, err, err_len, "chain timing needs the dense launch chain", RIBN_ERR_INVALID);
        if (ctx < 1 || (uint32_t)(ctx + iters + 1) > M->context)
            return fail(nullptr, err, err_len, "chain timing context outside the prepared context", RIBN_ERR_INVALID);
        if (!take_pages(M, (uint32_t)(ctx + iters + 1), &bench_pages))
            return fail(nullptr, err, err_len, "not enough free KV pages", RIBN_ERR_CAPACITY);
        const int slot = (int)M->max_seqs;
        // token 0 at every position the steps embed (the embedding reads tokens[pos] unchecked)
        const std::vector<uint32_t> toks((size_t)ctx + iters + 1, 0u);
        HIPCHK(reset_slot(M, slot, bench_pages, toks.data(), (uint32_t)toks.size()));
        M->h_state[slot].pos = ctx - 1;
        HIPCHK(hipMemcpyAsync(&M->d_slots[slot], &M->h_state[slot], sizeof(SeqState), hipMemcpyHostToDevice, M->stream));
        HIPCHK(select_slot(M, slot));
        const int ns = splits_for_ctx(ctx + (int)iters);
        if (splits_for_ctx(ctx) != ns) return fail(nullptr, err, err_len, "chain timing steps cross a split-count bucket", RIBN_ERR_INVALID);
        // every gate/up launch (its timing variant) folds its first start and last
        // end into its own pair of device words; captured into a graph of its
        // own (the decode graphs run the plain kernel)
        const int L = M->L;
        unsigned long long* clk = nullptr;
        HIPCHK(hipMalloc(&clk, sizeof(unsigned long long) * 2 * L));
        struct ClkFree {
            unsigned long long* p;
            ~ClkFree() { hipFree(p); }
        } clk_free{clk};
        std::vector<unsigned long long> init(2 * L), got(2 * L);
        for (int l = 0; l < L; l++) {
            init[2 * l] = ~0ull;
            init[2 * l + 1] = 0ull;
        }
        M->gu_clk = clk;
        hipGraph_t g = nullptr;
        hipError_t e1 = hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal);
        if (e1 == hipSuccess) {
            e1 = enqueue_step(M, false, ns, nullptr);
            const hipError_t e2 = hipStreamEndCapture(M->stream, &g);
            if (e1 == hipSuccess) e1 = e2;
        }
        M->gu_clk = nullptr;
        if (e1 != hipSuccess) {
            if (g) hipGraphDestroy(g);
            HIPCHK(e1);
        }
        hipGraphExec_t ex = nullptr;
        const hipError_t e3 = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        HIPCHK(e3);
        double ticks = 0.0;
        hipError_t e4 = hipSuccess;
        for (uint32_t i = 0; i < iters && e4 == hipSuccess; i++) {
            e4 = hipMemcpy(clk, init.data(), sizeof(unsigned long long) * 2 * L, hipMemcpyHostToDevice);
            if (e4 == hipSuccess) e4 = hipGraphLaunch(ex, M->stream);
            if (e4 == hipSuccess) e4 = hipStreamSynchronize(M->stream);
            if (e4 == hipSuccess) e4 = hipMemcpy(got.data(), clk, sizeof(unsigned long long) * 2 * L, hipMemcpyDeviceToHost);
            for (int l = 0; l < L && e4 == hipSuccess; l++) ticks += (double)(got[2 * l + 1] - got[2 * l]);
        }
        hipGraphExecDestroy(ex);
        HIPCHK(e4);
        int khz = 0;
        HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, M->device));
        *avg_ms = ticks / ((double)iters * L) / (double)khz;
        a = M->mv_gu[0];
        *bytes = qbytes(a.seg[0].w) + qbytes(a.seg[0].w2);
        return RIBN_OK;
    }
    default: return fail(nullptr, err, err_len, "unknown kernel selector", RIBN_ERR_INVALID);
    }
    if (attn) {
        hipEvent_t e0, e1;
        HIPCHK(hipEventCreate(&e0));
        HIPCHK(hipEventCreate(&e1));
        // as in the decode chain: long contexts merge in a launch of their own
        const bool apart = merge_apart_for(M, at.n_splits);
        at.defer = apart ? 2 : 0;
        auto run = [&]() -> hipError_t {
            hipError_t e2 = launch_attention(at, M->stream);
            if (e2 == hipSuccess && apart) e2 = launch_attention_merge(at, M->stream);
            return e2;
        };
        for (int i = 0; i < 3; i++) HIPCHK(run());
        HIPCHK(hipEventRecord(e0, M->stream));
        for (uint32_t i = 0; i < iters; i++) HIPCHK(run());
        HIPCHK(hipEventRecord(e1, M->stream));
        HIPCHK(hipEventSynchronize(e1));
        float ms = 0.f;
        HIPCHK(hipEventElapsedTime(&ms, e0, e1));
        *avg_ms = ms / iters;
        hipEventDestroy(e0);
        hipEventDestroy(e1);
        return RIBN_OK;
    }
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    for (int i = 0; i < 3; i++) HIPCHK(launch_matvec(a, nwg, M->stream));
    HIPCHK(hipEventRecord(e0, M->stream));
    for (uint32_t i = 0; i < iters; i++) HIPCHK(launch_matvec(a, nwg, M->stream));
    HIPCHK(hipEventRecord(e1, M->stream));
    HIPCHK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, e0, e1));
    *avg_ms = ms / iters;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return RIBN_OK;
}

extern "C" int ribn_rocm_argmax(const float* logits, uint64_t n, uint32_t* out, char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    if (!logits || !out || n == 0 || n > 0xffffffffull) return fail(nullptr, err, err_len, "bad argument", RIBN_ERR_INVALID);
    Scoped S;
    float* dl = nullptr;
    uint64_t* part = nullptr;
    uint32_t *ctr = nullptr, *dout = nullptr;
    HIPCHK(S.alloc(&dl, sizeof(float) * n));
    HIPCHK(S.alloc(&part, sizeof(uint64_t) * 1024));
    HIPCHK(S.alloc(&ctr, sizeof(uint32_t) * 2));
    dout = ctr + 1;
    HIPCHK(hipMemset(ctr, 0, 8));
    HIPCHK(hipMemcpy(dl, logits, sizeof(float) * n, hipMemcpyHostToDevice));
    HIPCHK(launch_argmax(dl, (uint32_t)n, part, ctr, dout, nullptr));
    HIPCHK(hipMemcpy(out, dout, 4, hipMemcpyDeviceToHost));
    return RIBN_OK;
}

// Timing of one persistent decode step on the scratch sequence (which must
// hold `ctx` positions, e.g. after ribn_rocm_generate): workgroup 0's wall
// clock at the step's start, at every barrier arrival and release, after every
// input staging and at every stage end, in ns from the start. *n receives the
// number of marks.
extern "C" int ribn_rocm_step_stamps(ribn_rocm_model* M, uint32_t ctx, double* out_ns, size_t cap, size_t* n,
                                     char* err, size_t err_len) {
    if (!M || !out_ns || !n) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->step_wg == 0) return fail(nullptr, err, err_len, "this model runs the launch chain", RIBN_ERR_INVALID);
    const size_t count = 64 * ((size_t)M->L + 1);
    if (cap < count) return fail(nullptr, err, err_len, "stamp array too small", RIBN_ERR_INVALID);
    if (ctx < 1 || ctx > M->context) return fail(nullptr, err, err_len, "ctx outside the context", RIBN_ERR_INVALID);
    const int slot = (int)M->max_seqs;
    uint64_t* d = nullptr;
    HIPCHK(hipMalloc(&d, sizeof(uint64_t) * count));
    HIPCHK(hipMemset(d, 0, sizeof(uint64_t) * count));
    SeqState s = M->h_state[slot];
    s.pos = (int)ctx - 1;
    HIPCHK(hipMemcpy(&M->d_slots[slot], &s, sizeof(SeqState), hipMemcpyHostToDevice));
    HIPCHK(select_slot(M, slot));
    StepArgs a = M->step_args;
    a.head = 1;
    a.stamps = d;
    HIPCHK(launch_step(a, M->step_key, M->step_wg, M->step_lds, M->stream));
    HIPCHK(hipStreamSynchronize(M->stream));
    std::vector<uint64_t> h(count);
    HIPCHK(hipMemcpy(h.data(), d, sizeof(uint64_t) * count, hipMemcpyDeviceToHost));
    hipFree(d);
    int khz = 0;
    HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, M->device));
    size_t m = 0;
    while (m < count && h[m] != 0) m++;
    for (size_t i = 0; i < m; i++) out_ns[i] = (double)(h[i] - h[0]) * 1e6 / (double)khz;
    *n = m;
    return RIBN_OK;
}

// ---------------------------------------------------------------------------
// Chunked-prefill parity entry points.

// Runs tokens[0..n) through chunked prefill (chunks of min(chunk, prepared)
// rows) on the scratch sequence; logits_out [n][vocab] of every row (final
// RMSNorm + head, same GEMM path) and hidden_out [(layers + 1)][n][hidden]
// (after the embedding and after every layer), both optional.
extern "C" int ribn_rocm_prefill_trace(ribn_rocm_model* M, const uint32_t* tokens, uint32_t n, uint32_t chunk,
                                       float* logits_out, float* hidden_out, char* err, size_t err_len) {
    if (!M || !tokens) return fail(nullptr, err, err_len, "null argument", RIBN_ERR_INVALID);
    if (M->faulted) return fail(nullptr, err, err_len, "ROCm execution is faulted", RIBN_ERR_FAULTED);
    if (M->has_pending) return fail(nullptr, err, err_len, "a submission is in flight", RIBN_ERR_BUSY);
    if (M->int_dot)
        return fail(nullptr, err, err_len, "traces run the float projections: not in the integer-dot mode", RIBN_ERR_INVALID);
    if (n == 0 || n + 1 > M->context) return fail(nullptr, err, err_len, "trace length outside the context", RIBN_ERR_INVALID);
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)M->V) return fail(nullptr, err, err_len, "token id out of range", RIBN_ERR_INVALID);
    if (M->hybrid)
        return fail(nullptr, err, err_len, "qwen35 hybrids have no chunked prefill (prompt rows run as decode steps)",
                    RIBN_ERR_INVALID);
    const int c = (int)std::max<uint32_t>(1, std::min<uint32_t>(chunk ? chunk : M->chunk, (uint32_t)M->chunk));
    std::vector<int32_t> pages;
    if (!take_pages(M, n + 1, &pages)) return fail(nullptr, err, err_len, "not enough free KV pages", RIBN_ERR_CAPACITY);
    const int slot = (int)M->max_seqs;
    float *dtrace = nullptr, *dlog = nullptr;
    hipError_t e = hipMalloc(&dtrace, sizeof(float) * (size_t)(M->L + 1) * c * M->H);
    if (e == hipSuccess && logits_out) e = hipMalloc(&dlog, sizeof(float) * (size_t)c * M->V);
    if (e == hipSuccess) e = reset_slot(M, slot, pages, tokens, n);
    if (e == hipSuccess) e = select_slot(M, slot);
    for (uint32_t p0 = 0; e == hipSuccess && p0 < n; p0 += c) {
        const int m = (int)std::min<uint32_t>(c, n - p0);
        e = prefill_chunk(M, slot, (int)p0, m, false, dtrace);
        if (e == hipSuccess && logits_out) {
            e = launch_rows_rms_f16(M->p_h, m, M->H, M->out_norm, M->eps, true, M->p_x16, M->H, M->stream);
            PrefillGemm g{};
            g.x = M->p_x16; g.m = m; g.k = M->H; g.y = dlog; g.ldy = M->V; g.mode = MV_STORE;
            g.nseg = 1;
            g.seg[0].w = M->out;
            if (e == hipSuccess) e = launch_prefill_gemm(g, M->stream);
            if (e == hipSuccess)
                e = hipMemcpyAsync(logits_out + (size_t)p0 * M->V, dlog, sizeof(float) * m * M->V, hipMemcpyDeviceToHost,
                                   M->stream);
        }
        for (int l = 0; e == hipSuccess && hidden_out && l <= M->L; l++)
            e = hipMemcpyAsync(hidden_out + ((size_t)l * n + p0) * M->H, dtrace + (size_t)l * m * M->H,
                               sizeof(float) * m * M->H, hipMemcpyDeviceToHost, M->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(M->stream);
    }
    if (dtrace) hipFree(dtrace);
    if (dlog) hipFree(dlog);
    give_pages(M, pages);
    if (e != hipSuccess) return fail(M, err, err_len, hip_msg("prefill trace", e));
    return RIBN_OK;
}

// Y[m][rows] = f16(X)[m][k] deq(W)^T with the prefill GEMM (X rounded to binary16
// on the device, W re-tiled like model tensors).
extern "C" int ribn_rocm_prefill_gemm(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t k, const float* x,
                                      uint64_t m, float* y, char* err, size_t err_len) {
    ribn_rocm_model* M = nullptr;
    std::string msg = check_shape(type, rows, k);
    if (!msg.empty() || !blocks || !x || !y || m == 0)
        return fail(nullptr, err, err_len, msg.empty() ? "null argument" : msg, RIBN_ERR_INVALID);
    if (type != GGML_Q8_0 && k % 256) return fail(nullptr, err, err_len, "k must be a multiple of 256", RIBN_ERR_INVALID);
    Scoped S;
    QMat q;
    float *dx = nullptr, *dy = nullptr;
    uint16_t* dx16 = nullptr;
    HIPCHK(upload_plain(S, type, rows, k, blocks, &q));
    HIPCHK(S.alloc(&dx, sizeof(float) * m * k));
    HIPCHK(S.alloc(&dy, sizeof(float) * m * rows));
    HIPCHK(S.alloc(&dx16, 2 * m * k));
    HIPCHK(hipMemcpy(dx, x, sizeof(float) * m * k, hipMemcpyHostToDevice));
    HIPCHK(launch_rows_rms_f16(dx, (int)m, (int)k, nullptr, 0.f, false, dx16, (int)k, nullptr));
    PrefillGemm g{};
    g.x = dx16; g.m = (int)m; g.k = (int)k; g.y = dy; g.ldy = (int)rows; g.mode = MV_STORE;
    g.nseg = 1;
    g.seg[0].w = q;
    g.ksplit = prefill_gemm_splits((int)m, (int)k, gemm_tiles((int)rows));
    if (g.ksplit > 1) HIPCHK(S.alloc(&g.part, sizeof(float) * g.ksplit * m * rows));
    HIPCHK(launch_prefill_gemm(g, nullptr));
    HIPCHK(hipMemcpy(y, dy, sizeof(float) * m * rows, hipMemcpyDeviceToHost));
    return RIBN_OK;
}
