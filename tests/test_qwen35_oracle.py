"""The qwen35 hybrid oracle (oracle/qwen35.c: Gated-DeltaNet recurrent layers + gated full attention), pinned
without running the reference (which is Rust):

- the delta rule against the reference's own algebraic identity: its chunked (UT-transform) form equals the
  token recurrence, with the reference test's literal inputs (crates/nvidia/tests/gdn_chunk_reference.rs:
  213-272; the chunk form restated in FP64 numpy from :78-206) and every chunk size;
- delta-rule closed forms: beta = 0 only decays the state; from a zero state with a unit key and beta = 1
  the state becomes k v^T and the read is (q . k) v / sqrt(d);
- the composed hybrid forward against an independent FP64 numpy forward written from the reference's host
  equations (crates/nvidia/src/qwen_reference.rs:31-556) and layer wiring (crates/nvidia/src/decode.rs:
  550-700), on the dequantized weights: logits and every layer's hidden state.
"""
import numpy as np
import pytest

import oracle_ffi as orc
import ribn_amd

# gdn_chunk_reference.rs:218-230 (inputs of chunked_gated_delta_rule_matches_token_recurrence)
QUERY = [0.2, -0.1, 0.7, 0.5, 0.3, -0.4, -0.6, 0.8, 0.1, 0.9, -0.2, 0.4, 0.3, 0.6, -0.5, -0.7, -0.1, 0.8, 0.4, -0.9,
         0.2]
KEY = [0.4, -0.3, 0.5, -0.2, 0.7, 0.1, 0.6, 0.2, -0.4, -0.5, 0.3, 0.8, 0.1, -0.8, 0.6, 0.7, 0.4, -0.2, -0.3, 0.9, 0.2]
VALUE = [0.7, -0.2, 0.1, 0.8, -0.6, 0.5, 0.4, -0.9, 0.3, 0.2, -0.1, 0.6, 0.9, -0.4]
LOG_DECAY = [-0.11, -0.27, -0.04, -0.33, -0.19, -0.08, -0.22]
BETA = [0.25, 0.73, 0.41, 0.88, 0.36, 0.64, 0.52]
INITIAL = [0.15, -0.2, 0.05, 0.31, -0.17, 0.09]


def _chunk_rule(q, k, v, log_decay, beta, s0, chunk):
    """The chunked gated delta rule (UT transform), FP64."""
    T, kd = q.shape
    vd = v.shape[1]
    S = s0.copy()
    out = np.zeros((T, vd))
    scale = 1.0 / np.sqrt(kd)
    for c0 in range(0, T, chunk):
        n = min(chunk, T - c0)
        cum = np.cumsum(log_decay[c0:c0 + n])
        qc, kc, vc, bc = q[c0:c0 + n], k[c0:c0 + n], v[c0:c0 + n], beta[c0:c0 + n]
        decay = np.exp(cum[:, None] - cum[None, :])
        intra = np.tril((qc @ kc.T) * scale * decay)
        lower = np.tril(bc[:, None] * (kc @ kc.T) * decay, -1)
        A = np.eye(n) + lower
        new_v = np.linalg.solve(A, bc[:, None] * vc)
        dec_k = np.linalg.solve(A, bc[:, None] * kc * np.exp(cum)[:, None])
        upd = new_v - dec_k @ S
        out[c0:c0 + n] = (qc * scale * np.exp(cum)[:, None]) @ S + intra @ upd
        S = S * np.exp(cum[-1]) + (kc * np.exp(cum[-1] - cum)[:, None]).T @ upd
    return out, S


def test_delta_rule_matches_the_chunked_identity():
    q, k, v = (np.array(x, np.float64).reshape(7, -1) for x in (QUERY, KEY, VALUE))
    s0 = np.array(INITIAL, np.float64).reshape(3, 2)
    state = s0.astype(np.float32)
    outs = []
    for t in range(7):
        state, o = orc.gdn_state_step(state, k[t], v[t], q[t], np.exp(np.float32(LOG_DECAY[t])), BETA[t])
        outs.append(o)
    outs = np.stack(outs)
    for chunk in range(1, 10):
        ref_o, ref_s = _chunk_rule(q, k, v, np.array(LOG_DECAY), np.array(BETA), s0, chunk)
        assert np.abs(outs - ref_o).max() <= 2e-5, chunk          # the reference test's tolerance
        assert np.abs(state - ref_s).max() <= 2e-5, chunk


def test_delta_rule_closed_forms():
    rng = np.random.default_rng(0)
    d = 16
    s = rng.standard_normal((d, d)).astype(np.float32)
    q, k, v = (rng.standard_normal(d).astype(np.float32) for _ in range(3))
    s2, _ = orc.gdn_state_step(s, k, v, q, 0.5, 0.0)            # beta 0: decay only
    assert np.allclose(s2, 0.5 * s, rtol=1e-6, atol=1e-7)
    k1 = np.zeros(d, np.float32)
    k1[3] = 1.0
    s3, o = orc.gdn_state_step(np.zeros((d, d), np.float32), k1, v, q, 0.9, 1.0)
    assert np.allclose(s3, np.outer(k1, v), atol=1e-7)
    assert np.allclose(o, q[3] * v / np.sqrt(d), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- FP64 brute force of the composed forward
def _weights(path):
    g = orc.Gguf(path)

    def T(name):
        r = g.tensor(name)
        if isinstance(r, int):
            return None
        t, dims, _, data = r
        return orc.dequantize(t, data).astype(np.float64).reshape(list(reversed(dims)))
    u = lambda k: g.u64("qwen35." + k)   # noqa: E731
    cfg = {k: u(k) for k in ("embedding_length", "block_count", "attention.head_count", "attention.head_count_kv",
                             "attention.key_length", "ssm.group_count", "ssm.time_step_rank", "ssm.state_size",
                             "full_attention_interval", "rope.dimension_count", "ssm.conv_kernel")}
    W = {"embd": T("token_embd.weight"), "out": T("output.weight"), "onorm": T("output_norm.weight"), "L": []}
    if W["out"] is None:
        W["out"] = W["embd"]
    names = ("attn_norm.weight", "post_attention_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight",
             "attn_qkv.weight", "attn_gate.weight", "ssm_beta.weight", "ssm_alpha.weight", "ssm_dt.bias", "ssm_a",
             "ssm_conv1d.weight", "ssm_norm.weight", "ssm_out.weight", "attn_q.weight", "attn_k.weight",
             "attn_v.weight", "attn_q_norm.weight", "attn_k_norm.weight", "attn_output.weight")
    for l in range(cfg["block_count"]):
        W["L"].append({n: T(f"blk.{l}.{n}") for n in names})
    g.close()
    return cfg, W


def _fp64_forward(cfg, W, tokens, eps=1e-6, base=1e7):
    H, L = cfg["embedding_length"], cfg["block_count"]
    hq, hkv, hd, rot = cfg["attention.head_count"], cfg["attention.head_count_kv"], cfg["attention.key_length"], \
        cfg["rope.dimension_count"]
    HK, HV, D, KC = cfg["ssm.group_count"], cfg["ssm.time_step_rank"], cfg["ssm.state_size"], cfg["ssm.conv_kernel"]
    every = cfg["full_attention_interval"]
    rms = lambda x, w: x / np.sqrt(np.mean(x * x) + eps) * w   # noqa: E731
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))                   # noqa: E731
    l2 = lambda x: x / max(np.sqrt(np.sum(x * x)), eps)        # noqa: E731

    def rope(x, pos):
        x = x.copy()
        half = rot // 2
        theta = pos * base ** (-(2.0 * np.arange(half)) / rot)
        c, s = np.cos(theta), np.sin(theta)
        a, b = x[:, :half].copy(), x[:, half:rot].copy()
        x[:, :half], x[:, half:rot] = a * c - b * s, a * s + b * c
        return x

    state = [np.zeros((HV, D, D)) for _ in range(L)]
    conv = [np.zeros((2 * HK * D + HV * D, KC - 1)) for _ in range(L)]
    Kc = [[] for _ in range(L)]
    Vc = [[] for _ in range(L)]
    logits, hidden = [], []
    for pos, tok in enumerate(tokens):
        h = W["embd"][tok].copy()
        trace = [h.copy()]
        for l in range(L):
            y = W["L"][l]
            xn = rms(h, y["attn_norm.weight"])
            if (l + 1) % every:
                mixed = y["attn_qkv.weight"] @ xn
                z = y["attn_gate.weight"] @ xn
                beta = sig(y["ssm_beta.weight"] @ xn)
                a = y["ssm_alpha.weight"] @ xn + y["ssm_dt.bias"]
                gate = np.where(a > 20, a, np.log1p(np.exp(a))) * y["ssm_a"]
                w = y["ssm_conv1d.weight"]                  # [channels][taps]
                window = np.concatenate([conv[l], mixed[:, None]], axis=1)
                out = np.sum(window * w, axis=1)
                conv[l] = window[:, 1:]
                act = out * sig(out)
                q = np.stack([l2(act[i * D:(i + 1) * D]) for i in range(HK)])
                k = np.stack([l2(act[(HK + i) * D:(HK + i + 1) * D]) for i in range(HK)])
                v = act[2 * HK * D:].reshape(HV, D)
                o = np.zeros((HV, D))
                for j in range(HV):
                    S = state[l][j] * np.exp(gate[j])
                    kk = k[j % HK]
                    dlt = (v[j] - kk @ S) * beta[j]
                    S = S + np.outer(kk, dlt)
                    state[l][j] = S
                    o[j] = (q[j % HK] @ S) / np.sqrt(D)
                zz = z.reshape(HV, D)
                gated = np.stack([o[j] / np.sqrt(np.mean(o[j] ** 2) + eps) * y["ssm_norm.weight"] * zz[j] * sig(zz[j])
                                  for j in range(HV)])
                h = h + y["ssm_out.weight"] @ gated.ravel()
            else:
                qg = (y["attn_q.weight"] @ xn).reshape(hq, 2 * hd)
                q = np.stack([rms(r, y["attn_q_norm.weight"]) for r in qg[:, :hd]])
                gate = qg[:, hd:]
                k = np.stack([rms(r, y["attn_k_norm.weight"]) for r in (y["attn_k.weight"] @ xn).reshape(hkv, hd)])
                v = (y["attn_v.weight"] @ xn).reshape(hkv, hd)
                q, k = rope(q, pos), rope(k, pos)
                Kc[l].append(k)
                Vc[l].append(v)
                kk, vv = np.stack(Kc[l]), np.stack(Vc[l])
                att = np.zeros((hq, hd))
                for qh in range(hq):
                    s = kk[:, qh // (hq // hkv)] @ q[qh] / np.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[qh] = (p / p.sum()) @ vv[:, qh // (hq // hkv)]
                h = h + y["attn_output.weight"] @ (att * sig(gate)).ravel()
            xn = rms(h, y["post_attention_norm.weight"])
            gt, up = y["ffn_gate.weight"] @ xn, y["ffn_up.weight"] @ xn
            h = h + y["ffn_down.weight"] @ (gt * sig(gt) * up)
            trace.append(h.copy())
        logits.append(W["out"] @ rms(h, W["onorm"]))
        hidden.append(np.stack(trace))
    return np.stack(logits), np.stack(hidden)


@pytest.mark.parametrize("interval", [2, 3])
def test_qwen35_oracle_matches_fp64_brute_force(tmp_path, interval):
    p = str(tmp_path / "q35.gguf")
    ribn_amd.synth_qwen35_gguf(p, hidden=256, layers=4, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=300,
                               ssm_groups=2, ssm_heads=4, ssm_state=64, full_attention_interval=interval,
                               rope_dims=32, seed=3 + interval, weight_std=0.05, norm_jitter=0.1)
    cfg, W = _weights(p)
    toks = [3, 77, 5, 120, 9, 64, 200, 1, 42]
    ref_l, ref_h = _fp64_forward(cfg, W, toks)
    o = orc.Qwen35Oracle(p, max_ctx=16)
    got = [o.step(t, want_hidden=True) for t in toks]
    o.close()
    lg = np.stack([g[0] for g in got])
    hd = np.stack([g[1] for g in got])
    assert np.linalg.norm(lg - ref_l) / np.linalg.norm(ref_l) < 1e-5
    for layer in range(hd.shape[1]):
        r = np.linalg.norm(hd[:, layer] - ref_h[:, layer]) / np.linalg.norm(ref_h[:, layer])
        assert r < 1e-5, (layer, r)
