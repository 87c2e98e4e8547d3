"""GPU parity of the whole token loop and the executor contract.

Bars (north star): per-layer hidden states and logits within rel-L2 2e-3 of the
FP32 oracle (binary16 KV cache on the device, the reference's cache type), and identical greedy tokens for 64
steps on seeded synthetic models. A greedy mismatch is excused only as a
near-tie: the oracle's own logits must put the device's pick within the
measured logit error of the oracle's pick; the run then stops comparing
because the two continuations legitimately diverge.
"""
import os
import sys
import zlib

import numpy as np
import pytest

import oracle_ffi as orc
import ribn_amd
from ribn_amd import BatchItem, STEP_DECODE, STEP_PREFILL, ADMIT_READY, ADMIT_REJECTED, ADMIT_DEFERRED

pytestmark = pytest.mark.gpu
REL_TOL = 2e-3

Q4KM = dict(weight_type=ribn_amd.GGML_Q4_K, attn_v_type=ribn_amd.GGML_Q6_K, ffn_down_type=ribn_amd.GGML_Q6_K,
            output_type=ribn_amd.GGML_Q6_K)
MODELS = {
    # name: (synth kwargs)
    "qwen3_q4km_hd64": dict(qwen3=True, hidden=256, layers=3, q_heads=4, kv_heads=2, head_dim=64, ffn=768,
                            vocab=512, **Q4KM),
    "qwen3_q4km_hd128_g4": dict(qwen3=True, hidden=512, layers=2, q_heads=8, kv_heads=2, head_dim=128, ffn=1024,
                                vocab=1024, **Q4KM),
    "qwen2_q8_0_g7": dict(qwen3=False, hidden=448 + 64, layers=2, q_heads=14, kv_heads=2, head_dim=64, ffn=1024,
                          vocab=640, weight_type=ribn_amd.GGML_Q8_0),
    # Qwen2.5-0.5B geometry (hidden 896 = 28 Q8_0 blocks, 14/2 heads x 64,
    # FFN 4864, q/k/v bias, all Q8_0), at 2 layers and a reduced vocabulary
    "qwen2_0p5b_shape_q8_0": dict(qwen3=False, hidden=896, layers=2, q_heads=14, kv_heads=2, head_dim=64,
                                  ffn=4864, vocab=1024, weight_type=ribn_amd.GGML_Q8_0),
    "qwen3_g8_tied": dict(qwen3=True, hidden=512, layers=1, q_heads=8, kv_heads=1, head_dim=64, ffn=512,
                          vocab=256, tied_output=True, **Q4KM),
}


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def model_paths(tmp_path_factory):
    d = tmp_path_factory.mktemp("models")
    out = {}
    for name, kw in MODELS.items():
        p = str(d / f"{name}.gguf")
        ribn_amd.synth_qwen_gguf(p, seed=zlib.crc32(name.encode()) % 1000, norm_jitter=0.15, weight_std=0.05, **kw)
        out[name] = p
    return out


# KV mode -> (oracle KV rounding, rel-L2 bound). The default binary16 cache (the
# reference's CUDA cache type) meets 2e-3 against the unrounded FP32 oracle. The
# optional bfloat16 cache cannot: its rounding alone moves hidden states by
# 2.2e-3..3.9e-3 rel-L2 on these models (FP64 simulation), and emulating it in
# the oracle does not help because tiny input differences flip roundings; it is
# held to 6e-3 against the BF16-rounding oracle.
KV_MODES = {"f16": (orc.QwenOracle.KV_F32, REL_TOL), "bf16": (orc.QwenOracle.KV_BF16, 6e-3)}


def _oracle_trace(path, tokens, ctx, hidden=False, kv_round=0):
    o = orc.QwenOracle(path, max_ctx=ctx, kv_round=kv_round)
    ls, hs = [], []
    for t in tokens:
        l, h = o.step(t, want_hidden=hidden)
        ls.append(l)
        hs.append(h)
    o.close()
    return np.stack(ls), (np.stack(hs) if hidden else None)


STEPS = ["persistent", "chain"]
# (model, kv) configurations without a compiled persistent step kernel: they run the launch chain
NO_STEP_KERNEL = {("qwen3_g8_tied", "bf16")}


def _check_path(m, name, kv, step):
    """The requested step path is the one that runs (persistent kernel when one is compiled)."""
    want = int(step == "persistent" and (name, kv) not in NO_STEP_KERNEL)
    assert m.info.persistent_step == want, (name, kv, step, m.info.persistent_step)
    if want:
        assert m.info.step_workgroups >= 256


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("step", STEPS)
@pytest.mark.parametrize("kv", list(KV_MODES))
@pytest.mark.parametrize("name", list(MODELS))
def test_trace_hidden_and_logits(model_paths, name, kv, step):
    path = model_paths[name]
    kv_round, tol = KV_MODES[kv]
    rng = np.random.default_rng(1)
    info_v = MODELS[name]["vocab"]
    tokens = rng.integers(0, info_v, 40).tolist()
    say(f"trace {name} kv={kv} step={step}")
    with ribn_amd.QwenRocm(path, context_tokens=128, max_sequences=2, kv=kv, step=step) as m:
        assert m.info.kv_f16 == int(kv == "f16")
        _check_path(m, name, kv, step)
        am, lg, hd = m.trace(tokens, logits=True, hidden=True)
    ref_l, ref_h = _oracle_trace(path, tokens, 128, hidden=True, kv_round=kv_round)
    for layer in range(ref_h.shape[1]):
        r = _rel(hd[:, layer], ref_h[:, layer])
        assert r <= tol, f"layer {layer} hidden rel-L2 {r:.2e}"
    r = _rel(lg, ref_l)
    say(f"  logits rel-L2 {r:.2e}")
    assert r <= tol
    err = np.abs(lg - ref_l).max()
    for p in range(len(tokens)):
        o_pick = int(orc.argmax(ref_l[p]))
        if am[p] != o_pick:
            margin = ref_l[p][o_pick] - ref_l[p][am[p]]
            assert margin <= 4 * err, f"pos {p}: argmax {am[p]} vs {o_pick}, margin {margin:.3e}"
        assert am[p] == orc.argmax(lg[p])   # the device argmax is the argmax of the device logits


@pytest.mark.parametrize("gemm", ["dequant", "resident"])
@pytest.mark.parametrize("chunk", [0, 16])
@pytest.mark.parametrize("kv", list(KV_MODES))
@pytest.mark.parametrize("name", list(MODELS))
def test_chunked_prefill_hidden_and_logits(model_paths, name, kv, chunk, gemm):
    """Chunked prefill (MFMA GEMMs, causal chunk attention) against the FP32 oracle: hidden rows after every
    layer and the logits of every row; chunk 16 splits the 40 rows over three chunks, so later chunks attend
    to cache entries written by earlier ones. gemm "resident": the same projections as hipBLASLt GEMMs on
    binary16 weight copies made at load."""
    path = model_paths[name]
    kv_round, tol = KV_MODES[kv]
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, MODELS[name]["vocab"], 40).tolist()
    say(f"prefill trace {name} kv={kv} chunk={chunk}")
    with ribn_amd.QwenRocm(path, context_tokens=128, max_sequences=2, kv=kv, gemm=gemm) as m:
        lg, hd = m.prefill_trace(tokens, chunk=chunk, logits=True, hidden=True)
    ref_l, ref_h = _oracle_trace(path, tokens, 128, hidden=True, kv_round=kv_round)
    for layer in range(ref_h.shape[1]):
        r = _rel(hd[:, layer], ref_h[:, layer])
        assert r <= tol, f"layer {layer} hidden rel-L2 {r:.2e}"
    r = _rel(lg, ref_l)
    say(f"  logits rel-L2 {r:.2e}")
    assert r <= tol


@pytest.mark.parametrize("step", STEPS)
@pytest.mark.parametrize("kv", list(KV_MODES))
def test_long_context_split_k(model_paths, kv, step):
    """700 positions: 8 splits of 96 over 44 pages, log-sum-exp merge across workgroups."""
    path = model_paths["qwen3_q4km_hd128_g4"]
    kv_round, tol = KV_MODES[kv]
    rng = np.random.default_rng(2)
    tokens = rng.integers(0, 1024, 700).tolist()
    say(f"trace 700 tokens kv={kv} step={step}")
    with ribn_amd.QwenRocm(path, context_tokens=1024, max_sequences=1, kv=kv, step=step) as m:
        _check_path(m, "qwen3_q4km_hd128_g4", kv, step)
        _, lg, _ = m.trace(tokens, logits=True)
    ref_l, _ = _oracle_trace(path, tokens, 1024, kv_round=kv_round)
    for lo in (0, 100, 300, 600):
        r = _rel(lg[lo:lo + 100], ref_l[lo:lo + 100])
        assert r <= tol, (lo, r)


@pytest.mark.parametrize("kv", list(KV_MODES))
def test_split_policy_regimes(tmp_path, kv):
    """8400 positions through every regime of the split policy: one workgroup up to 128 positions, then
    splits of about 128 (up to 2048), 256 (up to 8192) and 1024 positions (flash-decoding blocks across a
    whole 1024-position split); logits at each boundary and at the end against the FP32 oracle. One layer,
    one KV head, Q8_0, so the oracle's quadratic attention stays within seconds."""
    path = str(tmp_path / "long.gguf")
    ribn_amd.synth_qwen_gguf(path, qwen3=False, hidden=128, layers=1, q_heads=2, kv_heads=1, head_dim=64, ffn=256,
                             vocab=256, weight_type=ribn_amd.GGML_Q8_0, seed=7, norm_jitter=0.15, weight_std=0.05)
    kv_round, tol = KV_MODES[kv]
    n = 8400
    tokens = np.random.default_rng(5).integers(0, 256, n).tolist()
    say(f"trace {n} tokens kv={kv}")
    with ribn_amd.QwenRocm(path, context_tokens=n + 16, max_sequences=1, kv=kv) as m:
        _, lg, _ = m.trace(tokens, logits=True)
    ref_l, _ = _oracle_trace(path, tokens, n + 16, kv_round=kv_round)
    for lo, hi in ((0, 160), (2030, 2070), (8180, 8210), (n - 40, n)):
        r = _rel(lg[lo:hi], ref_l[lo:hi])
        say(f"  positions {lo}..{hi}: rel-L2 {r:.2e}")
        assert r <= tol, (lo, r)


def _oracle_greedy(path, prompt, n_new, ctx, kv_round=0):
    o = orc.QwenOracle(path, max_ctx=ctx, kv_round=kv_round)
    out, logits = [], []
    l = None
    for t in prompt:
        l, _ = o.step(t)
    for _ in range(n_new):
        tok = orc.argmax(l)
        out.append(tok)
        logits.append(l)
        l, _ = o.step(tok)
    o.close()
    return out, logits


@pytest.mark.parametrize("step", STEPS)
@pytest.mark.parametrize("kv", list(KV_MODES))
@pytest.mark.parametrize("name", ["qwen3_q4km_hd64", "qwen2_q8_0_g7", "qwen2_0p5b_shape_q8_0"])
def test_greedy_64_tokens(model_paths, name, kv, step):
    path = model_paths[name]
    kv_round, tol = KV_MODES[kv]
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, MODELS[name]["vocab"], 16).tolist()
    say(f"greedy {name} kv={kv} step={step}")
    with ribn_amd.QwenRocm(path, context_tokens=128, max_sequences=1, kv=kv, step=step) as m:
        _check_path(m, name, kv, step)
        toks, timing = m.generate(prompt, 64)
        toks2, _ = m.generate(prompt, 64)
        _, lg, _ = m.trace(prompt + toks.tolist()[:-1], logits=True)
    assert np.array_equal(toks, toks2), "repeated runs are not deterministic"
    ref, ref_logits = _oracle_greedy(path, prompt, 64, 128, kv_round)
    err = np.abs(lg[len(prompt) - 1:] - np.stack(ref_logits)[: lg.shape[0] - len(prompt) + 1]).max()
    for i, (a, b) in enumerate(zip(toks.tolist(), ref)):
        if a != b:
            l = ref_logits[i]
            margin = l[b] - l[a]
            assert margin <= 4 * err, f"step {i}: {a} vs {b}, oracle margin {margin:.3e} > 4*err {err:.3e}"
            say(f"  near-tie at step {i} (margin {margin:.2e}); stop comparing")
            break
    assert timing.decode_tokens == 63


def test_bf16_kv_against_fp32_oracle(model_paths):
    """The optional BF16 cache against the unrounded FP32 oracle: documented looser bound."""
    path = model_paths["qwen3_q4km_hd64"]
    tokens = np.random.default_rng(5).integers(0, 512, 40).tolist()
    with ribn_amd.QwenRocm(path, context_tokens=128, max_sequences=1, kv="bf16") as m:
        _, lg, hd = m.trace(tokens, logits=True, hidden=True)
    ref_l, ref_h = _oracle_trace(path, tokens, 128, hidden=True)
    worst = max(_rel(hd[:, l], ref_h[:, l]) for l in range(ref_h.shape[1]))
    say(f"  bf16 KV vs fp32 oracle: worst hidden rel-L2 {worst:.2e}, logits {_rel(lg, ref_l):.2e}")
    assert worst <= 6e-3 and _rel(lg, ref_l) <= 6e-3


# ---------------------------------------------------------------- executor contract
def _run_engine(m, prompts, max_out, chunk=5):
    """A minimal Engine (runtime/src/engine/scheduling.rs:6-83): decode rows first, then prefill chunks."""
    seqs = {}
    for i, p in enumerate(prompts):
        a = m.admit(100 + i, i + 1, p, max_out)
        assert a.kind == ADMIT_READY, a
        seqs[i + 1] = {"prompt": p, "prefix": 0, "out": []}
    while any(len(s["out"]) < max_out for s in seqs.values()):
        batch = []
        for sid, s in seqs.items():
            if len(s["out"]) >= max_out:
                continue
            if s["prefix"] >= len(s["prompt"]):
                batch.append(BatchItem(sid, STEP_DECODE, s["prefix"], 1, 1))
        for sid, s in seqs.items():
            if s["prefix"] < len(s["prompt"]):
                n = min(chunk, len(s["prompt"]) - s["prefix"])
                end = s["prefix"] + n
                batch.append(BatchItem(sid, STEP_PREFILL, s["prefix"], n, int(end == len(s["prompt"]))))
        m.prepare(batch)
        sub = m.submit(batch)
        res = None
        while res is None:
            res = m.poll(sub)
        assert [c.sequence for c in res] == [b.sequence for b in batch]
        for b, c in zip(batch, res):
            assert c.prefix == b.prefix + b.token_budget
            assert len(c.tokens) == b.output_budget
            seqs[c.sequence]["prefix"] = c.prefix
            seqs[c.sequence]["out"].extend(c.tokens)
    for sid in seqs:
        m.release(sid)
        m.release(sid)   # idempotent
    return [seqs[i + 1]["out"] for i in range(len(prompts))]


def _near_tie_match(name, got, ref, ref_logits):
    """Greedy streams agree, or diverge only where the oracle's top-2 margin is a near tie; the
    comparison stops at a divergence (the continuations differ from there on)."""
    for i, (a, b) in enumerate(zip(got, ref)):
        if a != b:
            l = ref_logits[i]
            margin = l[b] - l[a]
            assert margin <= 2e-3 * abs(l[b]) + 1e-3, f"{name} step {i}: {a} vs {b}, oracle margin {margin:.3e}"
            say(f"  {name}: near-tie at step {i} (margin {margin:.2e}); stop comparing")
            return


def test_executor_matches_generate(model_paths):
    """The executor's rows (chunked prefill, then batched decode of the three sequences through the MFMA
    GEMMs) against batch-1 generate and the oracle."""
    path = model_paths["qwen3_q4km_hd64"]
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, 512, n).tolist() for n in (7, 12, 3)]
    say("executor")
    with ribn_amd.QwenRocm(path, context_tokens=64, max_sequences=3, max_batch_tokens=64) as m:
        outs = _run_engine(m, prompts, 6)
        for p, o in zip(prompts, outs):
            g, _ = m.generate(p, 6)
            ref, ref_logits = _oracle_greedy(path, p, 6, 64, KV_MODES["f16"][0])
            _near_tie_match("generate", g.tolist(), ref, ref_logits)
            _near_tie_match("executor", o, ref, ref_logits)
        m.synchronize()


@pytest.mark.parametrize("gemm", ["dequant", "resident"])
@pytest.mark.parametrize("name", ["qwen3_q4km_hd128_g4", "qwen2_q8_0_g7", "qwen3_g8_tied"])
def test_batched_decode_rows_match_oracle(model_paths, name, gemm):
    """Five sequences decoding together: every batch's decode rows run as one batched step (per-row
    positions and page tables, split-K attention per row, GEMM head, per-row argmax)."""
    path = model_paths[name]
    rng = np.random.default_rng(6)
    prompts = [rng.integers(0, MODELS[name]["vocab"], n).tolist() for n in (5, 17, 9, 33, 2)]
    say(f"batched decode {name}")
    with ribn_amd.QwenRocm(path, context_tokens=64, max_sequences=5, max_batch_tokens=64, gemm=gemm) as m:
        outs = _run_engine(m, prompts, 12)
    for p, o in zip(prompts, outs):
        ref, ref_logits = _oracle_greedy(path, p, 12, 64, KV_MODES["f16"][0])
        _near_tie_match(name, o, ref, ref_logits)


def test_executor_contract_errors(model_paths):
    path = model_paths["qwen3_q4km_hd64"]
    with ribn_amd.QwenRocm(path, context_tokens=32, max_sequences=1, max_batch_tokens=16) as m:
        assert m.admit(1, 1, [], 4).kind == ADMIT_REJECTED
        assert m.admit(1, 1, [1, 2], 0).kind == ADMIT_REJECTED
        assert m.admit(1, 1, [1, 2], 40).kind == ADMIT_REJECTED            # exceeds context
        assert m.admit(1, 1, [600], 4).kind == ADMIT_REJECTED              # token id >= vocab
        assert m.admit(1, 1, [1], 4, stop_tokens=[9999]).kind == ADMIT_REJECTED
        assert m.admit(1, 1, [1], 4, temperature=0.7).kind == ADMIT_REJECTED
        assert m.admit(1, 1, [1, 2, 3], 4).kind == ADMIT_READY
        with pytest.raises(ribn_amd.RibnError):
            m.admit(2, 1, [1], 1)                                         # duplicate sequence
        assert m.admit(3, 2, [1], 1).kind == ADMIT_DEFERRED                 # no free sequence slot
        with pytest.raises(ribn_amd.RibnError):
            m.prepare([BatchItem(1, STEP_PREFILL, 1, 2, 1)])               # prefix mismatch
        with pytest.raises(ribn_amd.RibnError):
            m.prepare([BatchItem(1, STEP_PREFILL, 0, 2, 1)])               # output budget before the end
        with pytest.raises(ribn_amd.RibnError):
            m.prepare([BatchItem(1, STEP_DECODE, 0, 1, 1)])                # decode before the prompt ends
        with pytest.raises(ribn_amd.RibnError):
            m.prepare([BatchItem(1, STEP_PREFILL, 0, 20, 0)])              # beyond max_batch_tokens
        ok = [BatchItem(1, STEP_PREFILL, 0, 3, 1)]
        m.prepare(ok)
        with pytest.raises(ribn_amd.RibnError):
            m.prepare(ok)                                                  # one outstanding preparation
        m.abandon_preparation()
        m.abandon_preparation()                                            # idempotent
        with pytest.raises(ribn_amd.RibnError):
            m.submit(ok)                                                   # not prepared
        m.prepare(ok)
        with pytest.raises(ribn_amd.RibnError):
            m.submit([BatchItem(1, STEP_PREFILL, 0, 2, 0)])                # differs from preparation
        sid = m.submit(ok)
        with pytest.raises(ribn_amd.RibnError):
            m.poll(sid + 1)
        res = None
        while res is None:
            res = m.poll(sid)
        assert res[0].prefix == 3 and len(res[0].tokens) == 1
        m.release(1)
        assert m.admit(3, 2, [1], 1).kind == ADMIT_READY                    # capacity returned
        m.release(2)
        m.release(77)                                                      # unknown: Ok
