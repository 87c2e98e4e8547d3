"""CPU tests of the library's host side: exported ABI, GGUF writer, quantizers,
and the oracle's composed forward against an FP64 brute force on tiny models."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_ffi as orc
import ribn_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "ribn_rocm.h")).read()
    names = set(re.findall(r"\b(ribn_rocm_[a-z0-9_]+)\s*\(", header))
    assert len(names) >= 19
    lib = ctypes.CDLL(ribn_amd.LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.parametrize("t", [ribn_amd.GGML_Q8_0, ribn_amd.GGML_Q4_K, ribn_amd.GGML_Q6_K])
def test_quantizer_roundtrip_error_bound(t):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    enc = ribn_amd.quantize(t, x)
    be, bb = ribn_amd.BLOCK[t]
    assert enc.size == x.size // be * bb
    y = orc.dequantize(t, enc)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    bound = {8: 0.01, 12: 0.12, 14: 0.03}[t]
    assert rel < bound, rel


def test_synth_gguf_parses_with_the_oracle(tmp_path):
    p = str(tmp_path / "m.gguf")
    ribn_amd.synth_qwen_gguf(p, qwen3=True, hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=64, ffn=512,
                             vocab=300, attn_v_type=ribn_amd.GGML_Q6_K, ffn_down_type=ribn_amd.GGML_Q6_K,
                             output_type=ribn_amd.GGML_Q6_K, seed=5)
    g = orc.Gguf(p)
    assert g.rc == 0
    assert g.str("general.architecture") == "qwen3"
    assert g.u64("qwen3.block_count") == 2 and g.u64("qwen3.attention.head_count_kv") == 2
    t, dims, _, data = g.tensor("blk.1.attn_v.weight")
    assert t == ribn_amd.GGML_Q6_K and dims == [256, 128]
    t, dims, _, data = g.tensor("blk.0.ffn_gate.weight")
    assert t == ribn_amd.GGML_Q4_K and dims == [256, 512]
    w = orc.dequantize(t, data)
    assert abs(w.std() - 0.02) < 0.003 and abs(w.mean()) < 0.002
    t, dims, _, data = g.tensor("output_norm.weight")
    assert t == 0 and np.all(data.view(np.float32) == 1.0)
    g.close()
    # determinism: same seed, same bytes; other seed, other bytes
    p2 = str(tmp_path / "m2.gguf")
    ribn_amd.synth_qwen_gguf(p2, qwen3=True, hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=64, ffn=512,
                             vocab=300, attn_v_type=ribn_amd.GGML_Q6_K, ffn_down_type=ribn_amd.GGML_Q6_K,
                             output_type=ribn_amd.GGML_Q6_K, seed=5, threads=3)
    assert open(p, "rb").read() == open(p2, "rb").read()


def test_loader_rejects_unsupported_architecture(tmp_path):
    p = str(tmp_path / "bad.gguf")
    ribn_amd.synth_qwen_gguf(p, qwen3=True, hidden=256, layers=1, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=64)
    data = bytearray(open(p, "rb").read())
    i = data.find(b"qwen3")
    data[i:i + 5] = b"llama"
    bad = str(tmp_path / "bad2.gguf")
    open(bad, "wb").write(bytes(data))
    with pytest.raises(ribn_amd.RibnError) as e:
        ribn_amd.QwenRocm(bad)
    assert "general.architecture" in e.value.message and e.value.code == -3
    with pytest.raises(ribn_amd.RibnError) as e:
        ribn_amd.QwenRocm(str(tmp_path / "missing.gguf"))
    assert e.value.code == -3


# ---------------------------------------------------------------- FP64 brute force of the composed oracle
def _load_fp64(path):
    g = orc.Gguf(path)
    arch = g.str("general.architecture")
    cfg = {k: g.u64(f"{arch}.{k}") for k in ("embedding_length", "block_count", "attention.head_count",
                                              "attention.head_count_kv", "attention.key_length", "feed_forward_length")}

    def T(name):
        r = g.tensor(name)
        if isinstance(r, int):
            return None
        t, dims, _, data = r
        return orc.dequantize(t, data).astype(np.float64).reshape(list(reversed(dims)))
    W = {"embd": T("token_embd.weight"), "out": T("output.weight"), "onorm": T("output_norm.weight"), "L": []}
    if W["out"] is None:
        W["out"] = W["embd"]
    for l in range(cfg["block_count"]):
        W["L"].append({n: T(f"blk.{l}.{n}") for n in (
            "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
            "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight", "attn_q_norm.weight",
            "attn_k_norm.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias")})
    g.close()
    return cfg, W


def _fp64_forward(cfg, W, tokens, eps=1e-6, base=1e6):
    H, hq, hkv, hd = cfg["embedding_length"], cfg["attention.head_count"], cfg["attention.head_count_kv"], \
        cfg["attention.key_length"]
    grp = hq // hkv
    K = [[] for _ in W["L"]]
    Vc = [[] for _ in W["L"]]
    outs = []

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def rope(x, pos):
        x = x.reshape(-1, hd).copy()
        half = hd // 2
        p = np.arange(half)
        th = pos * base ** (-2.0 * p / hd)
        c, s = np.cos(th), np.sin(th)
        a, b = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half] = a * c - b * s
        x[:, half:] = a * s + b * c
        return x

    for pos, tok in enumerate(tokens):
        h = W["embd"][tok].copy()
        for l, y in enumerate(W["L"]):
            xn = rms(h, y["attn_norm.weight"])
            q, k, v = y["attn_q.weight"] @ xn, y["attn_k.weight"] @ xn, y["attn_v.weight"] @ xn
            if y["attn_q.bias"] is not None:
                q, k, v = q + y["attn_q.bias"], k + y["attn_k.bias"], v + y["attn_v.bias"]
            q, k = q.reshape(hq, hd), k.reshape(hkv, hd)
            if y["attn_q_norm.weight"] is not None:
                q = np.stack([rms(r, y["attn_q_norm.weight"]) for r in q])
                k = np.stack([rms(r, y["attn_k_norm.weight"]) for r in k])
            q, k = rope(q, pos), rope(k, pos)
            K[l].append(k)
            Vc[l].append(v.reshape(hkv, hd))
            kk, vv = np.stack(K[l]), np.stack(Vc[l])   # [t, hkv, hd]
            att = np.zeros((hq, hd))
            for qh in range(hq):
                s = kk[:, qh // grp] @ q[qh] / np.sqrt(hd)
                p = np.exp(s - s.max())
                att[qh] = (p / p.sum()) @ vv[:, qh // grp]
            h = h + y["attn_output.weight"] @ att.ravel()
            xn = rms(h, y["ffn_norm.weight"])
            gt, up = y["ffn_gate.weight"] @ xn, y["ffn_up.weight"] @ xn
            h = h + y["ffn_down.weight"] @ (gt / (1 + np.exp(-gt)) * up)
        outs.append(W["out"] @ rms(h, W["onorm"]))
    return np.stack(outs)


@pytest.mark.parametrize("qwen3,wt", [(True, ribn_amd.GGML_Q4_K), (False, ribn_amd.GGML_Q8_0)])
def test_oracle_forward_matches_fp64_brute_force(tmp_path, qwen3, wt):
    p = str(tmp_path / "tiny.gguf")
    ribn_amd.synth_qwen_gguf(p, qwen3=qwen3, hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=64, ffn=512,
                             vocab=128, weight_type=wt, seed=11, norm_jitter=0.2, weight_std=0.05)
    cfg, W = _load_fp64(p)
    toks = [3, 77, 5, 120, 9, 64]
    ref = _fp64_forward(cfg, W, toks)
    o = orc.QwenOracle(p, max_ctx=16)
    got = np.stack([o.step(t)[0] for t in toks])
    o.close()
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-5, rel


@pytest.mark.parametrize("layers", [1, 2])
def test_oracle_append_kv_equals_full_steps(tmp_path, layers):
    """orc_qwen_append_kv (K/V only, no readout) leaves the oracle in the state full steps do: the logits of
    every later position are bit-identical, and so is the FP64 brute force's agreement."""
    p = str(tmp_path / "kv.gguf")
    ribn_amd.synth_qwen_gguf(p, qwen3=True, hidden=256, layers=layers, q_heads=8, kv_heads=1, head_dim=128,
                             ffn=512, vocab=128, seed=13, norm_jitter=0.2, weight_std=0.05)
    toks = [3, 77, 5, 120, 9, 64, 11, 100, 2]
    for kv_round in (0, 2):
        full = orc.QwenOracle(p, max_ctx=16, kv_round=kv_round)
        part = orc.QwenOracle(p, max_ctx=16, kv_round=kv_round)
        ref = [full.step(t)[0] for t in toks]
        for t in toks[:6]:
            part.append_kv(t)
        got = [part.step(t)[0] for t in toks[6:]]
        full.close()
        part.close()
        for a, b in zip(got, ref[6:]):
            assert np.array_equal(a, b)
    cfg, W = _load_fp64(p)
    fp64 = _fp64_forward(cfg, W, toks)
    assert np.linalg.norm(np.stack(got) - fp64[6:]) / np.linalg.norm(fp64[6:]) < 5e-3   # kv_round 2: bf16 cache


def _gguf_bytes(tensors, arch="qwen3"):
    """A minimal GGUF v3 stream: one metadata key and the given (name, dims, type, offset) tensors."""
    import struct

    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    out = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 1)
    out += s("general.architecture") + struct.pack("<I", 8) + s(arch)
    for name, dims, typ, off in tensors:
        out += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", typ, off)
    out += b"\0" * ((-len(out)) % 32) + b"\0" * 64
    return out


def test_loader_rejects_overflowing_and_duplicate_tensors(tmp_path):
    """Element counts and byte lengths are checked products (TensorInfo::byte_len, crates/gguf/src/lib.rs:
    124-168): dims whose product wraps u64 fail instead of passing the end-of-file check; a repeated tensor
    name is rejected."""
    cases = {
        "wrap": [("w", [1 << 33, 1 << 31], 0, 0)],              # 2^64 elements: wraps to 0
        "bytes": [("w", [1 << 62, 2], 0, 0)],                   # 2^63 elements, 2^65 bytes
        "dup": [("w", [16], 0, 0), ("w", [16], 0, 64)],
    }
    for name, ts in cases.items():
        p = str(tmp_path / f"{name}.gguf")
        open(p, "wb").write(_gguf_bytes(ts))
        with pytest.raises(ribn_amd.RibnError) as e:
            ribn_amd.QwenRocm(p)
        assert e.value.code == -3, (name, e.value.message)
        assert ("overflows" in e.value.message) if name != "dup" else ("duplicate tensor" in e.value.message)


def test_oracle_threads_do_not_change_results(tmp_path):
    """The oracle's multi-threaded matvecs (the all-cores CPU baseline) give bit-identical logits."""
    p = str(tmp_path / "thr.gguf")
    ribn_amd.synth_qwen_gguf(p, qwen3=True, hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=64, ffn=512,
                             vocab=300, seed=17, norm_jitter=0.2, weight_std=0.05)
    toks = [3, 77, 5, 120, 9]
    out = []
    for threads in (1, 7):
        o = orc.QwenOracle(p, max_ctx=16)
        o.set_threads(threads)
        out.append(np.stack([o.step(t)[0] for t in toks]))
        o.close()
    assert np.array_equal(out[0], out[1])
