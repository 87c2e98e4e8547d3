"""Gemma 4 host CPU BF16 decoder restatement (oracle/gemma4.c), pinned by the
reference's own known answers and by invariants (CPU only).

- Operation KATs: the literal cases of crates/gemma4/tests/cpu_ops.rs:21-135 and
  cpu_attention.rs:22-92. They cover single rounding after FP32 accumulation, the
  RMS statistics, per-product rotary rounding with both factor halves, causal and
  sliding masks, and grouped heads.
- Inverse frequencies: against the FP32 bits recorded in the reference fixture
  (tests/golden/gemma4_rotary_inverse_frequency.json, a copy of
  crates/gemma4/tests/fixtures/rotary.json), within the reference test's 4-ULP
  budget (tests/rotary.rs:44-50), and against an FP64 evaluation of the same
  exponent.
- Decoder composition: the reference holds no golden logits for any small model
  (its archived ones need the 14.9 GB E4B package). The composed decoder is pinned
  by an independent numpy forward written from decoder.rs (test_gemma_composition.py,
  bit-identical logits) and, here, by the reference's own invariant: multi-row
  prefill equals serial decode bit for bit, across sliding-window and shared-KV
  boundaries (cpu_prefill.rs:67-147). Rejected chunks leave the continuation
  unchanged (cpu_prefill.rs:149-168).
"""
import json
import os

import numpy as np
import pytest

import gemma_oracle as g4

HERE = os.path.dirname(os.path.abspath(__file__))
L = g4.lib()


def b(x):
    return int(L.g4_bf16(float(x)))


def val(bits):
    return float(g4.load(np.array([bits], np.uint16))[0])


def arr(xs):
    return np.array([b(x) for x in xs], np.uint16)


def test_bf16_rounding_closed_forms():
    assert b(1.0) == 0x3F80 and b(-2.0) == 0xC000 and b(-0.0) == 0x8000
    halfway_even = np.array([0x3F808000], np.uint32).view(np.float32)[0]   # 1 + 2^-8: ties to 0x3f80
    halfway_odd = np.array([0x3F818000], np.uint32).view(np.float32)[0]    # ties to 0x3f82
    assert b(halfway_even) == 0x3F80 and b(halfway_odd) == 0x3F82
    assert b(float("nan")) == 0x7FC0 and b(float("inf")) == 0x7F80
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32)
    assert np.array_equal(g4.bf16(x), np.array([b(v) for v in x[:2000]] + list(g4.bf16(x[2000:])), np.uint16))


def test_linear_rounds_once_after_fp32_accumulation():
    # cpu_ops.rs:21-46
    w = arr([1.0, 2.0, 4.0, 0.5, -1.0, 2.0])
    x = arr([1.0, 1.0, 1.0])
    out = np.zeros(2, np.uint16)
    L.g4_project(g4.ptr(x), 1, 3, g4.ptr(w), 2, g4.ptr(out))
    assert list(out) == [b(7.0), b(1.5)]
    w = arr([0.1, 0.2, 0.3])
    out = np.zeros(1, np.uint16)
    L.g4_project(g4.ptr(x), 1, 3, g4.ptr(w), 1, g4.ptr(out))
    s = np.float32(val(b(0.1))) + np.float32(val(b(0.2)))
    s = np.float32(s + np.float32(val(b(0.3))))
    assert out[0] == b(s)


def test_rms_norm_fp32_statistics_and_direct_scale():
    # cpu_ops.rs:48-56
    scale = arr([1.0, 1.0])
    x = arr([3.0, 4.0])
    out = np.zeros(2, np.uint16)
    L.g4_rms_norm(g4.ptr(x), 1, 2, 1e-6, g4.ptr(scale), g4.ptr(out))
    inv = np.float32(np.float32(12.5) + np.float32(1e-6)) ** np.float32(-0.5)
    assert list(out) == [b(np.float32(3.0) * inv), b(np.float32(4.0) * inv)]
    # scale-free (value) normalization: no learned scale at all
    out2 = np.zeros(2, np.uint16)
    L.g4_rms_norm(g4.ptr(x), 1, 2, 1e-6, None, g4.ptr(out2))
    assert np.array_equal(out, out2)


def rotary(x, cos, sin, width=2):
    out = np.zeros(len(x), np.uint16)
    L.g4_apply_rotary(g4.ptr(x), 1, 1, width, g4.ptr(cos), g4.ptr(sin), g4.ptr(out))
    return list(out)


def test_rotary_rounds_each_product_and_reads_both_halves():
    # cpu_ops.rs:58-90
    assert rotary(np.array([0x8000, b(-2.0)], np.uint16), arr([1.0, 1.0]), arr([0.0, 0.0])) == [0x0000, b(-2.0)]
    expected = [b(2.0 * 1.0 + (-4.0) * 0.0), b(4.0 * 0.5 + 2.0 * 0.25)]
    assert rotary(arr([2.0, 4.0]), arr([1.0, 0.5]), arr([0.0, 0.25])) == expected
    assert rotary(arr([3.0, -4.0]), arr([0.0, 0.0]), arr([1.0, 1.0])) == [b(4.0), b(3.0)]


def e4b_like(head_dim, global_head_dim, theta_local, theta_global):
    return g4.config(vocab=16, hidden=16, intermediate=16, heads=2, kv_heads=1, head_dim=head_dim,
                     global_head_dim=global_head_dim, ple=4, layers=("S", "F"), theta_local=theta_local,
                     theta_global=theta_global)


def test_inverse_frequencies_match_the_reference_fixture_bits():
    import ctypes
    data = json.load(open(os.path.join(HERE, "golden", "gemma4_rotary_inverse_frequency.json")))
    geometries = {"e4b": (256, 512, 1e4, 1e6), "alternate_geometry": (10, 16, 32768.0, 1048576.0)}
    checked = 0
    for case in data["cases"]:
        hd, ghd, tl, tg = geometries[case["name"]]
        c = e4b_like(hd, ghd, tl, tg)
        for layer, kind in ((0, "sliding_attention"), (1, "full_attention")):
            exp = case["kinds"][kind]
            assert exp["head_dim"] == c.head_dim[layer]
            for pair, bits in enumerate(exp["inverse_frequency_bits"]):
                f = ctypes.c_float()
                assert L.g4_inverse_frequency(ctypes.byref(c), layer, pair, ctypes.byref(f)) == 0
                got = int(np.array([f.value], np.float32).view(np.uint32)[0])
                if bits == 0:
                    assert got == 0 and c.proportional[layer] and pair >= c.head_dim[layer] // 8
                    continue
                assert abs(got - bits) <= 4, (case["name"], kind, pair)
                theta = c.theta[layer]
                e = np.float32(np.float32(2 * pair) / np.float32(c.head_dim[layer]))
                exact = float(theta) ** (-float(e))
                assert abs(f.value - exact) / exact <= 3 * np.finfo(np.float32).eps
                checked += 1
            f = ctypes.c_float()
            assert L.g4_inverse_frequency(ctypes.byref(c), layer, c.head_dim[layer] // 2, ctypes.byref(f)) == -1
    assert checked == 128 + 64 + 5 + 2   # every nonzero recorded frequency


def test_factors_duplicate_halves_and_keep_padding_identity():
    # cpu_ops.rs:92-131 on the E4B full-attention geometry
    c = e4b_like(256, 512, 1e4, 1e6)
    width = 512
    pos = np.array([0, 5], np.uint32)
    cos = np.zeros(2 * width, np.uint16)
    sin = np.zeros(2 * width, np.uint16)
    assert L.g4_factors(c, 1, g4.ptr(pos), 2, g4.ptr(cos), g4.ptr(sin)) == 0
    for row in range(2):
        h = width // 2
        assert np.array_equal(cos[row * width:row * width + h], cos[row * width + h:(row + 1) * width])
        assert np.array_equal(sin[row * width:row * width + h], sin[row * width + h:(row + 1) * width])
    assert np.all(cos[:width] == 0x3F80) and np.all(sin[:width] == 0)
    active = width // 4
    assert np.all(cos[width + active:width + width // 2] == 0x3F80)
    assert np.all(sin[width + active:width + width // 2] == 0)
    assert np.any(sin[width:width + active] != 0)


def attn(q, k, v, heads, kv_heads, width, window, q_start=0, with_weights=True):
    seq = len(q) // (heads * width)
    kv = len(k) // (kv_heads * width)
    out = np.zeros(len(q), np.uint16)
    wts = np.zeros(heads * seq * kv, np.uint16) if with_weights else None
    rc = L.g4_attention(g4.ptr(q), seq, g4.ptr(k), g4.ptr(v), kv, heads, kv_heads, width, window, q_start, 0,
                        g4.ptr(out), g4.ptr(wts) if with_weights else None)
    assert rc == 0
    return list(out), wts


def test_attention_causal_and_sliding_masks():
    # cpu_attention.rs:22-62
    q = arr([1.0] * 4)
    k = arr([0.0] * 4)
    v = arr([1.0, 2.0, 3.0, 4.0])
    out, w = attn(q, k, v, 1, 1, 1, 0)
    assert out == [b(1.0), b(1.5), b(2.0), b(2.5)]
    for p in range(4):
        for key in range(4):
            assert w[p * 4 + key] == (b(np.float32(1.0) / np.float32(p + 1)) if key <= p else 0)
    out, w = attn(q, k, v, 1, 1, 1, 2)
    assert out == [b(1.0), b(1.5), b(2.5), b(3.5)]
    assert w[8] == 0 and w[9] == b(0.5) and w[10] == b(0.5)


def test_attention_grouped_heads_and_softmax():
    # cpu_attention.rs:64-92
    out, _ = attn(arr([1.0] * 4), arr([0.0] * 2), arr([10.0, 20.0]), 4, 2, 1, 0, with_weights=False)
    assert out == [b(10.0), b(10.0), b(20.0), b(20.0)]
    out, _ = attn(arr([1.0]), arr([1.0, 0.0]), arr([1.0, 2.0]), 1, 1, 1, 0, q_start=1, with_weights=False)
    e1, e0 = np.exp(np.float32(1.0)), np.exp(np.float32(0.0))
    total = np.float32(e1 + e0)
    w1, w0 = val(b(e1 / total)), val(b(e0 / total))
    assert out == [b(np.float32(np.float32(w1) * 1.0) + np.float32(np.float32(w0) * 2.0))]


def test_gelu_softcap_and_ple_combine_closed_forms():
    x = arr([0.0, 8.0, -8.0])
    out = np.zeros(3, np.uint16)
    L.g4_gelu_tanh(g4.ptr(x), 3, g4.ptr(out))
    assert list(out) == [b(0.0), b(8.0), b(-0.0)]
    x = arr([30.0, 0.0, -60.0])
    L.g4_softcap(g4.ptr(x), 3, 30.0, g4.ptr(out))
    t1 = val(b(np.tanh(np.float32(1.0))))
    assert out[0] == b(np.float32(t1) * np.float32(30.0)) and out[1] == b(0.0)
    assert out[2] == b(np.float32(val(b(np.tanh(np.float32(-2.0))))) * np.float32(30.0))
    a, c = arr([1.0]), arr([1.0])
    o = np.zeros(1, np.uint16)
    L.g4_ple_combine(g4.ptr(a), g4.ptr(c), 1, g4.ptr(o))
    assert o[0] == b(np.float32(2.0) * np.float32(0.70710677))


def small_model(window, shared):
    # small enough for serial checks, with a sliding window shorter than the
    # sequences and shared-KV tail layers (cpu_prefill.rs:12-53 uses a 7-wide model)
    c = g4.config(vocab=61, hidden=24, intermediate=40, heads=4, kv_heads=2, head_dim=8, global_head_dim=16, ple=6,
                  context=40, window=window, layers=("S", "F", "S", "S", "F"), shared=shared)
    w, keep = g4.synth_weights(c, seed=3, std=0.3)
    return c, w, keep


@pytest.mark.parametrize("window,shared", [(3, 0), (5, 2), (64, 2)])
def test_multirow_prefill_matches_serial_decode(window, shared):
    c, w, keep = small_model(window, shared)
    rng = np.random.default_rng(window)
    prompt = rng.integers(0, c.vocab, 13).tolist()
    serial = g4.Gemma4Oracle(c, w)
    serial_logits = [serial.prefill([t]) for t in prompt]
    assert serial.position == len(prompt)
    for chunks in ([13], [6, 7], [1, 4, 8], [5, 5, 3]):
        d = g4.Gemma4Oracle(c, w)
        pos = 0
        for n in chunks:
            lg = d.prefill(prompt[pos:pos + n])
            pos += n
            assert np.array_equal(lg, serial_logits[pos - 1]), (chunks, pos)
        # a state-only prefill followed by decode gives the same continuation
        s = g4.Gemma4Oracle(c, w)
        s.advance_prefill(prompt[:-1])
        assert np.array_equal(s.decode(prompt[-1]), serial_logits[-1])
        d.close()
        s.close()
    assert len({tuple(x) for x in serial_logits}) > 1


def test_rejected_chunks_preserve_the_continuation():
    c, w, keep = small_model(5, 2)
    a = g4.Gemma4Oracle(c, w)
    ref = a.prefill([1, 2, 3])
    nxt = a.decode(4)
    d = g4.Gemma4Oracle(c, w)
    assert np.array_equal(d.prefill([1, 2, 3]), ref)
    for bad in ([], [c.vocab], [1] * 40):
        with pytest.raises(ValueError):
            d.prefill(bad)
        assert d.position == 3
    assert np.array_equal(d.decode(4), nxt)


def test_configs0_tiny_gemma_greedy_is_deterministic():
    """64-token prompt, 32 greedy tokens; the first tokens must not collapse."""
    c = g4.config()
    w, keep = g4.synth_weights(c, seed=0)
    prompt = np.random.default_rng(0).integers(0, 32000, 64).tolist()
    a = g4.Gemma4Oracle(c, w).generate(prompt, 8)
    b2 = g4.Gemma4Oracle(c, w).generate(prompt, 8)
    assert a == b2 and all(0 <= t < 32000 for t in a)


def test_threaded_projection_is_bit_identical():
    """The all-cores CPU baseline splits g4_project's outputs across threads; every logit stays identical."""
    c = g4.config(vocab=512, hidden=128, intermediate=256, heads=4, kv_heads=2, head_dim=32, global_head_dim=32,
                  ple=32, layers=("S", "F"))
    w, keep = g4.synth_weights(c, seed=3)
    prompt = [5, 9, 100, 7, 300]
    ref = g4.Gemma4Oracle(c, w).prefill(prompt)
    g4.set_threads(5)
    try:
        got = g4.Gemma4Oracle(c, w).prefill(prompt)
    finally:
        g4.set_threads(1)
    assert np.array_equal(got, ref)
