"""The composed Gemma 4 decoder (oracle/gemma4.c, the configs[0] CPU baseline and the anchor of the GPU
GemmaDecode path) against an independent numpy forward written from the reference's Rust source
(tests/gemma_numpy_ref.py; crates/gemma4/src/cpu/decoder.rs:334-626).

- BF16 eager mode (FP32 operations, BF16 rounding at every reference rounding point, sequential FP32
  sums): the logits must be bit-identical, so any wiring difference (PLE pipeline, KV owners of shared
  layers, sliding windows, proportional rotary, soft cap, norm placement) fails.
- FP64 mode (no rounding): the eager decoder differs from exact arithmetic only by BF16 rounding noise;
  bound stated below.
- The configurations exercise every composition feature; mutation checks show each one changes the
  logits, so an identical result is evidence.
"""
import numpy as np
import pytest

import gemma_oracle as g4
from gemma_numpy_ref import Cfg, GemmaNumpy, _as_f32


def _oracle_rows(c, w, tokens, split):
    """Oracle logits after prefill(tokens[:split]) and then decode of each remaining token."""
    d = g4.Gemma4Oracle(c, w)
    rows = [_as_f32(d.prefill(tokens[:split]))]
    for t in tokens[split:]:
        rows.append(_as_f32(d.decode(t)))
    d.close()
    return rows


def test_configs0_logits_bit_identical_to_independent_forward():
    """configs[0] (hidden 512, 4 layers sliding/sliding/sliding/full, PLE 64, vocab 32000): the 64-token
    prompt's logits, every one of 32000 bit-identical; FP64 exact arithmetic within BF16 noise."""
    c = g4.config()
    w, named = g4.synth_weights(c, seed=0)
    prompt = np.random.default_rng(0).integers(0, c.vocab, 64).tolist()
    ref = _oracle_rows(c, w, prompt, 64)[0]
    got, _ = GemmaNumpy(Cfg(c), named, "bf16").forward(prompt)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    exact, _ = GemmaNumpy(Cfg(c), named, "fp64").forward(prompt)
    rel = np.linalg.norm(exact - ref) / np.linalg.norm(exact)
    # 4 layers of BF16 eager rounding (2^-9 relative per rounding, a few dozen rounding points per
    # path) on logits of magnitude ~2: measured 0.13; a wiring mistake moves them by O(1)
    assert rel < 0.25, rel
    assert int(np.argmax(exact)) == int(np.argmax(ref))


def _sharing_config():
    # sliding window 8 < sequence, full layers at head width 64 with quarter-proportional RoPE at 1e6 against
    # sliding layers at width 32 / 1e4, and the last two layers sharing the KV caches of their kind's last owner
    return g4.config(vocab=512, hidden=128, intermediate=256, heads=4, kv_heads=2, head_dim=32, global_head_dim=64,
                     ple=16, context=64, window=8, layers=("S", "F", "S", "S", "F"), shared=2, theta_global=1e6)


@pytest.mark.parametrize("split", [24, 12])
def test_shared_kv_sliding_and_proportional_layers_bit_identical(split):
    """Prefill of the first `split` tokens, then serial decode steps: every step's logits equal the
    independent forward over the same prefix, bit for bit (so the owner caches written in prefill and
    decode are read as the reference's decoder reads them)."""
    c = _sharing_config()
    assert [c.kv_owner[i] for i in range(5)] == [0, 1, 2, 2, 1]
    w, named = g4.synth_weights(c, seed=5, std=0.08)
    tokens = np.random.default_rng(6).integers(0, c.vocab, 24).tolist()
    rows = _oracle_rows(c, w, tokens, split)
    model = GemmaNumpy(Cfg(c), named, "bf16")
    for i, row in enumerate(rows):
        n = split + i
        got, _ = model.forward(tokens[:n])
        assert np.array_equal(got.view(np.uint32), row.view(np.uint32)), f"prefix {n}"


def test_composition_features_are_exercised():
    """Mutation checks: each composition feature the bit-exact tests cover changes the logits when it is
    wired differently, so those tests would fail on such a mistake."""
    c = _sharing_config()
    w, named = g4.synth_weights(c, seed=5, std=0.08)
    tokens = np.random.default_rng(6).integers(0, c.vocab, 24).tolist()
    base, _ = GemmaNumpy(Cfg(c), named, "bf16").forward(tokens)

    def mutated(edit):
        cfg = Cfg(c)
        edit(cfg)
        got, _ = GemmaNumpy(cfg, named, "bf16").forward(tokens)
        return float(np.abs(got - base).max())

    changes = {
        "own KV in every layer": mutated(lambda k: setattr(k, "kv_owner", list(range(5)))),
        "no sliding window": mutated(lambda k: setattr(k, "window", 10 ** 6)),
        "non-proportional full rope": mutated(lambda k: setattr(k, "proportional", [False] * 5)),
        "soft cap 50": mutated(lambda k: setattr(k, "softcap", 50.0)),
    }
    no_ple = dict(named)
    key = g4.PREFIX + "embed_tokens_per_layer.weight"
    no_ple[key] = np.zeros_like(named[key])
    got, _ = GemmaNumpy(Cfg(c), no_ple, "bf16").forward(tokens)
    changes["no per-layer token embedding"] = float(np.abs(got - base).max())
    for name, delta in changes.items():
        assert delta > 1e-3, (name, delta)
