"""The oracle's integer-dot mode (orc_quantize_q8_1, orc_gemv_q8_1, orc_qwen_set_gemv_mode): the reference's
experimental GemvMode::IntegerDot (crates/nvidia/src/decode.rs:298-312), lossy by design.

Pins:
- the Q8_1 packer against the reference's known-answer words (crates/nvidia/tests/cuda_activation.rs:8-44),
  against numpy's IEEE binary16 conversion for the header, and the rounding bound |x - d q| <= d/2;
- the integer-dot matvec against the reference's host fixtures and their binary64 expectations, computed
  from the fixture quants (q4_q8_1.rs, q6_q8_1.rs, q8_0_q8_1.rs): exact on dyadic inputs, within the packing
  error bound of the float product on lossy ones;
- the batched form (members, batch-major) equals the single-input form row by row;
- the composed decode in integer-dot mode stays within a stated distance of the float decode.
"""
import numpy as np
import pytest

import intdot_fixtures as fx
import oracle_ffi as orc
import ribn_amd

TYPES = [12, 14, 8]


def test_q8_1_known_answer_words():
    """cuda_activation.rs:8-44: five blocks, the first all zero, the others scaled copies of one pattern."""
    x = np.zeros(160, np.float32)
    for b, s in zip(range(1, 5), [1.0, 0.5, 2.0, 0.25]):
        for i, v in zip([0, 1, 2, 3, 4, 5, 31], [127, -127, 0.5, -0.5, 1.5, -1.5, 2.0]):
            x[b * 32 + i] = v * s
    w = orc.quantize_q8_1(x)
    assert list(w[:9]) == [0] * 9
    for b, header in zip(range(1, 5), [0x40003C00, 0x3C003800, 0x44004000, 0x38003400]):
        words = w[b * 9:(b + 1) * 9]
        assert words[0] == header
        assert words[1] == 0xFF01817F
        assert words[2] == 0x0000FE02
        assert list(words[3:8]) == [0] * 5
        assert words[8] == 0x02000000


def test_q8_1_rejects_bad_lengths():
    for n in (0, 31, 33):
        with pytest.raises(ValueError):
            orc.quantize_q8_1(np.zeros(n, np.float32))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q8_1_rounding_bounds_and_half_header(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(32 * 64) * rng.choice([1e-3, 1.0, 30.0], 32 * 64)).astype(np.float32)
    x[5 * 32:6 * 32] = 0.0
    scale, ssum, q = fx.unpack(orc.quantize_q8_1(x))
    xb = x.reshape(-1, 32)
    d32 = (np.abs(xb).max(axis=1) / np.float32(127.0)).astype(np.float32)
    # header: binary16 round-to-nearest-even of d and of the sum (numpy's conversion as the independent check)
    assert np.array_equal(scale, d32.astype(np.float16).astype(np.float64))
    exact = xb.astype(np.float64).sum(axis=1)
    tol = np.abs(exact) * 2.0 ** -11 + np.abs(xb).sum(axis=1) * 32 * 2.0 ** -24 + 1e-30
    assert np.all(np.abs(ssum - exact) <= tol)
    # q = round(x / d), |q| <= 127, all-zero block packs to zeros
    assert np.all(np.abs(q) <= 127)
    err = np.abs(xb.astype(np.float64) - d32[:, None].astype(np.float64) * q)
    assert np.all(err <= d32[:, None] * (0.5 + 1e-5) + 1e-30)
    assert np.all(q[5] == 0) and scale[5] == 0.0


@pytest.mark.parametrize("t", TYPES)
def test_fixture_metadata_matches_dequantize(t):
    """The fixture's encoded bytes decode (orc_dequantize_block, pinned by the GGUF KATs) to the values its
    generator intends, so the expectations below describe these bytes."""
    for b in fx.BLOCKS[t]():
        got = orc.dequantize_block(t, bytes(b["enc"])).astype(np.float64)
        if t == 12:
            g = np.arange(256) // 32
            want = b["d"] * np.array(b["scales"])[g] * b["quants"] - b["dmin"] * np.array(b["minima"])[g]
        elif t == 14:
            want = b["d"] * np.array(b["scales"])[np.arange(256) // 16] * b["quants"]
        else:
            want = b["d"] * b["quants"]
        assert np.array_equal(got, want)


@pytest.mark.parametrize("t", TYPES)
def test_exact_activations_pack_without_loss(t):
    x = fx.activations(True)
    packed = orc.quantize_q8_1(x)
    y = orc.gemv_q8_1(t, fx.encoded(t), fx.ROWS, fx.INPUTS, packed)[0]
    for r, (po, fo, bound, mag) in enumerate(fx.expected(t, x, packed)):
        assert bound == 0.0
        assert po == fo
        assert abs(float(y[r]) - po) <= abs(po) * 2.0 ** -24 + 1e-12, (r, y[r], po)


@pytest.mark.parametrize("t", TYPES)
def test_lossy_activations_within_packing_bound(t):
    x = fx.activations(False)
    packed = orc.quantize_q8_1(x)
    y = orc.gemv_q8_1(t, fx.encoded(t), fx.ROWS, fx.INPUTS, packed)[0]
    differs = False
    for r, (po, fo, bound, mag) in enumerate(fx.expected(t, x, packed)):
        assert bound > 0.0
        assert abs(float(y[r]) - po) <= abs(po) * 2.0 ** -24 + 1e-9, (r, y[r], po)
        assert abs(float(y[r]) - fo) <= bound + mag * 2.0 ** -23 * 32 + 1e-5
        differs |= abs(po - fo) > 1e-4
    assert differs


@pytest.mark.parametrize("t", TYPES)
def test_batched_members_equal_single(t):
    rng = np.random.default_rng(9)
    k, rows = 512, 24
    w = rng.standard_normal((rows, k)).astype(np.float32) * 0.05
    blocks = np.frombuffer(b"".join(ribn_amd.quantize(t, w[r]) for r in range(rows)), np.uint8)
    xs = rng.standard_normal((3, k)).astype(np.float32)
    packed = np.concatenate([orc.quantize_q8_1(x) for x in xs])
    yb = orc.gemv_q8_1(t, blocks, rows, k, packed, members=3, threads=4)
    for m in range(3):
        y1 = orc.gemv_q8_1(t, blocks, rows, k, orc.quantize_q8_1(xs[m]))[0]
        assert np.array_equal(yb[m], y1)
        # and the lossy result is close to the float matvec
        ref = orc.gemv(t, blocks, rows, k, xs[m])
        assert np.linalg.norm(y1 - ref) <= 0.02 * np.linalg.norm(ref)


def test_qwen_int_dot_mode_stays_near_float(tmp_path):
    """Stated bound of the lossy mode on a 4-layer Qwen3 model (Q4_K, Q6_K V/down/output): the integer-dot
    logits stay within rel-L2 0.08 of the float decode over 24 steps (measured 0.041: Q8_1 keeps about
    2^-8 of each block's maximum per activation), with a positive distance (the mode is active)."""
    path = str(tmp_path / "m.gguf")
    ribn_amd.synth_qwen_gguf(path, hidden=256, layers=4, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=512,
                             attn_v_type=ribn_amd.GGML_Q6_K, ffn_down_type=ribn_amd.GGML_Q6_K,
                             output_type=ribn_amd.GGML_Q6_K, weight_std=0.05, norm_jitter=0.1, seed=3)
    toks = np.random.default_rng(4).integers(0, 512, 24).tolist()
    runs = []
    for mode in (orc.QwenOracle.GEMV_FLOAT, orc.QwenOracle.GEMV_INT_DOT):
        o = orc.QwenOracle(path, max_ctx=64)
        o.set_gemv_mode(mode)
        runs.append(np.stack([o.step(t)[0] for t in toks]))
        o.close()
    f, i = runs
    rel = np.linalg.norm(i - f) / np.linalg.norm(f)
    assert 1e-5 < rel <= 0.08, rel
