"""CPU tests: pin the oracle against the reference's known answers and closed forms.

Nothing here needs a GPU. Each oracle function is checked against data the
reference's own tests hold (tests/golden/gguf_kats.json, made by
tests/golden/make_kats.py from crates/gguf/src/lib.rs and crates/nvidia/tests/q*_q8_1.rs)
or against mathematics that a plausible slip would violate.
"""
import json
import os
import struct
import tempfile

import numpy as np
import pytest

import oracle_ffi as orc

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "gguf_kats.json")))


def bits(v):
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


# ---------------------------------------------------------------- f16 decode
def test_f16_exhaustive_against_ieee_binary16():
    """f16_to_f32 (lib.rs:539-551) equals IEEE binary16 for all 65536 patterns; NaN is canonical."""
    lib = orc.lib()
    pats = np.arange(65536, dtype=np.uint16)
    ieee = pats.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(p)) for p in pats], dtype=np.float32)
    finite = ~np.isnan(ieee)
    assert np.array_equal(got[finite].view(np.uint32), ieee[finite].view(np.uint32))
    assert np.all(got[~finite].view(np.uint32) == 0x7FC00000)


# ---------------------------------------------------------------- dequant KATs
@pytest.mark.parametrize("kat", GOLD["kats"], ids=lambda k: f"type{k['type']}")
def test_reference_dequant_kats(kat):
    out = orc.dequantize_block(kat["type"], bytes.fromhex(kat["block"]))
    assert isinstance(out, np.ndarray) and out.size == kat["len"]
    for idx, b in kat.get("expect_bits", {}).items():
        assert out.view(np.uint32)[int(idx)] == b
    if "expect_all_bits" in kat:
        assert np.all(out.view(np.uint32) == kat["expect_all_bits"])


def test_reference_dequant_error_cases():
    assert orc.dequantize_block(12, bytes(143)) == -2          # InvalidTensorBlockLength
    assert orc.dequantize_block(22, bytes(82)) == -1           # UnsupportedTensorType(22)


@pytest.mark.parametrize("case", GOLD["byte_lens"], ids=lambda c: f"type{c['type']}-{c['dims']}")
def test_reference_byte_len(case):
    got = orc.byte_len(case["type"], case["dims"])
    if case["bytes"] is None:
        assert got < 0
    else:
        assert got == case["bytes"]


def test_layout_table_spot_values():
    assert orc.layout(8) == (32, 34)
    assert orc.layout(12) == (256, 144)
    assert orc.layout(14) == (256, 210)
    assert orc.layout(0) == (1, 4) and orc.layout(1) == (1, 2)
    assert orc.layout(999) is None


def test_dyadic_builder_identity():
    """Every decoded value equals d*sc*q - dmin*m exactly (q4_q8_1.rs:205-228 pattern)."""
    assert len(GOLD["builders"]) == 15 * 2 + 24
    for b in GOLD["builders"]:
        out = orc.dequantize_block(b["type"], bytes.fromhex(b["block"]))
        np.testing.assert_array_equal(out.astype(np.float64), np.array(b["expect"], dtype=np.float64))


# ---------------------------------------------------------------- GGUF parser
def _push_str(buf, s):
    buf += struct.pack("<Q", len(s)) + s.encode()


def parser_fixture():
    """The parser fixture of lib.rs:1219-1250 as bytes."""
    b = bytearray(struct.pack("<IIQQ", 0x46554747, 3, 1, 3))
    _push_str(b, "general.architecture"); b += struct.pack("<I", 8); _push_str(b, "qwen3")
    _push_str(b, "general.alignment"); b += struct.pack("<II", 4, 32)
    _push_str(b, "test.array"); b += struct.pack("<IIQII", 9, 4, 2, 1, 0)
    _push_str(b, "token_embd.weight"); b += struct.pack("<IQQIQ", 2, 4, 8, 1, 0)
    b += bytes(256)
    return bytes(b)


def _open_bytes(data):
    with tempfile.NamedTemporaryFile(suffix=".gguf", delete=False) as f:
        f.write(data)
        p = f.name
    g = orc.Gguf(p)
    os.unlink(p)
    return g


def test_parser_fixture():
    g = _open_bytes(parser_fixture())
    assert g.rc == 0
    assert orc.lib().orc_gguf_version(g.h) == 3
    assert orc.lib().orc_gguf_tensor_count(g.h) == 1
    assert g.str("general.architecture") == "qwen3"
    assert g.u64("general.alignment") == 32
    t, dims, start, data = g.tensor("token_embd.weight")
    assert t == 1 and dims == [4, 8] and data.size == 64
    g.close()


def test_parser_rejects_bad_magic_version_duplicates():
    bad = bytearray(parser_fixture()); bad[0] = 0
    assert _open_bytes(bytes(bad)).rc == -3
    v2 = bytearray(parser_fixture()); v2[4] = 2
    assert _open_bytes(bytes(v2)).rc == -4
    dup = bytearray(struct.pack("<IIQQ", 0x46554747, 3, 0, 2))
    for _ in range(2):
        _push_str(dup, "general.name"); dup += struct.pack("<I", 8); _push_str(dup, "x")
    assert _open_bytes(bytes(dup)).rc == -6
    trunc = parser_fixture()[:20]
    assert _open_bytes(trunc).rc == -5


# ---------------------------------------------------------------- host equations
def test_rms_norm_closed_form():
    x = np.full(64, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y = orc.rms_norm(x, w, 0.0)
    np.testing.assert_allclose(y, w, rtol=1e-6)       # constant c: x/rms = 1
    y2 = orc.rms_norm(x, w, 9.0)                      # rms^2 + eps = 18
    np.testing.assert_allclose(y2, 3.0 / np.sqrt(18.0) * w, rtol=1e-6)


def test_rope_identity_norm_and_additivity():
    rng = np.random.default_rng(1)
    v = rng.standard_normal(4 * 128).astype(np.float32)
    np.testing.assert_array_equal(orc.rope(v, 4, 128, 128, 0, 1e6), v)   # pos 0 is the identity
    r = orc.rope(v, 4, 128, 128, 37, 1e6)
    half = 64
    for h in range(4):
        a, b = v[h * 128:(h + 1) * 128], r[h * 128:(h + 1) * 128]
        np.testing.assert_allclose(a[:half] ** 2 + a[half:] ** 2, b[:half] ** 2 + b[half:] ** 2, rtol=1e-5, atol=1e-6)
    # rope(pos a) then rope(pos b) == rope(pos a+b) (rotation group), pairs (p, p+half)
    r2 = orc.rope(orc.rope(v, 4, 128, 128, 5, 1e4), 4, 128, 128, 7, 1e4)
    r12 = orc.rope(v, 4, 128, 128, 12, 1e4)
    np.testing.assert_allclose(r2, r12, rtol=1e-4, atol=1e-5)
    # partial rotary: dims >= rot pass through
    rp = orc.rope(v, 4, 128, 64, 9, 1e4)
    for h in range(4):
        np.testing.assert_array_equal(rp[h * 128 + 64:(h + 1) * 128], v[h * 128 + 64:(h + 1) * 128])
    # pair 0 rotates by exactly theta = pos
    x = np.zeros(128, np.float32); x[0] = 1.0
    y = orc.rope(x, 1, 128, 128, 3, 1e6)
    np.testing.assert_allclose([y[0], y[64]], [np.cos(3.0), np.sin(3.0)], rtol=1e-6)


def test_argmax_ties_and_nan():
    l = np.array([1.0, 5.0, np.nan, 5.0, -np.inf], np.float32)
    assert orc.argmax(l) == 1
    assert orc.argmax(np.array([np.nan, np.nan, -1.0], np.float32)) == 2
    assert orc.argmax(np.array([np.nan, np.nan], np.float32)) == 0
    assert orc.argmax(np.array([-3.0, -2.0, -2.0], np.float32)) == 1


def test_gemv_matches_fp64_dot_of_dequantized():
    rng = np.random.default_rng(2)
    for t, k in ((8, 96), (12, 512), (14, 512)):
        rows = 7
        blocks = np.frombuffer(b"".join(bytes.fromhex(b["block"]) for b in GOLD["builders"] if b["type"] == t),
                               dtype=np.uint8)
        be, bb = orc.layout(t)
        need = rows * (k // be) * bb
        reps = -(-need // blocks.size)
        blocks = np.tile(blocks, reps)[:need]
        x = rng.standard_normal(k).astype(np.float32)
        y = orc.gemv(t, blocks, rows, k, x)
        w = orc.dequantize(t, blocks).reshape(rows, k).astype(np.float64)
        ref = w @ x.astype(np.float64)
        np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
        assert np.array_equal(orc.gemv(t, blocks, rows, k, x, threads=3), y)   # threads do not change rows


def test_kv_rounding_helpers():
    """orc_round_f16 vs numpy binary16 casts; orc_round_bf16 vs torch bfloat16 casts (both RNE)."""
    import torch
    lib = orc.lib()
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.standard_normal(20000) * s for s in (1e-7, 1e-5, 1e-2, 1, 1e3, 6e4)]).astype(np.float32)
    x = np.concatenate([x, np.float32([65504, 65519.9, 65520, -65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 0.0])])
    f16 = np.array([lib.orc_round_f16(float(v)) for v in x], np.float32)
    np.testing.assert_array_equal(f16, x.astype(np.float16).astype(np.float32))
    bf = np.array([lib.orc_round_bf16(float(v)) for v in x], np.float32)
    np.testing.assert_array_equal(bf, torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy())
