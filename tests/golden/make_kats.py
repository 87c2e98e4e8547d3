"""Writes gguf_kats.json: the known-answer vectors of the reference's own GGUF tests.

Inputs and expected outputs are the values stated in crates/gguf/src/lib.rs
(dequantizes_supported_scalar_and_quantized_blocks :1480-1566,
rejects_invalid_dequantization_blocks :1568-1583,
computes_quantized_tensor_block_sizes :1585-1625, parser fixture :1219-1276)
and the dyadic block builders of crates/nvidia/tests/q4_q8_1.rs:15-50,
q6_q8_1.rs:13-45 and q8_0_q8_1.rs:10-29, re-expressed as data. Expected values
of the builders are the exact f64 products d*sc*q - dmin*m the reference
asserts (q4_q8_1.rs:205-228). Run: python tests/golden/make_kats.py
"""
import json
import os
import struct


def half_bits_value(bits):
    e = (bits >> 10) & 31
    f = bits & 1023
    mag = f * 2.0 ** -24 if e == 0 else (1 + f / 1024) * 2.0 ** (e - 15)
    return -mag if bits & 0x8000 else mag


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def q4k_block(seed):
    scales = [1, 17, 33, 63, 32, 47, 62, 48]
    minima = [63, 32, 17, 1, 47, 48, 33, 62]
    d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
    m_bits = [0x2800, 0x2C00, 0x3000][seed % 3]
    enc = bytearray(144)
    enc[0:2] = struct.pack("<H", d_bits)
    enc[2:4] = struct.pack("<H", m_bits)
    for g in range(4):
        enc[4 + g] = scales[g] | ((scales[g + 4] >> 4) << 6)
        enc[8 + g] = minima[g] | ((minima[g + 4] >> 4) << 6)
        enc[12 + g] = (scales[g + 4] & 15) | ((minima[g + 4] & 15) << 4)
    quants = [(i * 7 + seed * 3 + i // 32) % 16 for i in range(256)]
    for g in range(8):
        for i in range(32):
            enc[16 + (g // 2) * 32 + i] |= quants[g * 32 + i] << ((g % 2) * 4)
    d, dm = half_bits_value(d_bits), half_bits_value(m_bits)
    expect = [d * scales[i // 32] * quants[i] - dm * minima[i // 32] for i in range(256)]
    return bytes(enc), expect


def q6k_block(seed):
    scales = [3, -5, 11, -13, 19, -23, 29, -31, 7, -9, 15, -17, 21, -25, 27, -2]
    d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
    enc = bytearray(210)
    quants = [((i * 7 + seed * 3 + i // 32) % 64) - 32 for i in range(256)]
    for g in range(8):
        low_base = (g // 4) * 64 + (g % 2) * 32
        low_shift = 0 if g % 4 < 2 else 4
        high_base = 128 + (g // 4) * 32
        high_shift = (g % 4) * 2
        for i in range(32):
            u = quants[g * 32 + i] + 32
            enc[low_base + i] |= (u & 15) << low_shift
            enc[high_base + i] |= ((u >> 4) & 3) << high_shift
    for i, s in enumerate(scales):
        enc[192 + i] = s & 0xFF
    enc[208:210] = struct.pack("<H", d_bits)
    d = half_bits_value(d_bits)
    expect = [d * scales[i // 16] * quants[i] for i in range(256)]
    return bytes(enc), expect


def q8_0_block(seed):
    d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
    quants = [((i * 11 + seed * 5) % 61) - 30 for i in range(32)]
    enc = bytearray(34)
    enc[0:2] = struct.pack("<H", d_bits)
    for i, q in enumerate(quants):
        enc[2 + i] = q & 0xFF
    d = half_bits_value(d_bits)
    return bytes(enc), [d * q for q in quants]


def main():
    kats = []
    kats.append({"type": 0, "block": struct.pack("<f", 1.5).hex(), "expect_bits": {"0": f32_bits(1.5)}, "len": 1})
    kats.append({"type": 1, "block": struct.pack("<H", 0x3C00).hex(), "expect_bits": {"0": f32_bits(1.0)}, "len": 1})
    q8 = bytearray(34); q8[0:2] = struct.pack("<H", 0x3C00); q8[2] = 0x80; q8[3] = 0x7F
    kats.append({"type": 8, "block": bytes(q8).hex(), "expect_bits": {"0": f32_bits(-128.0), "1": f32_bits(127.0)}, "len": 32})
    q4 = bytearray(144); q4[0:2] = struct.pack("<H", 0x3C00); q4[4:8] = b"\x01" * 4; q4[16] = 0x10
    kats.append({"type": 12, "block": bytes(q4).hex(), "expect_bits": {"0": f32_bits(0.0), "32": f32_bits(1.0)}, "len": 256})
    q6 = bytearray(210); q6[192:208] = b"\x01" * 16; q6[208:210] = struct.pack("<H", 0x3C00)
    kats.append({"type": 14, "block": bytes(q6).hex(), "expect_all_bits": f32_bits(-32.0), "len": 256})
    errors = [{"type": 12, "len": 143, "error": "block_length"}, {"type": 22, "len": 82, "error": "unsupported"}]
    byte_lens = [{"type": 12, "dims": [256], "bytes": 144}, {"type": 12, "dims": [128, 2], "bytes": None},
                 {"type": 23, "dims": [256], "bytes": 136}, {"type": 21, "dims": [256], "bytes": 110}]
    builders = []
    for seed in range(15):   # ROWS*(INPUTS/256) = 5*3 blocks, as the reference builder
        e, x = q4k_block(seed); builders.append({"type": 12, "block": e.hex(), "expect": x})
        e, x = q6k_block(seed); builders.append({"type": 14, "block": e.hex(), "expect": x})
    for seed in range(24):
        e, x = q8_0_block(seed); builders.append({"type": 8, "block": e.hex(), "expect": x})
    out = {"kats": kats, "errors": errors, "byte_lens": byte_lens, "builders": builders}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf_kats.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print("wrote", path)


if __name__ == "__main__":
    main()
