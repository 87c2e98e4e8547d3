"""Host fixtures of the reference's integer-dot tests (Q8_1 activations x Q4_K / Q6_K / Q8_0 weights),
built from the generator rules those tests state:

- crates/nvidia/tests/q4_q8_1.rs:13-47    Q4_K blocks (scales, minima, d / dmin patterns, quants)
- crates/nvidia/tests/q6_q8_1.rs:13-45    Q6_K blocks (signed 16-entry scale pattern, quants - 32)
- crates/nvidia/tests/q8_0_q8_1.rs:10-28  Q8_0 blocks
- activations(exact): dyadic values a Q8_1 block holds without loss; activations(lossy): values it does not
- expected(): the per-row binary64 sums of those tests' `reference()` (packed output, float output, packing
  error bound, arithmetic magnitude), computed from the fixture quants, not from the encoded bytes.

All fixtures are 5 rows of 768 inputs.
"""
import numpy as np

INPUTS = 768
ROWS = 5


def half(bits):
    return float(np.uint16(bits).view(np.float16))


def q4k_blocks():
    scales = [1, 17, 33, 63, 32, 47, 62, 48]
    minima = [63, 32, 17, 1, 47, 48, 33, 62]
    out = []
    for seed in range(ROWS * (INPUTS // 256)):
        d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
        m_bits = [0x2800, 0x2C00, 0x3000][seed % 3]
        enc = np.zeros(144, np.uint8)
        enc[0:2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
        enc[2:4] = np.frombuffer(np.uint16(m_bits).tobytes(), np.uint8)
        for g in range(4):
            enc[4 + g] = scales[g] | ((scales[g + 4] >> 4) << 6)
            enc[8 + g] = minima[g] | ((minima[g + 4] >> 4) << 6)
            enc[12 + g] = (scales[g + 4] & 15) | ((minima[g + 4] & 15) << 4)
        quants = np.array([(i * 7 + seed * 3 + i // 32) % 16 for i in range(256)], np.int64)
        for g in range(8):
            for i in range(32):
                enc[16 + (g // 2) * 32 + i] |= quants[g * 32 + i] << ((g % 2) * 4)
        out.append(dict(enc=enc, quants=quants, scales=scales, minima=minima, d=half(d_bits), dmin=half(m_bits)))
    return out


def q6k_blocks():
    scales = [3, -5, 11, -13, 19, -23, 29, -31, 7, -9, 15, -17, 21, -25, 27, -2]
    out = []
    for seed in range(ROWS * (INPUTS // 256)):
        d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
        enc = np.zeros(210, np.uint8)
        quants = np.array([(i * 7 + seed * 3 + i // 32) % 64 - 32 for i in range(256)], np.int64)
        for g in range(8):
            low_base = (g // 4) * 64 + (g % 2) * 32
            low_shift = 0 if g % 4 < 2 else 4
            high_base = 128 + (g // 4) * 32
            high_shift = (g % 4) * 2
            for i in range(32):
                u = int(quants[g * 32 + i] + 32)
                enc[low_base + i] |= (u & 15) << low_shift
                enc[high_base + i] |= ((u >> 4) & 3) << high_shift
        enc[192:208] = np.array(scales, np.int8).view(np.uint8)
        enc[208:210] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
        out.append(dict(enc=enc, quants=quants, scales=scales, d=half(d_bits)))
    return out


def q8_0_blocks():
    out = []
    for seed in range(ROWS * (INPUTS // 32)):
        d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
        quants = np.array([(i * 11 + seed * 5) % 61 - 30 for i in range(32)], np.int64)
        enc = np.zeros(34, np.uint8)
        enc[0:2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
        enc[2:] = quants.astype(np.int8).view(np.uint8)
        out.append(dict(enc=enc, quants=quants, d=half(d_bits)))
    return out


BLOCKS = {12: q4k_blocks, 14: q6k_blocks, 8: q8_0_blocks}


def encoded(t):
    return np.concatenate([b["enc"] for b in BLOCKS[t]()])


def activations(exact):
    i = np.arange(INPUTS)
    if exact:
        integer = np.where(i % 32 == 0, 127, np.where(i % 32 == 1, -127, (i * 7) % 17 - 8))
        return (integer.astype(np.float32) * np.array([0.25, 0.125, 0.0625], np.float32)[(i // 32) % 3]).astype(
            np.float32)
    return (((i * 17 + 3) % 101 - 50).astype(np.float32) * np.float32(0.0137)).astype(np.float32)


def unpack(packed):
    """Per 32-block: (scale, sum) decoded from the header halves, and the 32 signed bytes."""
    w = packed.reshape(-1, 9)
    scale = np.array([half(x & 0xFFFF) for x in w[:, 0]])
    ssum = np.array([half(x >> 16) for x in w[:, 0]])
    q = w[:, 1:].copy().view(np.int8).reshape(-1, 32).astype(np.int64)
    return scale, ssum, q


def expected(t, x, packed):
    """Rows of (packed_output, float_output, packing_error_bound, arithmetic_magnitude)."""
    blocks = BLOCKS[t]()
    scale, ssum, q = unpack(packed)
    x = x.astype(np.float64)
    per_row = INPUTS // (32 if t == 8 else 256)
    rows = []
    for r in range(ROWS):
        po = fo = bound = mag = 0.0
        for bi in range(per_row):
            b = blocks[r * per_row + bi]
            if t == 8:
                j = bi
                wq, a = b["quants"], b["d"]
                dot = int(np.dot(wq, q[j]))
                xs = x[j * 32:(j + 1) * 32]
                fo += float(np.sum(a * wq * xs))
                bound += float(np.sum(abs(a) * np.abs(wq) * np.abs(scale[j] * q[j] - xs)))
                mag += float(np.sum(np.abs(a * wq * scale[j] * q[j])))
                po += a * scale[j] * dot
                mag += abs(a * scale[j] * dot)
                continue
            for g in range(8):
                j = bi * 8 + g
                xs = x[j * 32:(j + 1) * 32]
                wq = b["quants"][g * 32:(g + 1) * 32]
                if t == 12:
                    a = b["d"] * b["scales"][g]
                    mb = b["dmin"] * b["minima"][g]
                    dot = int(np.dot(wq, q[j]))
                    fo += float(np.sum((a * wq - mb) * xs))
                    bound += float(np.sum(abs(a) * wq * np.abs(scale[j] * q[j] - xs)))
                    mag += float(np.sum(np.abs(a * wq * scale[j] * q[j])))
                    po += a * scale[j] * dot - mb * ssum[j]
                    mag += abs(mb * ssum[j])
                    bound += abs(mb) * abs(ssum[j] - float(np.sum(xs)))
                else:
                    for h in range(2):
                        a = b["d"] * b["scales"][g * 2 + h]
                        sl = slice(16 * h, 16 * h + 16)
                        dot = int(np.dot(wq[sl] + 32, q[j][sl]))
                        asum = int(np.sum(q[j][sl]))
                        fo += float(np.sum(a * wq[sl] * xs[sl]))
                        bound += float(np.sum(abs(a) * np.abs(wq[sl]) * np.abs(scale[j] * q[j][sl] - xs[sl])))
                        mag += float(np.sum(np.abs(a * wq[sl] * scale[j] * q[j][sl])))
                        po += a * scale[j] * (dot - 32 * asum)
                        mag += abs(a * scale[j] * (dot - 32 * asum))
        rows.append((po, fo, bound, mag))
    return rows
