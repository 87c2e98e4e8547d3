"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- test infrastructure only."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "liboracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            import subprocess
            subprocess.check_call(["make", "-C", os.path.join(ROOT, "oracle")])
        _lib = ctypes.CDLL(LIB)
        c = ctypes
        _lib.orc_f16_to_f32.restype = c.c_float
        _lib.orc_f16_to_f32.argtypes = [c.c_uint16]
        _lib.orc_tensor_layout.argtypes = [c.c_uint32, c.POINTER(c.c_uint64), c.POINTER(c.c_uint64)]
        _lib.orc_dequantize_block.argtypes = [c.c_uint32, c.c_void_p, c.c_size_t, c.c_void_p]
        _lib.orc_dequantize.restype = c.c_int64
        _lib.orc_dequantize.argtypes = [c.c_uint32, c.c_void_p, c.c_size_t, c.c_void_p]
        _lib.orc_tensor_byte_len.restype = c.c_int64
        _lib.orc_tensor_byte_len.argtypes = [c.c_uint32, c.POINTER(c.c_uint64), c.c_uint32]
        _lib.orc_gguf_open.argtypes = [c.c_char_p, c.POINTER(c.c_void_p)]
        _lib.orc_gguf_close.argtypes = [c.c_void_p]
        _lib.orc_gguf_version.argtypes = [c.c_void_p]
        _lib.orc_gguf_version.restype = c.c_uint32
        _lib.orc_gguf_tensor_count.argtypes = [c.c_void_p]
        _lib.orc_gguf_tensor_count.restype = c.c_uint64
        _lib.orc_gguf_get_u64.argtypes = [c.c_void_p, c.c_char_p, c.POINTER(c.c_uint64)]
        _lib.orc_gguf_get_str.argtypes = [c.c_void_p, c.c_char_p, c.c_char_p, c.c_size_t]
        _lib.orc_gguf_tensor.argtypes = [c.c_void_p, c.c_char_p, c.POINTER(c.c_uint32), c.POINTER(c.c_uint64),
                                         c.POINTER(c.c_uint32), c.POINTER(c.c_uint64), c.POINTER(c.c_uint64)]
        _lib.orc_gguf_bytes.restype = c.c_void_p
        _lib.orc_gguf_bytes.argtypes = [c.c_void_p]
        _lib.orc_gemv_q.argtypes = [c.c_uint32, c.c_void_p, c.c_uint64, c.c_uint64, c.c_void_p, c.c_void_p, c.c_int]
        _lib.orc_rms_norm.argtypes = [c.c_void_p, c.c_void_p, c.c_void_p, c.c_int, c.c_float]
        _lib.orc_rope_neox.argtypes = [c.c_void_p, c.c_int, c.c_int, c.c_int, c.c_int64, c.c_float]
        _lib.orc_argmax.restype = c.c_uint32
        _lib.orc_argmax.argtypes = [c.c_void_p, c.c_int]
        _lib.orc_qwen_open.argtypes = [c.c_char_p, c.c_int, c.POINTER(c.c_void_p)]
        _lib.orc_qwen_close.argtypes = [c.c_void_p]
        _lib.orc_qwen_config.argtypes = [c.c_void_p, c.c_void_p, c.POINTER(c.c_float), c.POINTER(c.c_float)]
        _lib.orc_qwen_step.argtypes = [c.c_void_p, c.c_uint32, c.c_int, c.c_void_p, c.c_void_p, c.c_void_p]
        _lib.orc_qwen_append_kv.argtypes = [c.c_void_p, c.c_uint32, c.c_int]
        _lib.orc_qwen_reset.argtypes = [c.c_void_p]
        _lib.orc_qwen_set_kv_round.argtypes = [c.c_void_p, c.c_int]
        _lib.orc_qwen_set_threads.argtypes = [c.c_void_p, c.c_int]
        _lib.orc_q35_open.argtypes = [c.c_char_p, c.c_int, c.POINTER(c.c_void_p)]
        _lib.orc_q35_close.argtypes = [c.c_void_p]
        _lib.orc_q35_config.argtypes = [c.c_void_p, c.c_void_p]
        _lib.orc_q35_step.argtypes = [c.c_void_p, c.c_uint32, c.c_int, c.c_void_p, c.c_void_p]
        _lib.orc_q35_reset.argtypes = [c.c_void_p]
        _lib.orc_q35_set_kv_round.argtypes = [c.c_void_p, c.c_int]
        _lib.orc_gdn_state_step.argtypes = [c.c_void_p, c.c_void_p, c.c_void_p, c.c_void_p, c.c_float, c.c_float,
                                            c.c_int, c.c_int, c.c_void_p]
        _lib.orc_round_f16.restype = c.c_float
        _lib.orc_round_f16.argtypes = [c.c_float]
        _lib.orc_round_bf16.restype = c.c_float
        _lib.orc_round_bf16.argtypes = [c.c_float]
        _lib.orc_quantize_q8_1.argtypes = [c.c_void_p, c.c_uint64, c.c_void_p]
        _lib.orc_gemv_q8_1.argtypes = [c.c_uint32, c.c_void_p, c.c_uint64, c.c_uint64, c.c_void_p, c.c_uint32,
                                       c.c_void_p, c.c_int]
        _lib.orc_qwen_set_gemv_mode.argtypes = [c.c_void_p, c.c_int]
    return _lib


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def layout(t):
    be, bb = ctypes.c_uint64(), ctypes.c_uint64()
    rc = lib().orc_tensor_layout(t, ctypes.byref(be), ctypes.byref(bb))
    return None if rc else (be.value, bb.value)


def dequantize_block(t, enc: bytes):
    enc = np.frombuffer(bytes(enc), dtype=np.uint8).copy()
    out = np.zeros(256, dtype=np.float32)
    rc = lib().orc_dequantize_block(t, enc.ctypes.data, enc.size, out.ctypes.data)
    if rc < 0:
        return rc
    return out[:rc].copy()


def dequantize(t, enc: np.ndarray) -> np.ndarray:
    enc = np.ascontiguousarray(enc, dtype=np.uint8)
    be, bb = layout(t)
    out = np.zeros(enc.size // bb * be, dtype=np.float32)
    rc = lib().orc_dequantize(t, enc.ctypes.data, enc.size, out.ctypes.data)
    assert rc == out.size, rc
    return out


def byte_len(t, dims):
    d = (ctypes.c_uint64 * len(dims))(*dims)
    return lib().orc_tensor_byte_len(t, d, len(dims))


def gemv(t, blocks, rows, k, x, threads=1):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(rows, dtype=np.float32)
    assert lib().orc_gemv_q(t, blocks.ctypes.data, rows, k, x.ctypes.data, y.ctypes.data, threads) == 0
    return y


def quantize_q8_1(x):
    """Q8_1 words (n/32 blocks of 9 u32) of a float vector (orc_quantize_q8_1)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * 9, dtype=np.uint32)
    rc = lib().orc_quantize_q8_1(x.ctypes.data, x.size, out.ctypes.data)
    if rc:
        raise ValueError(f"orc_quantize_q8_1: {rc}")
    return out


def gemv_q8_1(t, blocks, rows, k, packed, members=1, threads=1):
    """Integer-dot matvec over Q8_1 inputs: y [members][rows] (orc_gemv_q8_1)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    assert packed.size == members * (k // 32) * 9
    y = np.zeros((members, rows), dtype=np.float32)
    rc = lib().orc_gemv_q8_1(t, blocks.ctypes.data, rows, k, packed.ctypes.data, members, y.ctypes.data, threads)
    if rc:
        raise ValueError(f"orc_gemv_q8_1: {rc}")
    return y


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.zeros_like(x)
    lib().orc_rms_norm(x.ctypes.data, w.ctypes.data, y.ctypes.data, x.size, eps)
    return y


def rope(v, heads, hd, rot, pos, base):
    v = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().orc_rope_neox(v.ctypes.data, heads, hd, rot, pos, base)
    return v


def argmax(l):
    l = np.ascontiguousarray(l, dtype=np.float32)
    return lib().orc_argmax(l.ctypes.data, l.size)


class Gguf:
    def __init__(self, path):
        self.h = ctypes.c_void_p()
        self.rc = lib().orc_gguf_open(path.encode(), ctypes.byref(self.h))

    def close(self):
        if self.h:
            lib().orc_gguf_close(self.h)
            self.h = None

    def u64(self, key):
        v = ctypes.c_uint64()
        rc = lib().orc_gguf_get_u64(self.h, key.encode(), ctypes.byref(v))
        return None if rc else v.value

    def str(self, key):
        b = ctypes.create_string_buffer(256)
        rc = lib().orc_gguf_get_str(self.h, key.encode(), b, 256)
        return None if rc else b.value.decode()

    def tensor(self, name):
        t = ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        nd = ctypes.c_uint32()
        start, ln = ctypes.c_uint64(), ctypes.c_uint64()
        rc = lib().orc_gguf_tensor(self.h, name.encode(), ctypes.byref(t), dims, ctypes.byref(nd),
                                   ctypes.byref(start), ctypes.byref(ln))
        if rc:
            return rc
        base = lib().orc_gguf_bytes(self.h)
        data = np.ctypeslib.as_array((ctypes.c_uint8 * ln.value).from_address(base + start.value)).copy()
        return t.value, list(dims[: nd.value]), start.value, data


class QwenOracle:
    """FP32 dense-Qwen forward (oracle.c orc_qwen_*)."""

    KV_F32, KV_F16, KV_BF16 = 0, 1, 2

    def __init__(self, path, max_ctx=512, kv_round=0):
        self.h = ctypes.c_void_p()
        rc = lib().orc_qwen_open(path.encode(), max_ctx, ctypes.byref(self.h))
        if rc:
            raise RuntimeError(f"oracle open failed: {rc}")
        lib().orc_qwen_set_kv_round(self.h, kv_round)
        cfg = (ctypes.c_int32 * 8)()
        eps, base = ctypes.c_float(), ctypes.c_float()
        lib().orc_qwen_config(self.h, cfg, ctypes.byref(eps), ctypes.byref(base))
        (self.hidden, self.layers, self.q_heads, self.kv_heads, self.head_dim, self.ffn, self.vocab,
         self.rot) = list(cfg)
        self.pos = 0

    def step(self, token, want_hidden=False):
        logits = np.zeros(self.vocab, dtype=np.float32)
        hid = np.zeros((self.layers + 1, self.hidden), dtype=np.float32) if want_hidden else None
        rc = lib().orc_qwen_step(self.h, int(token), self.pos, logits.ctypes.data,
                                 None if hid is None else hid.ctypes.data, None)
        assert rc == 0, rc
        self.pos += 1
        return logits, hid

    def set_threads(self, n):
        """Matvec worker threads (results are bit-identical for every count)."""
        lib().orc_qwen_set_threads(self.h, int(n))

    GEMV_FLOAT, GEMV_INT_DOT = 0, 2

    def set_gemv_mode(self, mode):
        """Projection mode of the following steps (GEMV_INT_DOT: Q8_1 activations, integer dots)."""
        lib().orc_qwen_set_gemv_mode(self.h, int(mode))

    def append_kv(self, token):
        """Advance one position, writing the K/V cache entries only (no readout)."""
        assert lib().orc_qwen_append_kv(self.h, int(token), self.pos) == 0
        self.pos += 1

    def reset(self):
        lib().orc_qwen_reset(self.h)
        self.pos = 0

    def close(self):
        if self.h:
            lib().orc_qwen_close(self.h)
            self.h = None


def gdn_state_step(state, k, v, q, decay, beta):
    """The delta rule on one head (orc_gdn_state_step), state [key_dim][value_dim]: returns (new state, output)."""
    st = np.ascontiguousarray(state, dtype=np.float32).copy()
    kd, vd = st.shape
    out = np.zeros(vd, dtype=np.float32)
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (k, v, q)]
    lib().orc_gdn_state_step(st.ctypes.data, arrs[0].ctypes.data, arrs[1].ctypes.data, arrs[2].ctypes.data,
                             float(decay), float(beta), kd, vd, out.ctypes.data)
    return st, out


class Qwen35Oracle:
    """FP32 qwen35 hybrid forward (oracle/qwen35.c)."""

    def __init__(self, path, max_ctx=256, kv_round=0):
        self.h = ctypes.c_void_p()
        rc = lib().orc_q35_open(path.encode(), max_ctx, ctypes.byref(self.h))
        if rc:
            raise RuntimeError(f"qwen35 oracle open failed: {rc}")
        lib().orc_q35_set_kv_round(self.h, kv_round)
        cfg = (ctypes.c_int32 * 12)()
        lib().orc_q35_config(self.h, cfg)
        (self.hidden, self.layers, self.q_heads, self.kv_heads, self.head_dim, self.ffn, self.vocab, self.rot,
         self.ssm_groups, self.ssm_heads, self.ssm_state, self.interval) = list(cfg)
        self.pos = 0

    def step(self, token, want_hidden=False):
        logits = np.zeros(self.vocab, dtype=np.float32)
        hid = np.zeros((self.layers + 1, self.hidden), dtype=np.float32) if want_hidden else None
        rc = lib().orc_q35_step(self.h, int(token), self.pos, logits.ctypes.data,
                                None if hid is None else hid.ctypes.data)
        assert rc == 0, rc
        self.pos += 1
        return logits, hid

    def reset(self):
        lib().orc_q35_reset(self.h)
        self.pos = 0

    def close(self):
        if self.h:
            lib().orc_q35_close(self.h)
            self.h = None
