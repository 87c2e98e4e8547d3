"""ribn_amd: Python binding of librocm_ribn (the MI355X backend of ribn's token loop).

The product is the C ABI in ``include/ribn_rocm.h`` (C++/HIP, built in-tree as
``ribn_amd/librocm_ribn.so``). This module is a thin ctypes mirror of it, shaped
like the reference's Rust surfaces so tests read like the reference's own:

* :class:`QwenRocm` - ``GenerationExecutor`` (crates/runtime/src/executor.rs:171-254)
  with ``admit / prepare / abandon_preparation / submit / poll / release /
  synchronize``, plus the device-resident greedy loop (``generate``) and a
  teacher-forced ``trace``.
* kernel-level helpers: ``dequantize`` (dequantize_block, crates/gguf/src/lib.rs:508),
  ``gemv`` (gguf_gemv, crates/nvidia/src/qwen_reference.rs:31), ``argmax``
  (model_ops.rs:203).

There is no CPU fallback: importing fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# RIBN_ROCM_LIB points at an alternative build of the same library (development only).
LIB_PATH = os.environ.get("RIBN_ROCM_LIB") or os.path.join(_HERE, "librocm_ribn.so")

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 8, 12, 14
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210)}

RIBN_OK, RIBN_PENDING = 0, 1
LOAD_KV_BF16 = 1
LOAD_PERSISTENT_STEP = 2
LOAD_RESIDENT_F16 = 4
LOAD_INT_DOT = 8
LOAD_GEMM_FROM_PLANES = 16
LOAD_ATTN_MERGE_IN_LAUNCH = 32
ADMIT_READY, ADMIT_REJECTED, ADMIT_DEFERRED = 0, 1, 2
STEP_PREFILL, STEP_DECODE = 0, 1


class RibnError(RuntimeError):
    """An error status from librocm_ribn (ExecutionError)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
        "(there is no CPU fallback)"
    )
_lib = ctypes.CDLL(LIB_PATH)

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_ERR = 4096


class LoadOptions(ctypes.Structure):
    _fields_ = [("context_tokens", ctypes.c_uint32), ("max_sequences", ctypes.c_uint32),
                ("max_batch_tokens", ctypes.c_uint32), ("kv_pages", ctypes.c_uint32),
                ("device", ctypes.c_int32), ("flags", ctypes.c_uint32)]


class Info(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("context_tokens", ctypes.c_uint32),
                ("max_sequences", ctypes.c_uint32), ("max_batch_tokens", ctypes.c_uint32),
                ("max_decode_tokens", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
                ("layers", ctypes.c_uint32), ("q_heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("ffn", ctypes.c_uint32), ("vocab", ctypes.c_uint32),
                ("rope_dims", ctypes.c_uint32), ("weight_bytes", ctypes.c_uint64), ("kv_bytes", ctypes.c_uint64),
                ("kv_f16", ctypes.c_uint32), ("persistent_step", ctypes.c_uint32),
                ("step_workgroups", ctypes.c_uint32)]


class TokenOptions(ctypes.Structure):
    _fields_ = [("max_output_tokens", ctypes.c_uint32), ("temperature", ctypes.c_float),
                ("stop_tokens", _u32p), ("n_stop_tokens", ctypes.c_uint32)]


class BatchItemC(ctypes.Structure):
    _fields_ = [("sequence", ctypes.c_uint64), ("kind", ctypes.c_uint32), ("prefix", ctypes.c_uint32),
                ("token_budget", ctypes.c_uint32), ("output_budget", ctypes.c_uint32)]


class StepCompletionC(ctypes.Structure):
    _fields_ = [("sequence", ctypes.c_uint64), ("prefix", ctypes.c_uint32), ("n_tokens", ctypes.c_uint32),
                ("token", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class Timing(ctypes.Structure):
    _fields_ = [("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double),
                ("prefill_tokens", ctypes.c_uint32), ("decode_tokens", ctypes.c_uint32)]


class SynthConfig(ctypes.Structure):
    _fields_ = [("qwen3", ctypes.c_int32), ("hidden", ctypes.c_uint32), ("layers", ctypes.c_uint32),
                ("q_heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("ffn", ctypes.c_uint32), ("vocab", ctypes.c_uint32), ("context_length", ctypes.c_uint32),
                ("rope_base", ctypes.c_float), ("rms_eps", ctypes.c_float), ("weight_std", ctypes.c_float),
                ("norm_jitter", ctypes.c_float), ("seed", ctypes.c_uint64), ("weight_type", ctypes.c_uint32),
                ("attn_v_type", ctypes.c_uint32), ("ffn_down_type", ctypes.c_uint32),
                ("output_type", ctypes.c_uint32), ("embd_type", ctypes.c_uint32),
                ("tied_output", ctypes.c_int32), ("threads", ctypes.c_int32)]


class SynthHybrid(ctypes.Structure):
    _fields_ = [("ssm_groups", ctypes.c_uint32), ("ssm_heads", ctypes.c_uint32), ("ssm_state", ctypes.c_uint32),
                ("conv_kernel", ctypes.c_uint32), ("full_attention_interval", ctypes.c_uint32),
                ("rope_dims", ctypes.c_uint32), ("ssm_type", ctypes.c_uint32)]


def _sig(name, res, *args):
    f = getattr(_lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_c = ctypes
_sig("ribn_rocm_load_gguf", _c.c_int, _c.c_char_p, _c.POINTER(LoadOptions), _c.POINTER(_c.c_void_p), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_free", None, _c.c_void_p)
_sig("ribn_rocm_info", _c.c_int, _c.c_void_p, _c.POINTER(Info))
_sig("ribn_rocm_admit", _c.c_int, _c.c_void_p, _c.c_uint64, _c.c_uint64, _u32p, _c.c_uint32,
     _c.POINTER(TokenOptions), _c.POINTER(_c.c_int32), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_prepare", _c.c_int, _c.c_void_p, _c.POINTER(BatchItemC), _c.c_size_t, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_abandon", _c.c_int, _c.c_void_p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_submit", _c.c_int, _c.c_void_p, _c.POINTER(BatchItemC), _c.c_size_t, _c.POINTER(_c.c_uint64),
     _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_poll", _c.c_int, _c.c_void_p, _c.c_uint64, _c.POINTER(StepCompletionC), _c.c_size_t,
     _c.POINTER(_c.c_size_t), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_release", _c.c_int, _c.c_void_p, _c.c_uint64, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_synchronize", _c.c_int, _c.c_void_p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_generate", _c.c_int, _c.c_void_p, _u32p, _c.c_uint32, _c.c_uint32, _u32p, _c.POINTER(Timing),
     _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_trace", _c.c_int, _c.c_void_p, _u32p, _c.c_uint32, _u32p, _f32p, _f32p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_batch_logits", _c.c_int, _c.c_void_p, _c.POINTER(_c.c_uint64), _f32p, _c.c_size_t,
     _c.POINTER(_c.c_size_t), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_dequantize", _c.c_int, _c.c_uint32, _u8p, _c.c_uint64, _c.c_uint64, _f32p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_gemv", _c.c_int, _c.c_uint32, _u8p, _c.c_uint64, _c.c_uint64, _f32p, _f32p, _c.c_float, _f32p,
     _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_bench_gemv", _c.c_int, _c.c_uint32, _c.c_uint64, _c.c_uint64, _c.c_uint32, _c.POINTER(_c.c_double),
     _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_quantize_q8_1", _c.c_int, _f32p, _c.c_uint64, _u32p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_gemv_q8_1", _c.c_int, _c.c_uint32, _u8p, _c.c_uint64, _c.c_uint64, _u32p, _c.c_uint32, _f32p,
     _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_bench_gemv_q8_1", _c.c_int, _c.c_uint32, _c.c_uint64, _c.c_uint64, _c.c_uint32, _c.c_uint32,
     _c.POINTER(_c.c_double), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_argmax", _c.c_int, _f32p, _c.c_uint64, _u32p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_bench_model_kernel", _c.c_int, _c.c_void_p, _c.c_uint32, _c.c_uint32, _c.POINTER(_c.c_double),
     _c.POINTER(_c.c_uint64), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_step_stamps", _c.c_int, _c.c_void_p, _c.c_uint32, _c.POINTER(_c.c_double), _c.c_size_t,
     _c.POINTER(_c.c_size_t), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_prefill_trace", _c.c_int, _c.c_void_p, _u32p, _c.c_uint32, _c.c_uint32, _f32p, _f32p, _c.c_char_p,
     _c.c_size_t)
_sig("ribn_rocm_prefill_gemm", _c.c_int, _c.c_uint32, _u8p, _c.c_uint64, _c.c_uint64, _f32p, _c.c_uint64, _f32p,
     _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_synth_qwen_gguf", _c.c_int, _c.c_char_p, _c.POINTER(SynthConfig), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_synth_qwen35_gguf", _c.c_int, _c.c_char_p, _c.POINTER(SynthConfig), _c.POINTER(SynthHybrid), _c.c_char_p,
     _c.c_size_t)
_sig("ribn_rocm_quantize", _c.c_int, _c.c_uint32, _f32p, _c.c_uint64, _u8p)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _check(rc: int, buf) -> int:
    if rc < 0:
        raise RibnError(rc, buf.value.decode(errors="replace"))
    return rc


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


# --------------------------------------------------------------------------
# synthetic models and kernel-level helpers

def synth_qwen_gguf(path: str, *, qwen3: bool = True, hidden: int, layers: int, q_heads: int, kv_heads: int,
                    head_dim: int, ffn: int, vocab: int, weight_type: int = GGML_Q4_K, attn_v_type: int = 0,
                    ffn_down_type: int = 0, output_type: int = 0, embd_type: int = 0, rope_base: float = 1e6,
                    rms_eps: float = 1e-6, weight_std: float = 0.02, norm_jitter: float = 0.0, seed: int = 0,
                    context_length: int = 32768, tied_output: bool = False, threads: int = 0) -> str:
    """Write a seeded synthetic dense-Qwen GGUF v3 (N(0, weight_std) weights, GGML-quantized)."""
    cfg = SynthConfig(int(qwen3), hidden, layers, q_heads, kv_heads, head_dim, ffn, vocab, context_length,
                      rope_base, rms_eps, weight_std, norm_jitter, seed, weight_type, attn_v_type, ffn_down_type,
                      output_type, embd_type, int(tied_output), threads)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_synth_qwen_gguf(path.encode(), ctypes.byref(cfg), err, _ERR), err)
    return path


def synth_qwen35_gguf(path: str, *, hidden: int, layers: int, q_heads: int, kv_heads: int, head_dim: int, ffn: int,
                      vocab: int, ssm_groups: int, ssm_heads: int, ssm_state: int, full_attention_interval: int = 4,
                      rope_dims: int = 0, conv_kernel: int = 4, ssm_type: int = GGML_Q8_0,
                      weight_type: int = GGML_Q4_K, attn_v_type: int = 0, ffn_down_type: int = 0, output_type: int = 0,
                      embd_type: int = 0, rope_base: float = 1e7, rms_eps: float = 1e-6, weight_std: float = 0.02,
                      norm_jitter: float = 0.0, seed: int = 0, context_length: int = 32768, tied_output: bool = False,
                      threads: int = 0) -> str:
    """Write a seeded synthetic qwen35 hybrid GGUF v3 (Gated-DeltaNet recurrent layers, a gated full-attention
    layer every `full_attention_interval` layers)."""
    cfg = SynthConfig(1, hidden, layers, q_heads, kv_heads, head_dim, ffn, vocab, context_length, rope_base, rms_eps,
                      weight_std, norm_jitter, seed, weight_type, attn_v_type, ffn_down_type, output_type, embd_type,
                      int(tied_output), threads)
    hy = SynthHybrid(ssm_groups, ssm_heads, ssm_state, conv_kernel, full_attention_interval, rope_dims, ssm_type)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_synth_qwen35_gguf(path.encode(), ctypes.byref(cfg), ctypes.byref(hy), err, _ERR), err)
    return path


def quantize(type_: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    be, bb = BLOCK[type_]
    if x.size % be:
        raise ValueError("size is not a multiple of the block size")
    out = np.zeros(x.size // be * bb, dtype=np.uint8)
    if _lib.ribn_rocm_quantize(type_, _ptr(x, _f32p), x.size, _ptr(out, _u8p)) != 0:
        raise RibnError(-1, "quantize failed")
    return out


def dequantize(type_: int, blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Device dequantization (bit-exact with dequantize_block)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(rows * k, dtype=np.float32)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_dequantize(type_, _ptr(blocks, _u8p), rows, k, _ptr(out, _f32p), err, _ERR), err)
    return out.reshape(rows, k)


def gemv(type_: int, blocks: np.ndarray, rows: int, k: int, x: np.ndarray, rms_weight: Optional[np.ndarray] = None,
         eps: float = 1e-6) -> np.ndarray:
    """Fused dequant-matvec on the device: y = W x (optionally W rms_norm(x) * w)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    w = None if rms_weight is None else np.ascontiguousarray(rms_weight, dtype=np.float32)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_gemv(type_, _ptr(blocks, _u8p), rows, k, _ptr(x, _f32p),
                               None if w is None else _ptr(w, _f32p), eps, _ptr(y, _f32p), err, _ERR), err)
    return y


def bench_gemv(type_: int, rows: int, k: int, iters: int = 50) -> float:
    """Average device milliseconds per matvec launch (HIP events)."""
    ms = ctypes.c_double()
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_bench_gemv(type_, rows, k, iters, ctypes.byref(ms), err, _ERR), err)
    return ms.value


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """Q8_1 words (len(x) / 32 blocks of 9) packed on the device (the reference's quantize_q8_1)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size // 32 * 9, dtype=np.uint32)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_quantize_q8_1(_ptr(x, _f32p), x.size, _ptr(out, _u32p), err, _ERR), err)
    return out


def gemv_q8_1(type_: int, blocks: np.ndarray, rows: int, k: int, packed: np.ndarray, members: int = 1) -> np.ndarray:
    """Integer-dot matvec of `members` Q8_1-packed inputs on the device: y [members][rows]."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    y = np.empty((members, rows), dtype=np.float32)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_gemv_q8_1(type_, _ptr(blocks, _u8p), rows, k, _ptr(packed, _u32p), members,
                                    _ptr(y, _f32p), err, _ERR), err)
    return y


def bench_gemv_q8_1(type_: int, rows: int, k: int, members: int = 1, iters: int = 50) -> float:
    """Average device milliseconds per integer-dot matvec launch (HIP events)."""
    ms = ctypes.c_double()
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_bench_gemv_q8_1(type_, rows, k, members, iters, ctypes.byref(ms), err, _ERR), err)
    return ms.value


def prefill_gemm(type_: int, blocks: np.ndarray, rows: int, k: int, x: np.ndarray) -> np.ndarray:
    """Y = f16(X) dequant(W)^T with the prefill MFMA GEMM; X is [m][k]."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    y = np.empty((m, rows), dtype=np.float32)
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_prefill_gemm(type_, _ptr(blocks, _u8p), rows, k, _ptr(x, _f32p), m, _ptr(y, _f32p), err,
                                       _ERR), err)
    return y


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    out = ctypes.c_uint32()
    err = ctypes.create_string_buffer(_ERR)
    _check(_lib.ribn_rocm_argmax(_ptr(logits, _f32p), logits.size, ctypes.byref(out), err, _ERR), err)
    return out.value


# --------------------------------------------------------------------------
# GenerationExecutor mirror

@dataclass(frozen=True)
class BatchItem:
    """BatchItem (executor.rs:75-85)."""
    sequence: int
    kind: int
    prefix: int
    token_budget: int
    output_budget: int


@dataclass(frozen=True)
class StepCompletion:
    """StepCompletion (executor.rs:113-117)."""
    sequence: int
    prefix: int
    tokens: tuple


@dataclass(frozen=True)
class Admission:
    kind: int          # ADMIT_READY / ADMIT_REJECTED / ADMIT_DEFERRED
    message: str = ""


def _items(batch: Sequence[BatchItem]):
    arr = (BatchItemC * max(1, len(batch)))()
    for i, b in enumerate(batch):
        arr[i] = BatchItemC(b.sequence, b.kind, b.prefix, b.token_budget, b.output_budget)
    return arr


class QwenRocm:
    """A loaded dense Qwen GGUF on one MI355X (QwenCuda, crates/qwen/src/cuda.rs:30-121)."""

    def __init__(self, path: str, *, context_tokens: int = 0, max_sequences: int = 0, max_batch_tokens: int = 0,
                 kv_pages: int = 0, device: int = 0, kv: str = "f16", step: str = "chain", gemm: str = "dequant",
                 gemv: str = "float", gemm_copy: bool = True, attn_merge: str = "apart"):
        """step: "persistent" (one kernel launch per token step when the library has a kernel compiled for
        this model's configuration, else the launch chain) or "chain" (per-stage launches in HIP graphs).
        gemm: "dequant" (chunked prefill and batched decode on the dequantizing MFMA GEMM) or "resident"
        (binary16 copies of the weights made at load, hipBLASLt GEMMs).
        gemv: "float" (default) or "int-dot": sampled decode rows run the lossy integer-dot projections over
        Q8_1-packed inputs (the reference's GemvMode::IntegerDot).
        gemm_copy: the dequantizing GEMMs read a GEMM-ordered copy of the Q4_K / Q6_K weights made at load
        (default) or, False, the decode planes (same results; for comparisons).
        attn_merge: "apart" (default: a long context's decode-attention split partials are merged by a launch
        of their own) or "in-launch" (the attention launch merges them; for comparisons)."""
        if attn_merge not in ("apart", "in-launch"):
            raise ValueError("attn_merge must be 'apart' or 'in-launch'")
        if gemv not in ("float", "int-dot"):
            raise ValueError("gemv must be 'float' or 'int-dot'")
        if gemm not in ("dequant", "resident"):
            raise ValueError("gemm must be 'dequant' or 'resident'")
        if step not in ("persistent", "chain"):
            raise ValueError("step must be 'persistent' or 'chain'")
        opts = LoadOptions(context_tokens, max_sequences, max_batch_tokens, kv_pages, device,
                           (LOAD_KV_BF16 if kv == "bf16" else 0) | (LOAD_PERSISTENT_STEP if step == "persistent" else 0)
                           | (LOAD_RESIDENT_F16 if gemm == "resident" else 0) | (LOAD_INT_DOT if gemv == "int-dot" else 0)
                           | (0 if gemm_copy else LOAD_GEMM_FROM_PLANES)
                           | (LOAD_ATTN_MERGE_IN_LAUNCH if attn_merge == "in-launch" else 0))
        if kv not in ("f16", "bf16"):
            raise ValueError("kv must be 'f16' or 'bf16'")
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(_ERR)
        _check(_lib.ribn_rocm_load_gguf(path.encode(), ctypes.byref(opts), ctypes.byref(h), err, _ERR), err)
        self._h = h
        info = Info()
        _lib.ribn_rocm_info(self._h, ctypes.byref(info))
        self.info = info

    # lifecycle
    def close(self):
        if getattr(self, "_h", None):
            _lib.ribn_rocm_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _call(self, fn, *args):
        err = ctypes.create_string_buffer(_ERR)
        rc = fn(self._h, *args, err, _ERR)
        return _check(rc, err), err.value.decode(errors="replace")

    # executor contract
    def admit(self, request_id: int, sequence: int, tokens: Sequence[int], max_output_tokens: int,
              temperature: float = 0.0, stop_tokens: Sequence[int] = ()) -> Admission:
        toks = _u32(tokens)
        stops = _u32(stop_tokens) if len(stop_tokens) else np.zeros(1, np.uint32)
        opt = TokenOptions(max_output_tokens, temperature, _ptr(stops, _u32p), len(stop_tokens))
        kind = ctypes.c_int32(-1)
        _, msg = self._call(_lib.ribn_rocm_admit, request_id, sequence, _ptr(toks, _u32p) if toks.size else None,
                            toks.size, ctypes.byref(opt), ctypes.byref(kind))
        return Admission(kind.value, msg if kind.value != ADMIT_READY else "")

    def prepare(self, batch: Sequence[BatchItem]) -> None:
        self._call(_lib.ribn_rocm_prepare, _items(batch), len(batch))

    def abandon_preparation(self) -> None:
        self._call(_lib.ribn_rocm_abandon)

    def submit(self, batch: Sequence[BatchItem]) -> int:
        sid = ctypes.c_uint64()
        self._call(_lib.ribn_rocm_submit, _items(batch), len(batch), ctypes.byref(sid))
        return sid.value

    def poll(self, submission: int):
        cap = max(1, self.info.max_sequences)
        out = (StepCompletionC * cap)()
        n = ctypes.c_size_t()
        rc, _ = self._call(_lib.ribn_rocm_poll, submission, out, cap, ctypes.byref(n))
        if rc == RIBN_PENDING:
            return None
        return [StepCompletion(out[i].sequence, out[i].prefix, (out[i].token,) if out[i].n_tokens else ())
                for i in range(n.value)]

    def batch_logits(self):
        """Logits of the decode rows the last completed submission ran as one batched step:
        (sequence ids, [rows][vocab]); empty when it ran none."""
        cap = max(1, self.info.max_sequences)
        seqs = np.zeros(cap, dtype=np.uint64)
        out = np.zeros((cap, self.info.vocab), dtype=np.float32)
        n = ctypes.c_size_t()
        self._call(_lib.ribn_rocm_batch_logits, seqs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                   _ptr(out, _f32p), cap, ctypes.byref(n))
        return seqs[: n.value].tolist(), out[: n.value].copy()

    def release(self, sequence: int) -> None:
        self._call(_lib.ribn_rocm_release, sequence)

    def synchronize(self) -> None:
        self._call(_lib.ribn_rocm_synchronize)

    # lower seams
    def generate(self, prompt: Sequence[int], n_new: int):
        p = _u32(prompt)
        out = np.zeros(n_new, dtype=np.uint32)
        t = Timing()
        self._call(_lib.ribn_rocm_generate, _ptr(p, _u32p), p.size, n_new, _ptr(out, _u32p), ctypes.byref(t))
        return out, t

    def trace(self, tokens: Sequence[int], logits: bool = True, hidden: bool = False):
        t = _u32(tokens)
        n = t.size
        am = np.zeros(n, dtype=np.uint32)
        lg = np.zeros((n, self.info.vocab), dtype=np.float32) if logits else None
        hd = np.zeros((n, self.info.layers + 1, self.info.hidden), dtype=np.float32) if hidden else None
        self._call(_lib.ribn_rocm_trace, _ptr(t, _u32p), n, _ptr(am, _u32p),
                   None if lg is None else _ptr(lg, _f32p), None if hd is None else _ptr(hd, _f32p))
        return am, lg, hd

    def prefill_trace(self, tokens: Sequence[int], chunk: int = 0, logits: bool = True, hidden: bool = False):
        """Chunked-prefill trace: (logits [n][vocab], hidden [n][layers + 1][hidden]) per row."""
        t = _u32(tokens)
        n = t.size
        lg = np.zeros((n, self.info.vocab), dtype=np.float32) if logits else None
        hd = np.zeros((self.info.layers + 1, n, self.info.hidden), dtype=np.float32) if hidden else None
        self._call(_lib.ribn_rocm_prefill_trace, _ptr(t, _u32p), n, chunk, None if lg is None else _ptr(lg, _f32p),
                   None if hd is None else _ptr(hd, _f32p))
        return lg, (None if hd is None else np.ascontiguousarray(hd.transpose(1, 0, 2)))

    def step_stamps(self, ctx: int):
        """Wall-clock marks (ns) of one persistent step at context ctx (see ribn_rocm_step_stamps)."""
        cap = 64 * (self.info.layers + 1)
        out = (ctypes.c_double * cap)()
        n = ctypes.c_size_t()
        self._call(_lib.ribn_rocm_step_stamps, ctx, out, cap, ctypes.byref(n))
        return np.frombuffer(out, dtype=np.float64, count=n.value).copy()

    def bench_kernel(self, which: int, iters: int = 50, ctx: int = 0):
        ms = ctypes.c_double()
        nbytes = ctypes.c_uint64(ctx)
        self._call(_lib.ribn_rocm_bench_model_kernel, which, iters, ctypes.byref(ms), ctypes.byref(nbytes))
        return ms.value, nbytes.value


# --------------------------------------------------------------------------
# GemmaDecode mirror (crates/gemma4/src/executor/backend.rs:10-33)

class GemmaInfo(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_uint32), ("hidden", ctypes.c_uint32), ("layers", ctypes.c_uint32),
                ("context", ctypes.c_uint32)]


_u16p = ctypes.POINTER(ctypes.c_uint16)
_sig("ribn_rocm_gemma_open", _c.c_int, _c.c_char_p, _c.c_int32, _c.POINTER(_c.c_void_p), _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_gemma_close", None, _c.c_void_p)
_sig("ribn_rocm_gemma_info", _c.c_int, _c.c_void_p, _c.POINTER(GemmaInfo))
_sig("ribn_rocm_gemma_prefill", _c.c_int, _c.c_void_p, _u32p, _c.c_uint32, _u16p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_gemma_advance_prefill", _c.c_int, _c.c_void_p, _u32p, _c.c_uint32, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_gemma_decode", _c.c_int, _c.c_void_p, _c.c_uint32, _u16p, _c.c_char_p, _c.c_size_t)
_sig("ribn_rocm_gemma_position", _c.c_uint32, _c.c_void_p)
_sig("ribn_rocm_gemma_reset", _c.c_int, _c.c_void_p)


class GemmaRocm:
    """The Gemma 4 text decoder on the GPU behind the GemmaDecode seam: prefill / advance_prefill /
    decode return or skip the BF16 logits (uint16 bit patterns, post soft cap) of the chunk's last
    token; a rejected chunk leaves the position unchanged (RibnError)."""

    def __init__(self, package_dir: str, device: int = 0):
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(_ERR)
        _check(_lib.ribn_rocm_gemma_open(package_dir.encode(), device, ctypes.byref(h), err, _ERR), err)
        self._h = h
        info = GemmaInfo()
        _lib.ribn_rocm_gemma_info(self._h, ctypes.byref(info))
        self.vocab, self.hidden, self.layers, self.context = info.vocab, info.hidden, info.layers, info.context

    def close(self):
        if getattr(self, "_h", None):
            _lib.ribn_rocm_gemma_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        self.close()

    @property
    def position(self) -> int:
        return int(_lib.ribn_rocm_gemma_position(self._h))

    def reset(self):
        _lib.ribn_rocm_gemma_reset(self._h)

    def prefill(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.vocab, np.uint16)
        err = ctypes.create_string_buffer(_ERR)
        _check(_lib.ribn_rocm_gemma_prefill(self._h, _ptr(t, _u32p), t.size, _ptr(out, _u16p), err, _ERR), err)
        return out

    def advance_prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        err = ctypes.create_string_buffer(_ERR)
        _check(_lib.ribn_rocm_gemma_advance_prefill(self._h, _ptr(t, _u32p), t.size, err, _ERR), err)

    def decode(self, token: int) -> np.ndarray:
        out = np.empty(self.vocab, np.uint16)
        err = ctypes.create_string_buffer(_ERR)
        _check(_lib.ribn_rocm_gemma_decode(self._h, int(token), _ptr(out, _u16p), err, _ERR), err)
        return out

    @staticmethod
    def argmax(logits: np.ndarray) -> int:
        """First maximum of BF16 logits (cpu/decoder.rs:316-332)."""
        v = (np.asarray(logits, np.uint16).astype(np.uint32) << 16).view(np.float32)
        if v.size == 0 or np.isnan(v[0]):   # nothing compares greater than a NaN first entry
            return 0
        return int(np.argmax(np.where(np.isnan(v), -np.inf, v)))


__all__ = [
    "QwenRocm", "GemmaRocm", "synth_qwen35_gguf", "BatchItem", "StepCompletion", "Admission", "RibnError", "synth_qwen_gguf", "quantize",
    "dequantize", "gemv", "bench_gemv", "prefill_gemm", "argmax", "LIB_PATH", "GGML_F32", "GGML_F16", "GGML_Q8_0", "GGML_Q4_K",
    "GGML_Q6_K", "BLOCK", "STEP_PREFILL", "STEP_DECODE", "ADMIT_READY", "ADMIT_REJECTED", "ADMIT_DEFERRED",
]
