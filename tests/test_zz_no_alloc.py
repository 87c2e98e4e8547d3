"""The allocation-free argmax entry point (ribn_rocm_argmax_noalloc) against ribn_rocm_argmax, through the C ABI.
Device buffers and the stream come from the HIP runtime the library itself links (libamdhip64 through ctypes;
torch is not imported, since it carries a runtime of its own). Two calls in a row on one stream, the second
smaller, a third smaller still; ties and NaN; the size limit."""
import ctypes

import numpy as np
import pytest

import ribn_amd

pytestmark = pytest.mark.gpu

_f = ribn_amd._lib.ribn_rocm_argmax_noalloc
_f.restype = ctypes.c_int
_f.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
H2D, D2H = 1, 2


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")   # already loaded by librocm_ribn: the same runtime instance
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipSetDevice.argtypes = [ctypes.c_int]
    return hip


def test_argmax_noalloc_matches_argmax():
    hip = _hip()
    assert hip.hipSetDevice(0) == 0
    rng = np.random.default_rng(12)
    big = rng.standard_normal(151936).astype(np.float32)
    big[[5000, 90000]] = 9.0                       # tie: the lower index wins
    small = rng.standard_normal(1000).astype(np.float32)
    small[3] = np.nan                              # NaN skipped
    small[700] = 7.0
    d_in, d_out, stream = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(d_in), big.nbytes) == 0
    assert hip.hipMalloc(ctypes.byref(d_out), 4) == 0
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    err = ctypes.create_string_buffer(4096)
    try:
        for x in (big, small, big[:4097]):
            assert hip.hipMemcpy(d_in, x.ctypes.data, x.nbytes, H2D) == 0
            rc = _f(d_in, x.size, d_out, stream, err, 4096)
            assert rc == 0, err.value
            assert hip.hipStreamSynchronize(stream) == 0
            got = np.zeros(1, np.uint32)
            assert hip.hipMemcpy(got.ctypes.data, d_out, 4, D2H) == 0
            assert int(got[0]) == ribn_amd.argmax(x), (x.size, int(got[0]))
        assert ribn_amd.argmax(big) == 5000 and ribn_amd.argmax(small) == 700
        assert _f(d_in, 0, d_out, stream, err, 4096) != 0
        assert _f(d_in, 1 << 31, d_out, stream, err, 4096) != 0 and b"outside" in err.value
        assert _f(None, 10, d_out, stream, err, 4096) != 0
    finally:
        hip.hipStreamSynchronize(stream)
        hip.hipStreamDestroy(stream)
        hip.hipFree(d_in)
        hip.hipFree(d_out)
