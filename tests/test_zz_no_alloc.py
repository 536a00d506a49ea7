"""The allocation-free matvec (hg_q8_tensor_matvec_noalloc): device pointers in and out, its
activation scratch in a fixed library-held device array, results bit-identical to
hg_q8_tensor_matvec.  Calls in a row, each later one with a smaller input, so stale scratch
contents of an earlier call would show in a later one.

Device buffers and the stream come from the HIP runtime the library itself uses (the test's
plumbing; the entry point allocates nothing)."""
import ctypes as C

import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs

pytestmark = pytest.mark.gpu
H2D, D2H = 1, 2


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def hip():
    import hobbylm_amd as hg
    hg.lib()                       # loads libamdhip64 (the runtime the library is linked to)
    rt = C.CDLL("libamdhip64.so.7")
    for fn in ("hipMalloc", "hipFree", "hipMemcpy", "hipStreamCreate", "hipStreamDestroy",
               "hipStreamSynchronize"):
        getattr(rt, fn).restype = C.c_int
    rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    rt.hipFree.argtypes = [C.c_void_p]
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rt.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
    rt.hipStreamDestroy.argtypes = [C.c_void_p]
    rt.hipStreamSynchronize.argtypes = [C.c_void_p]
    return rt


def _dev(hip, nbytes):
    p = C.c_void_p()
    assert hip.hipMalloc(C.byref(p), nbytes) == 0
    return p


def test_noalloc_matvec_matches_matvec(hip):
    import hobbylm_amd as hg
    rng = np.random.default_rng(17)
    st = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(st)) == 0
    # (out, in): the largest input first, then smaller ones (a partial last chunk at 544)
    for n, k in [(64, 32768), (1024, 4096), (300, 544)]:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        t = hg.Q8Tensor.from_q8_0(gs.quantize_q8_0(w), n, k)
        want = t.matvec(x)
        xd, yd = _dev(hip, 4 * k), _dev(hip, 4 * n)
        nan = np.full(n, np.nan, np.float32)
        assert hip.hipMemcpy(xd, x.ctypes.data_as(C.c_void_p), 4 * k, H2D) == 0
        assert hip.hipMemcpy(yd, nan.ctypes.data_as(C.c_void_p), 4 * n, H2D) == 0
        for rep in range(2):   # the same call twice on the shared scratch
            t.matvec_noalloc(xd.value, yd.value, st.value)
            assert hip.hipStreamSynchronize(st) == 0
            got = np.empty(n, np.float32)
            assert hip.hipMemcpy(got.ctypes.data_as(C.c_void_p), yd, 4 * n, D2H) == 0
            assert _bits_equal(got, want), (n, k, rep)
        hip.hipFree(xd)
        hip.hipFree(yd)
        t.close()
    hip.hipStreamDestroy(st)


def test_noalloc_rejects_inputs_beyond_the_scratch():
    import hobbylm_amd as hg
    w = np.zeros((8, 32768 + 32), np.float32)
    t = hg.Q8Tensor.quantize(w)
    with pytest.raises(hg.HgError, match="maximum"):
        t.matvec_noalloc(1, 1, 0)   # refused before any launch: the pointers are never used
    t.close()
