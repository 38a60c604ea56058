"""qwen_hip_op_matmat_int8_noalloc: the batched int8 projection on the caller's device
buffers with its scratch (activation pieces + scales) in a file-scope device array, so
the call allocates nothing.  Checked against qwen_hip_op_matmat_int8 (same kernels, host
buffers) to the bit, on two calls in a row, the second with a smaller input (the array
keeps the first call's bytes), plus the size limit's error path."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from qwen3_tts_amd import hip, synth  # noqa: E402


class _Dev:
    """Device buffers for the test (the test may allocate; the entry point does not)."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipDeviceSynchronize.argtypes = []
        self.bufs = []

    def put(self, a):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), a.nbytes) == 0
        self.bufs.append(p)
        assert self.rt.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0      # host to device
        return p

    def empty(self, nbytes):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), nbytes) == 0
        self.bufs.append(p)
        return p

    def get(self, p, a):
        assert self.rt.hipMemcpy(a.ctypes.data, p, a.nbytes, 2) == 0      # device to host
        return a

    def free(self):
        for p in self.bufs:
            self.rt.hipFree(p)
        self.bufs = []


def _case(oracle, dev, rows, cols, B, seed):
    L = hip.lib()
    rng = np.random.default_rng(seed)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    q, s = oracle.quantize_int8(w)
    X = rng.standard_normal((cols, B)).astype(np.float32)
    X[:, 0] *= 1e-3
    want = np.empty((rows, B), np.float32)
    hip.check(L.qwen_hip_op_matmat_int8(want.ctypes.data, q.ctypes.data, s.ctypes.data, X.ctypes.data, rows, cols, B),
              "matmat_int8")
    Xs = np.ascontiguousarray(X.T)                      # stream-major [B][cols]
    dW, dS, dX = dev.put(q), dev.put(s), dev.put(Xs)
    dY = dev.empty(rows * B * 4)
    rc = L.qwen_hip_op_matmat_int8_noalloc(dY, dW, dS, dX, rows, cols, B, None)
    assert rc == 0, hip.last_error()
    assert dev.rt.hipDeviceSynchronize() == 0
    got = dev.get(dY, np.empty((B, rows), np.float32))
    assert np.array_equal(got.T, want)
    return got


def test_noalloc_matches_allocating_entry_point(oracle):
    print("[case] matmat_int8_noalloc: 2048x6144 B=32, then 300x2048 B=5", flush=True)
    dev = _Dev()
    try:
        _case(oracle, dev, 2048, 6144, 32, 1)
        _case(oracle, dev, 300, 2048, 5, 2)           # smaller: stale bytes of the first call stay in the array
    finally:
        dev.free()


def test_noalloc_rejects_oversize():
    L = hip.lib()
    one = C.c_void_p(16)                                 # never dereferenced: the shape check fails first
    assert L.qwen_hip_op_matmat_int8_noalloc(one, one, one, one, 64, 8256, 4, None) == -1
    assert "8192" in hip.last_error()
    assert L.qwen_hip_op_matmat_int8_noalloc(one, one, one, one, 64, 1024, 65, None) == -1
    assert L.qwen_hip_op_matmat_int8_noalloc(one, one, one, one, 64, 1000, 4, None) == -1
