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


def test_noalloc_under_graph_capture(oracle):
    """The call recorded on a created stream inside hipStreamBeginCapture in global mode
    (where HIP refuses hipMalloc from any thread), the graph instantiated and replayed three
    times with eager work and host synchronisation between the replays; every replay equals
    qwen_hip_op_matmat_int8 to the bit."""
    print("[case] matmat_int8_noalloc under stream capture: 1024x2048 B=8, 3 replays", flush=True)
    L = hip.lib()
    dev = _Dev()
    rt = dev.rt
    rt.hipStreamCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
    rt.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    rt.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    rt.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    rt.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    rt.hipStreamSynchronize.argtypes = [C.c_void_p]
    rt.hipGraphExecDestroy.argtypes = [C.c_void_p]
    rt.hipGraphDestroy.argtypes = [C.c_void_p]
    rt.hipStreamDestroy.argtypes = [C.c_void_p]
    rt.hipMemsetAsync.argtypes = [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p]
    rows, cols, B = 1024, 2048, 8
    rng = np.random.default_rng(7)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    q, s = oracle.quantize_int8(w)
    X = rng.standard_normal((cols, B)).astype(np.float32)
    want = np.empty((rows, B), np.float32)
    hip.check(L.qwen_hip_op_matmat_int8(want.ctypes.data, q.ctypes.data, s.ctypes.data, X.ctypes.data, rows, cols, B),
              "matmat_int8")
    st, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    try:
        dW, dS, dX = dev.put(q), dev.put(s), dev.put(np.ascontiguousarray(X.T))
        dY = dev.empty(rows * B * 4)
        assert rt.hipStreamCreateWithFlags(C.byref(st), 1) == 0          # hipStreamNonBlocking, default priority
        # an eager call on the stream first (the device's array address is looked up here)
        assert L.qwen_hip_op_matmat_int8_noalloc(dY, dW, dS, dX, rows, cols, B, st) == 0, hip.last_error()
        assert rt.hipStreamSynchronize(st) == 0
        assert np.array_equal(dev.get(dY, np.empty((B, rows), np.float32)).T, want)
        assert rt.hipStreamBeginCapture(st, 0) == 0                      # hipStreamCaptureModeGlobal
        rc = L.qwen_hip_op_matmat_int8_noalloc(dY, dW, dS, dX, rows, cols, B, st)
        err = hip.last_error() if rc else ""
        assert rt.hipStreamEndCapture(st, C.byref(graph)) == 0
        assert rc == 0, err
        assert rt.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for rep in range(3):
            # eager work between replays: clear the output on the same stream
            assert rt.hipMemsetAsync(dY, 0, rows * B * 4, st) == 0
            assert rt.hipStreamSynchronize(st) == 0
            assert rt.hipGraphLaunch(exe, st) == 0
            assert rt.hipStreamSynchronize(st) == 0
            got = dev.get(dY, np.empty((B, rows), np.float32))
            assert np.array_equal(got.T, want), f"replay {rep}"
    finally:
        if exe.value:
            rt.hipGraphExecDestroy(exe)
        if graph.value:
            rt.hipGraphDestroy(graph)
        if st.value:
            rt.hipStreamDestroy(st)
        dev.free()
