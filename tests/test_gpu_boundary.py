"""GPU tests of the level-1 boundary: the backend vtable pair and the per-op kernel
entry points, each against the reference's own kernels (oracle/_ref), plus the
reference's two GPU self-tests restated over this library.

* qwen_gpu_selftest (qwen_tts_backend.c:195-272): W 2048x2048 bf16 (truncated
  xorshift32 values x 0.1 from seed 0x1234567), x, X[2048][8]; the CPU backend's
  matvec/matmat against the GPU backend's; the reference's pass bar is max-abs error
  over max |y| < 1e-2, held here at 1e-5 (f32 accumulation on both sides).
* --gpu-selftest-talker (main.c:1394-1432): 6 steps of LCG embeddings through the CPU
  step and the device state from an empty cache, RMS-relative error < 2e-3 per step
  (the reference's bar), and the north-star bars as well.
"""
import numpy as np
import pytest

from conftest import model_dir, need_ref, rel_l2

pytestmark = [pytest.mark.gpu, need_ref]

from qwen3_tts_amd import hip, synth  # noqa: E402


def _xorshift_unit(n, state):
    """rnd_unit of qwen_tts_backend.c:190-193 (xorshift32, 24-bit fraction to [-1, 1])."""
    vals = [0] * n
    s = state
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        vals[i] = s & 0xFFFFFF
    f = np.array(vals, np.float32) / np.float32(0xFFFFFF)
    return (f * np.float32(2.0) - np.float32(1.0)).astype(np.float32), s


def test_backend_selftest_matvec_matmat():
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    rows, cols, B = 2048, 2048, 8
    w, st = _xorshift_unit(rows * cols, 0x1234567)
    W = (((w * np.float32(0.1)).view(np.uint32)) >> 16).astype(np.uint16).reshape(rows, cols)   # f32_to_bf16_trunc
    x, st = _xorshift_unit(cols, st)
    X, st = _xorshift_unit(cols * B, st)
    X = X.reshape(cols, B)
    L = hip.lib()
    assert L.qwen_hip_available() == 1
    ctx = L.qwen_hip_init()
    assert ctx
    try:
        y_cpu = np.empty(rows, np.float32); y_gpu = np.empty(rows, np.float32)
        R.ref_matvec_bf16(y_cpu.ctypes.data, W.ctypes.data, x.ctypes.data, rows, cols)
        L.qwen_hip_matvec_bf16(ctx, y_gpu.ctypes.data, W.ctypes.data, x.ctypes.data, rows, cols)
        rel = np.abs(y_gpu - y_cpu).max() / np.abs(y_cpu).max()
        print(f"[result] selftest matvec_bf16 rel {rel:.3e}")
        assert rel < 1e-5
        Y_cpu = np.empty((rows, B), np.float32); Y_gpu = np.empty((rows, B), np.float32)
        R.ref_matmat_bf16(Y_cpu.ctypes.data, W.ctypes.data, X.ctypes.data, rows, cols, B)
        L.qwen_hip_matmat_bf16(ctx, Y_gpu.ctypes.data, W.ctypes.data, X.ctypes.data, rows, cols, B)
        rel = np.abs(Y_gpu - Y_cpu).max() / np.abs(Y_cpu).max()
        print(f"[result] selftest matmat_bf16 rel {rel:.3e}")
        assert rel < 1e-5
        # second calls reuse the device copy cached under the same host address
        y2 = np.empty(rows, np.float32); Y2 = np.empty((rows, B), np.float32)
        L.qwen_hip_matvec_bf16(ctx, y2.ctypes.data, W.ctypes.data, x.ctypes.data, rows, cols)
        L.qwen_hip_matmat_bf16(ctx, Y2.ctypes.data, W.ctypes.data, X.ctypes.data, rows, cols, B)
        assert np.array_equal(y2, y_gpu) and np.array_equal(Y2, Y_gpu)
        # a different matrix (another address) is uploaded, not confused with the cached one
        W2 = np.ascontiguousarray(W[::-1])
        y3 = np.empty(rows, np.float32); y3c = np.empty(rows, np.float32)
        L.qwen_hip_matvec_bf16(ctx, y3.ctypes.data, W2.ctypes.data, x.ctypes.data, rows, cols)
        R.ref_matvec_bf16(y3c.ctypes.data, W2.ctypes.data, x.ctypes.data, rows, cols)
        assert np.abs(y3 - y3c).max() / np.abs(y3c).max() < 1e-5
        # B = 1 equals the matvec (qwen_tts_kernels.h:110-114)
        y1 = np.empty((rows, 1), np.float32)
        L.qwen_hip_matmat_bf16(ctx, y1.ctypes.data, W.ctypes.data, x.ctypes.data, rows, cols, 1)
        assert rel_l2(y1[:, 0], y_gpu) < 1e-6
    finally:
        L.qwen_hip_free(ctx)


def test_talker_selftest_lcg_embeds():
    """main.c:1394-1432 over the 0.6B model: both sides start from an empty cache, the
    reference's RMS-rel < 2e-3 bar per step.

    On this random-init 28-layer model the bar is statistical.  Every path here agrees with
    the reference to ~2e-7 until the first K/V element whose two f32 values straddle a bf16
    truncation boundary; that one-ulp flip moves the residual by ~1e-4 and the following
    layers amplify it to 4e-4 .. 3e-3 at the last layer, depending only on where the first
    flip falls.  The per-kernel step (k_mv's bf16 order) is held to the reference's bar on
    its LCG embeddings; the default step (the role-specialised kernel's bf16 build: the
    same exact products summed in the MFMA's f32 order) is held to that bar on its first
    three layers (before the first flip, 1e-6) and, against the reference, to no more than
    the per-kernel step's deviation over 13 paired cases (these six steps and seven seeded
    two-step runs): mean ratio <= 1.25, every case <= 4e-3."""
    from oracle.oracle import RefModel
    d, s, _ = model_dir("0.6B")
    ref = RefModel(d, s, prec="bf16", threads=8)
    N, h = 6, s.hidden
    emb = np.empty(N * h, np.float32)
    r = 0x1234567
    for i in range(N * h):
        r = (r * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        emb[i] = np.float32((r >> 40) / float(1 << 24)) * np.float32(2.0) - np.float32(1.0)
    emb = emb.reshape(N, h)
    layers = hip.layers_from_ref(ref, hip.BF16)
    cos, sin = ref.rope()
    gk = hip.Talker(s, layers, ref.final_norm(), cos, sin, hip.BF16, 256)   # per-kernel steps
    gf = hip.Talker(s, layers, ref.final_norm(), cos, sin, hip.BF16, 256)   # default (fused) steps

    def rms_rel(a, c):
        return float(np.sqrt(((a.astype(np.float64) - c) ** 2).sum()) / (np.sqrt((c.astype(np.float64) ** 2).sum()) + 1e-9))

    pairs = []
    ref.kv_len = 0
    for st in range(N):
        res_r, hc = ref.step_layers(emb[st])
        hk = gk.step(emb[st], st, graph=False)
        res_f, hf = gf.step_layers(emb[st], st)
        rk, rf = rms_rel(hk, hc), rms_rel(hf, hc)
        print(f"[result] talker selftest step {st}: RMS-rel per-kernel {rk:.3e} fused {rf:.3e}, argmax cpu "
              f"{int(np.argmax(hc))} gpu {int(np.argmax(hk))} / {int(np.argmax(hf))}")
        assert rk < 2e-3
        assert np.abs(hk - hc).max() <= 2e-2 and rel_l2(hk, hc) <= 1e-3
        if st == 0:
            for l in range(3):
                assert rel_l2(res_f[l], res_r[l]) < 1e-6, (l, rel_l2(res_f[l], res_r[l]))
        pairs.append((rk, rf))
    for seed in range(7):
        rng = np.random.default_rng(100 + seed)
        e2 = rng.uniform(-1, 1, (2, h)).astype(np.float32)
        ref.kv_len = 0
        for st in range(2):
            hc = ref.step(e2[st])
            pairs.append((rms_rel(gk.step(e2[st], st, graph=False), hc), rms_rel(gf.step(e2[st], st), hc)))
    pk, pf = np.array(pairs).T
    print(f"[result] talker selftest paired: per-kernel mean {pk.mean():.3e} max {pk.max():.3e}, "
          f"fused mean {pf.mean():.3e} max {pf.max():.3e}")
    assert pf.mean() <= 1.25 * pk.mean() and pf.max() <= 4e-3 and pk.max() <= 4e-3
    gk.free()
    gf.free()


@pytest.mark.parametrize("seq,dim", [(1, 1024), (3, 2048), (2, 1000)])
def test_op_rms_norm_vs_reference(seq, dim):
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    rng = np.random.default_rng(dim + seq)
    x = (rng.standard_normal((seq, dim)) * 3).astype(np.float32)
    w = (1 + rng.standard_normal(dim) * 0.1).astype(np.float32)
    want = np.empty_like(x); got = np.empty_like(x)
    R.ref_rms_norm(want.ctypes.data, x.ctypes.data, w.ctypes.data, seq, dim, np.float32(1e-6))
    hip.check(hip.lib().qwen_hip_op_rms_norm(got.ctypes.data, x.ctypes.data, w.ctypes.data, seq, dim, np.float32(1e-6)),
              "rms_norm")
    for i in range(seq):
        assert rel_l2(got[i], want[i]) < 1e-6
        assert np.abs(got[i] - want[i]).max() < 1e-5 * np.abs(want[i]).max()


@pytest.mark.parametrize("seq,nh", [(1, 16), (1, 8), (4, 16)])
def test_op_rms_norm_per_head_vs_reference(seq, nh):
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    hd = 128
    rng = np.random.default_rng(nh * 10 + seq)
    x = rng.standard_normal((seq, nh * hd)).astype(np.float32)
    w = (1 + rng.standard_normal(hd) * 0.1).astype(np.float32)
    want = x.copy(); got = x.copy()
    R.ref_rms_norm_per_head(want.ctypes.data, w.ctypes.data, seq, nh, hd, np.float32(1e-6))
    hip.check(hip.lib().qwen_hip_op_rms_norm_per_head(got.ctypes.data, w.ctypes.data, seq, nh, hd, np.float32(1e-6)),
              "rms_norm_per_head")
    # the reference's rsqrt + Newton step (under -ffast-math) differs from a correctly
    # rounded 1/sqrt in the last bits
    assert np.abs(got - want).max() <= 4e-7 * np.abs(want).max()


@pytest.mark.parametrize("n", [3072, 6144, 1, 1000])
def test_op_swiglu_vs_reference(n):
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    rng = np.random.default_rng(n)
    gu = (rng.standard_normal(2 * n) * 4).astype(np.float32)
    gu[:8] = [0.0, 1.0, -80.0, 2.0, 80.0, -1.0, 1e-30, 3.0][: min(8, 2 * n)]
    want = gu.copy()
    R.ref_swiglu(want.ctypes.data, n)
    want = want[:n]
    got = np.empty(n, np.float32)
    hip.check(hip.lib().qwen_hip_op_swiglu(got.ctypes.data, gu.ctypes.data, n), "swiglu")
    # expf implementations differ by an ulp or two
    assert np.all(np.abs(got - want) <= 4e-7 * np.abs(want) + 1e-30)


@pytest.mark.parametrize("prec", ["bf16", "int8", "q4"])
@pytest.mark.parametrize("in_dim,out_dim", [(1024, 2048), (2048, 3072)])
def test_op_argmax_matvec_vs_reference(oracle, prec, in_dim, out_dim):
    """qwen_argmax_matvec_* (k.c:4652-4759, k.c:2620-2656): the CP's greedy lm-head pick."""
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    L = hip.lib()
    rng = np.random.default_rng(in_dim + out_dim)
    w = synth.f32_to_bf16_rne((rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32))
    for trial in range(4):
        x = rng.standard_normal(in_dim).astype(np.float32)
        if prec == "bf16":
            want = R.ref_argmax_matvec_bf16(x.ctypes.data, w.ctypes.data, in_dim, out_dim)
            got = L.qwen_hip_op_argmax_matvec(0, x.ctypes.data, w.ctypes.data, None, in_dim, out_dim)
            y = oracle.matvec(0, w, None, x, out_dim, in_dim, f64=True)
        elif prec == "int8":
            q, sc = oracle.quantize_int8(w)
            want = R.ref_argmax_matvec_int8(x.ctypes.data, q.ctypes.data, sc.ctypes.data, in_dim, out_dim)
            got = L.qwen_hip_op_argmax_matvec(1, x.ctypes.data, q.ctypes.data, sc.ctypes.data, in_dim, out_dim)
            y = oracle.matvec(1, q, sc, x, out_dim, in_dim, f64=True)
        else:
            b = oracle.quantize_q4_0(w)
            want = R.ref_argmax_matvec_q4_0(x.ctypes.data, b.ctypes.data, in_dim, out_dim)
            got = L.qwen_hip_op_argmax_matvec(2, x.ctypes.data, b.ctypes.data, None, in_dim, out_dim)
            y = oracle.matvec(2, b, None, x, out_dim, in_dim, f64=True)
        top2 = np.sort(y)[-2:]
        assert got == want or top2[1] - top2[0] < 1e-5 * abs(top2[1]), (trial, got, want)
    # ties: the lowest index wins (identical rows)
    w2 = np.tile(w[:1], (out_dim, 1))
    x = rng.standard_normal(in_dim).astype(np.float32)
    if prec == "bf16":
        assert L.qwen_hip_op_argmax_matvec(0, x.ctypes.data, w2.ctypes.data, None, in_dim, out_dim) == 0


def _glue():
    import ctypes as C
    import os
    from conftest import ROOT
    path = os.path.join(ROOT, "oracle", "_ref", "libqwen_glue.so")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref/libqwen_glue.so not built")
    G = C.CDLL(path)
    vp, i = C.c_void_p, C.c_int
    G.qwen_hip_glue_talker_init.argtypes = [vp, i]; G.qwen_hip_glue_talker_init.restype = vp
    G.qwen_hip_glue_talker_step.argtypes = [vp, vp, vp, vp]; G.qwen_hip_glue_talker_step.restype = i
    G.qwen_hip_glue_upload_kv.argtypes = [vp, vp, i]; G.qwen_hip_glue_upload_kv.restype = i
    G.qwen_hip_glue_talker_prefill.argtypes = [vp, vp, vp, i]; G.qwen_hip_glue_talker_prefill.restype = i
    G.qwen_hip_glue_cp_init.argtypes = [vp]; G.qwen_hip_glue_cp_init.restype = vp
    G.qwen_hip_glue_cp_predict.argtypes = [vp, vp, i, vp]; G.qwen_hip_glue_cp_predict.restype = i
    G.qwen_hip_glue_cp_step.argtypes = [vp, vp, vp, i]; G.qwen_hip_glue_cp_step.restype = i
    return G


@pytest.mark.parametrize("name,prec", [("mini", "int8"), ("mini17", "int4"), ("mini17", "bf16")])
def test_glue_drives_reference_ctx(name, prec):
    """The reference-side glue over a ctx the reference loaded (ref_harness builds it the
    way qwen_tts_load_ex does): Talker init from the ctx's layers at their precision,
    the CPU prefill handed over with upload_kv, steps through the qwen_talker_step hook
    (kv_len and dec_x bookkeeping), the device prefill, and the CP frame in front of
    qwen_cp_predict -- each against a second reference ctx of the same weights running
    the reference's own functions."""
    import ctypes as C
    from oracle.oracle import RefModel
    print(f"[case] glue {name} {prec}", flush=True)
    G = _glue()
    d, s, _ = model_dir(name)
    cpu = RefModel(d, s, prec=prec, threads=8)       # the reference's own path
    dev = RefModel(d, s, prec=prec, threads=8)       # the ctx the glue drives
    ctx = dev.lib.ref_ctx(dev.h)
    st = G.qwen_hip_glue_talker_init(ctx, 512)
    assert st, hip.last_error()
    emb = cpu.codec_emb()
    rng = np.random.default_rng(12)
    E = synth.bf16_to_f32(emb[rng.integers(0, 2048, 20)]).astype(np.float32)
    # CPU prefill of 20 positions on both ctxs, the device gets it through upload_kv
    cpu.kv_len = 0
    dev.kv_len = 0
    cpu.prefill(E)
    dev.prefill(E)
    assert G.qwen_hip_glue_upload_kv(st, ctx, 20) == 0
    for i in range(6):
        e = synth.bf16_to_f32(emb[int(rng.integers(0, 2048))]).astype(np.float32)
        h_c = cpu.step(e)
        h_g = np.empty(s.hidden, np.float32)
        assert G.qwen_hip_glue_talker_step(st, ctx, e.ctypes.data, h_g.ctypes.data) == 0
        assert dev.kv_len == cpu.kv_len == 21 + i
        _ = _check(h_g, h_c, f"glue step {i}")
        _ = _check(dev.dec_x(), cpu.dec_x(), f"glue dec_x {i}")
    # the device prefill through the glue: dec_x and kv_len like qwen_talker_prefill's
    cpu.kv_len = 0
    dx_c = cpu.prefill(E)
    assert G.qwen_hip_glue_talker_prefill(st, ctx, E.ctypes.data, 20) == 0
    assert dev.kv_len == 20
    _check(dev.dec_x(), dx_c, "glue prefill dec_x")
    hip.lib().qwen_hip_talker_free(st)
    # CP frame
    cp = G.qwen_hip_glue_cp_init(ctx)
    assert cp, hip.last_error()
    for f in range(3):
        th = rng.standard_normal(s.hidden).astype(np.float32)
        th /= np.sqrt((th ** 2).mean())
        code0 = int(rng.integers(0, 2048))
        out = (C.c_int * 15)()
        assert G.qwen_hip_glue_cp_predict(cp, th.ctypes.data, code0, out) == 0
        assert list(out) == list(cpu.cp_predict(th, code0)), f
    hip.lib().qwen_hip_cp_free(cp)


def _check(a, b, tag):
    assert np.abs(a - b).max() <= 2e-2, tag
    r = rel_l2(a, b)
    assert r <= 1e-3, (tag, r)
    return r


def test_backend_vtable_hip_kind_through_reference_dispatch():
    """The HIP kind of the reference's backend vtable (qwen_tts_backend.h:34-49), as the
    glue builds it (qwen_hip_glue_backend_new), installed with the reference's own
    qwen_backend_install_global (qwen_tts_backend.c:157-174) and driven through the
    reference's dispatch: qwen_matvec_bf16, the fused bf16 QKV matvec and qwen_matmat_bf16
    (qwen_tts_kernels.c:1091-1092, 2094-2101, 1327-1328) reach the device, equal the
    vtable's own calls to the bit, and agree with the reference's CPU path (run before the
    install and after the uninstall) within float-order tolerance."""
    import ctypes as C
    print("[case] backend vtable (HIP kind) via qwen_backend_install_global", flush=True)
    G = _glue()
    vp, i = C.c_void_p, C.c_int

    class Backend(C.Structure):
        _fields_ = [("kind", C.c_int), ("name", C.c_char_p), ("impl", vp),
                    ("matvec_bf16", vp), ("matmat_bf16", vp), ("free", vp)]

    G.qwen_hip_glue_backend_new.restype = C.POINTER(Backend)
    G.qwen_backend_install_global.argtypes = [C.POINTER(Backend)]
    G.qwen_matvec_bf16.argtypes = [vp, vp, vp, i, i]
    G.qwen_matmat_bf16.argtypes = [vp, vp, vp, i, i, i]
    G.qwen_matvec_bf16_qkv.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i, i]
    MV = C.CFUNCTYPE(None, C.POINTER(Backend), vp, vp, vp, i, i)
    MM = C.CFUNCTYPE(None, C.POINTER(Backend), vp, vp, vp, i, i, i)
    FR = C.CFUNCTYPE(None, C.POINTER(Backend))
    b = G.qwen_hip_glue_backend_new()
    assert b, "no HIP backend"
    assert b.contents.kind == 3 and b.contents.name == b"hip"
    rng = np.random.default_rng(11)
    rows, cols, B = 1000, 2048, 7
    W = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    X = rng.standard_normal((cols, B)).astype(np.float32)
    qd, kvd = 512, 256
    Wq = synth.f32_to_bf16_rne((rng.standard_normal((qd, cols)) * 0.02).astype(np.float32))
    Wk = synth.f32_to_bf16_rne((rng.standard_normal((kvd, cols)) * 0.02).astype(np.float32))
    Wv = synth.f32_to_bf16_rne((rng.standard_normal((kvd, cols)) * 0.02).astype(np.float32))

    def through_dispatch():
        y, Y = np.empty(rows, np.float32), np.empty((rows, B), np.float32)
        q, k, v = np.empty(qd, np.float32), np.empty(kvd, np.float32), np.empty(kvd, np.float32)
        G.qwen_matvec_bf16(y.ctypes.data, W.ctypes.data, x.ctypes.data, rows, cols)
        G.qwen_matmat_bf16(Y.ctypes.data, W.ctypes.data, X.ctypes.data, rows, cols, B)
        G.qwen_matvec_bf16_qkv(q.ctypes.data, k.ctypes.data, v.ctypes.data, Wq.ctypes.data, Wk.ctypes.data,
                               Wv.ctypes.data, x.ctypes.data, cols, qd, kvd)
        return y, Y, q, k, v

    cpu = through_dispatch()                          # no hook: the reference's CPU kernels
    try:
        y_vt, Y_vt = np.empty(rows, np.float32), np.empty((rows, B), np.float32)
        MV(b.contents.matvec_bf16)(b, y_vt.ctypes.data, W.ctypes.data, x.ctypes.data, rows, cols)
        MM(b.contents.matmat_bf16)(b, Y_vt.ctypes.data, W.ctypes.data, X.ctypes.data, rows, cols, B)
        G.qwen_backend_install_global(b)
        dev = through_dispatch()
    finally:
        G.qwen_backend_install_global(None)
    again = through_dispatch()                        # uninstalled: the CPU path again
    FR(b.contents.free)(b)
    assert np.array_equal(dev[0], y_vt) and np.array_equal(dev[1], Y_vt)
    for a, c in zip(again, cpu):
        assert np.array_equal(a, c)
    for got, want in zip(dev, cpu):
        err = rel_l2(got, want)
        print(f"[result] vtable dispatch vs reference CPU: rel-L2 {err:.2e}")
        assert err <= 1e-5
