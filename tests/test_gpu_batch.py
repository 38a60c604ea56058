"""GPU parity of the batched (B-stream, ragged) step and its MFMA projection.

Oracle: the C restatement (oracle/), one independent decode per stream on that
stream's own KV cache, over the reference-loaded weights (oracle_talker).  The
reference's batched step computes exactly these per-stream single steps
(qwen_tts_talker.c:1192-1270: per-sequence norm/RoPE/KV/attention, weights shared), so
each stream is held to the north-star tolerance (max-abs 2e-2, rel-L2 1e-3 of the
hidden state) and its KV rows to the single-step KV checks.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import model_dir, need_ref, rel_l2

pytestmark = pytest.mark.gpu

from qwen3_tts_amd import hip, synth  # noqa: E402


def _matmat(q, s, X):
    rows, cols = q.shape
    B = X.shape[1]
    Y = np.empty((rows, B), np.float32)
    Xc = np.ascontiguousarray(X, np.float32)
    hip.check(hip.lib().qwen_hip_op_matmat_int8(Y.ctypes.data, q.ctypes.data, s.ctypes.data, Xc.ctypes.data,
                                               rows, cols, B), "matmat_int8")
    return Y


@pytest.mark.parametrize("rows,cols,B", [(16, 64, 1), (64, 2048, 32), (4096, 1024, 16), (2048, 6144, 32),
                                         (257, 320, 5), (100, 2048, 33), (48, 8192, 64), (12288, 2048, 8)])
def test_op_matmat_int8(oracle, rows, cols, B):
    """Y = (W*scale) @ X against the f64 product of the dequantised weights: the exact
    int8-piece contraction leaves only the activation split (|e| <= max|x| 2^-20) and
    the final roundings."""
    print(f"[case] matmat int8 {rows}x{cols} B={B}", flush=True)
    rng = np.random.default_rng(rows + cols + B)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    q, s = oracle.quantize_int8(w)
    X = rng.standard_normal((cols, B)).astype(np.float32)
    X[:, 0] *= 1e-3                                     # streams of very different magnitude
    if B > 2:
        X[:, 2] = 0.0                                   # an all-zero stream
    Y = _matmat(q, s, X)
    Wf = q.astype(np.float64) * s.astype(np.float64)[:, None]
    Y64 = Wf @ X.astype(np.float64)
    for j in range(B):
        den = np.abs(Y64[:, j]).max()
        if den == 0:
            assert np.all(Y[:, j] == 0)
            continue
        err = np.abs(Y[:, j] - Y64[:, j]).max() / den
        assert err < 1e-5, (j, err)


def test_op_matmat_int8_exact_inputs(oracle):
    """Activations that the three int8 planes hold exactly (multiples of 2^-14 of a
    power-of-two scale): the product is the exact dot product rounded once, so it
    equals the f64 result rounded to f32 (times the row scale)."""
    rows, cols, B = 64, 2048, 16
    rng = np.random.default_rng(4)
    q = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
    s = np.ones(rows, np.float32)
    X = (rng.integers(-(1 << 20), 1 << 20, (cols, B)) * 2.0 ** -14).astype(np.float32)   # |x| < 64
    Y = _matmat(q, s, X)
    exact = q.astype(np.float64) @ X.astype(np.float64)
    assert np.array_equal(Y, exact.astype(np.float32))


def test_op_matmat_int8_tiny_negative_activations(oracle):
    """Activations just below zero next to O(1) ones (SwiGLU outputs of very negative
    gates): y = x/s in (-2^-25, 0) makes y - floor(y) round up to 1.0 in f32, which once
    turned piece plane 2 into 128 (an int8 -128, an error of 2s on that element).  Every
    stream, and each of the four tall-tile / split-K plans (K = 1024, 2048, 3072, 6144),
    against the f64 product."""
    rng = np.random.default_rng(0x71C)
    for rows, cols, B in [(64, 1024, 32), (256, 2048, 32), (128, 3072, 16), (2048, 6144, 32)]:
        print(f"[case] matmat int8 tiny negatives {rows}x{cols} B={B}", flush=True)
        w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        q, s = oracle.quantize_int8(w)
        X = rng.standard_normal((cols, B)).astype(np.float32)
        tiny = rng.random((cols, B)) < 0.25
        X[tiny] = -(rng.random(int(tiny.sum())) * 1e-9 + 1e-12).astype(np.float32)
        Y = _matmat(q, s, X)
        Y64 = (q.astype(np.float64) * s.astype(np.float64)[:, None]) @ X.astype(np.float64)
        for j in range(B):
            err = np.abs(Y[:, j] - Y64[:, j]).max() / np.abs(Y64[:, j]).max()
            assert err < 1e-5, (rows, cols, j, err)


def test_op_matmat_matches_matvec_per_column(oracle):
    """Each column of the batched product is the single-stream matvec of that column
    (qwen_tts_kernels.h:117-122: 'with B==1 it equals matvec'), to the f32 rounding of
    the matvec's own 3072-term accumulation."""
    rows, cols, B = 1024, 3072, 6
    rng = np.random.default_rng(9)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    q, s = oracle.quantize_int8(w)
    X = rng.standard_normal((cols, B)).astype(np.float32)
    Y = _matmat(q, s, X)
    for j in range(B):
        y = np.empty(rows, np.float32)
        xj = np.ascontiguousarray(X[:, j])
        hip.check(hip.lib().qwen_hip_op_matvec_int8(y.ctypes.data, q.ctypes.data, s.ctypes.data,
                                                   xj.ctypes.data, rows, cols), "mv")
        assert rel_l2(Y[:, j], y) < 5e-6


def _matmat_q4(blocks, rows, cols, X):
    B = X.shape[1]
    Y = np.empty((rows, B), np.float32)
    Xc = np.ascontiguousarray(X, np.float32)
    hip.check(hip.lib().qwen_hip_op_matmat_q4_0(Y.ctypes.data, blocks.ctypes.data, Xc.ctypes.data, rows, cols, B),
              "matmat_q4_0")
    return Y


@pytest.mark.parametrize("rows,cols,B", [(16, 64, 1), (64, 2048, 32), (4096, 1024, 16), (2048, 6144, 32),
                                         (257, 320, 5), (100, 2048, 33), (48, 8192, 64), (12288, 2048, 8)])
def test_op_matmat_q4_0(oracle, rows, cols, B):
    """Y = dequant(W_q4) @ X (weights read once for all B columns) against the f64 product
    of the dequantised weights (oracle dequant_q4_0, k.c:2810-2819): each block's dot
    product is an exact integer sum rounded once, so only f32 roundings remain."""
    print(f"[case] matmat q4_0 {rows}x{cols} B={B}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + B)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    blocks = oracle.quantize_q4_0(w)
    X = rng.standard_normal((cols, B)).astype(np.float32)
    X[:, 0] *= 1e-3
    if B > 2:
        X[:, 2] = 0.0
    Y = _matmat_q4(blocks, rows, cols, X)
    Wf = oracle.dequant_q4_0(blocks, rows, cols).astype(np.float64)
    Y64 = Wf @ X.astype(np.float64)
    for j in range(B):
        den = np.abs(Y64[:, j]).max()
        if den == 0:
            assert np.all(Y[:, j] == 0)
            continue
        err = np.abs(Y[:, j] - Y64[:, j]).max() / den
        assert err < 1e-5, (j, err)


def test_op_matmat_q4_0_exact_inputs(oracle):
    """Power-of-two block scales (the second block of each row scaled by zero) and
    activations that the int8 planes hold exactly: every block's integer dot product, its
    conversion and its scaling are exact, so Y equals the f64 product."""
    rows, cols, B = 32, 64, 16
    rng = np.random.default_rng(5)
    nib = rng.integers(0, 16, (rows, cols))
    blocks = np.zeros((rows, cols // 32, 18), np.uint8)
    for r in range(rows):
        for j in range(cols // 32):
            e = int(rng.integers(-6, 3))
            h = np.float16(2.0 ** e) if j == 0 else np.float16(0.0)
            blocks[r, j, :2] = np.frombuffer(h.tobytes(), np.uint8)
            q = nib[r, 32 * j:32 * j + 32]
            blocks[r, j, 2:] = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    X = (rng.integers(-(1 << 14), 1 << 14, (cols, B)) * 2.0 ** -10).astype(np.float32)
    Y = _matmat_q4(blocks, rows, cols, X)
    Wf = oracle.dequant_q4_0(blocks.reshape(-1), rows, cols).astype(np.float64)
    assert np.array_equal(Y, (Wf @ X.astype(np.float64)).astype(np.float32))


# ------------------------------------------------------------------ batched Talker step

def _ref(name, prec):
    from oracle.oracle import RefModel
    d, shape, _ = model_dir(name)
    return RefModel(d, shape, prec=prec, threads=8), shape


def _streams(ref, prec_code, B, kv_max):
    from oracle.oracle import oracle_talker
    return [oracle_talker(ref, prec_code, kv_max) for _ in range(B)]


@need_ref
@pytest.mark.parametrize("prec,B", [("int8", 5), ("int8", 32), ("bf16", 3), ("bf16", 32), ("int4", 2), ("int4", 17), ("int4", 32)])
def test_batch_step_ragged_vs_oracle(oracle, prec, B):
    """B streams prefilled to different lengths (upload_slot), then stepped together,
    each at its own position; every stream against its own oracle decode."""
    print(f"[case] batch step {prec} B={B}", flush=True)
    ref, shape = _ref("mini", prec)
    pc = hip.PREC[prec]
    kv_max = 96
    layers = hip.layers_from_ref(ref, pc)
    cos, sin = ref.rope()
    g = hip.Talker(shape, layers, ref.final_norm(), cos, sin, pc, kv_max)
    bt = hip.TalkerBatch(g, B)
    streams = _streams(ref, pc, B, kv_max)
    emb = ref.codec_emb()
    rng = np.random.default_rng(100 + B)
    pre = [int(rng.integers(0, 40)) for _ in range(B)]
    pre[0] = 0
    H, L, kvd = shape.hidden, shape.layers, shape.kv_dim
    kvk = np.zeros((B, L, kv_max, kvd), np.uint16)
    kvv = np.zeros_like(kvk)
    for b in range(B):
        t, keep = streams[b]
        for p in range(pre[b]):
            oracle.talker_step(t, synth.bf16_to_f32(emb[int(rng.integers(0, 2048))]), p)
        kvk[b], kvv[b] = keep["kv_k"], keep["kv_v"]
    for b in range(B):
        bt.upload_slot(b, kvk, kvv, pre[b])
        if pre[b]:
            k2, v2 = bt.download_slot(b, pre[b])
            assert np.array_equal(k2[:, :pre[b]], kvk[b][:, :pre[b]]) and np.array_equal(v2[:, :pre[b]], kvv[b][:, :pre[b]])
    pos = np.array(pre, np.int32)
    worst = 0.0
    for it in range(6):
        E = np.stack([synth.bf16_to_f32(emb[int(rng.integers(0, 2048))]) for _ in range(B)])
        got = bt.step(E, pos)
        for b in range(B):
            want, _ = oracle.talker_step(streams[b][0], E[b], int(pos[b]))
            assert np.abs(got[b] - want).max() <= 2e-2, (it, b)
            err = rel_l2(got[b], want)
            assert err <= 1e-3, (it, b, err)
            worst = max(worst, err)
        pos += 1
    # KV rows written by the batched step: truncated bf16 of the stream's own k/v
    for b in range(B):
        n = int(pos[b])
        kg, vg = bt.download_slot(b, n)
        kr, vr = streams[b][1]["kv_k"], streams[b][1]["kv_v"]
        for a_, b_ in [(kg, kr), (vg, vr)]:
            fa, fb = synth.bf16_to_f32(a_[:, :n]), synth.bf16_to_f32(b_[:, :n])
            num = np.linalg.norm((fa - fb).astype(np.float64), axis=-1)
            den = np.linalg.norm(fb.astype(np.float64), axis=-1)
            assert (num <= 1e-2 * den + 1e-6).all(), float((num / np.maximum(den, 1e-30)).max())
    print(f"[result] batch {prec} B={B}: worst hidden rel-L2 {worst:.2e}")
    bt.free()
    g.free()


@need_ref
def test_batch_of_identical_streams_matches_single_step():
    """B copies of one stream (the reference's batch self-test, cu:657-730 /
    t.c:1301-1402): every row equals the single-state step to the tolerance."""
    ref, shape = _ref("mini", "int8")
    layers = hip.layers_from_ref(ref, hip.INT8)
    cos, sin = ref.rope()
    g = hip.Talker(shape, layers, ref.final_norm(), cos, sin, hip.INT8, 64)
    B = 4
    bt = hip.TalkerBatch(g, B)
    emb = ref.codec_emb()
    for pos in range(8):
        e = synth.bf16_to_f32(emb[pos * 41 + 3])
        single = g.step(e, pos)
        got = bt.step(np.tile(e, (B, 1)), np.full(B, pos, np.int32))
        # rows of the batch are bit-identical to each other; against the single step
        # (VALU f32 sums) they differ by f32 rounding, which can flip a truncated bf16
        # K/V bit (2^-8 relative) and so reach ~1e-4 after 2 layers
        for b in range(B):
            assert np.array_equal(got[b], got[0])
            assert rel_l2(got[b], single) <= 1e-3, (pos, rel_l2(got[b], single))
    bt.free()
    g.free()


@need_ref
@pytest.mark.parametrize("B", [5, 20, 32])
def test_batch_fold_pieces_matches_separate_launch(B):
    """int8: the activation pieces made inside each projection launch (the default) and
    in a launch of their own are the same bytes, so the outputs are the same bit for bit:
    every layer's residual (ungraphed step) and the graphed step's hidden state.  B = 5 and
    20 have padding streams (16 and 32 columns)."""
    print(f"[case] fold pieces B={B}", flush=True)
    ref, shape = _ref("mini", "int8")
    layers = hip.layers_from_ref(ref, hip.INT8)
    cos, sin = ref.rope()
    g = hip.Talker(shape, layers, ref.final_norm(), cos, sin, hip.INT8, 64)
    bt = hip.TalkerBatch(g, B)
    assert bt.fold_pieces(True)
    emb = ref.codec_emb()
    rng = np.random.default_rng(7 + B)
    pos = rng.integers(0, 40, B).astype(np.int32)
    for it in range(3):
        E = np.stack([synth.bf16_to_f32(emb[int(rng.integers(0, 2048))]) for _ in range(B)])
        assert bt.fold_pieces(True)
        r1, h1 = bt.step_layers(E, pos)
        g1 = bt.step(E, pos)
        assert not bt.fold_pieces(False)
        r2, h2 = bt.step_layers(E, pos)     # same position: rewrites the same KV rows
        g2 = bt.step(E, pos)
        assert np.array_equal(r1, r2) and np.array_equal(h1, h2), it
        assert np.array_equal(g1, g2) and np.array_equal(g1, h1), it
        pos += 1
    bt.free()
    g.free()


def test_batch_rejects_bad_arguments():
    shape = synth.SHAPES["tiny"]
    t = synth.generate(shape, 0x5EED0009, 0.0, threads=4, only=lambda n: n.startswith("talker.model."))
    layers = hip.layers_from_tensors(t, shape)
    cos, sin = synth.rope_tables(shape.head_dim, shape.rope_theta, 32)
    g = hip.Talker(shape, layers, synth.bf16_to_f32(t["talker.model.norm.weight"]), cos, sin, hip.BF16, 32,
                   quantize_to=hip.INT8)
    L = hip.lib()
    assert not L.qwen_hip_talker_batch_init(g.h, 0)
    assert not L.qwen_hip_talker_batch_init(g.h, 65)
    assert not L.qwen_hip_talker_batch_init(None, 4)
    bt = hip.TalkerBatch(g, 2)
    E = np.zeros((2, shape.hidden), np.float32)
    with pytest.raises(RuntimeError):
        bt.step(E, np.array([0, 32], np.int32))        # position past kv_max
    bt.free()
    g.free()


@need_ref
@pytest.mark.parametrize("prec", ["bf16", "int8"])
def test_cp_batch_step_vs_oracle(oracle, prec):
    """CP batch twin: B residual streams, one 2-layer pass each at its own position,
    against the oracle's CP pass per stream."""
    from test_gpu_parity import _gpu_cp
    from oracle.oracle import oracle_talker
    ref, shape = _ref("mini", prec)
    pc = hip.PREC[prec]
    cp = _gpu_cp(ref, shape, pc)
    B = 6
    streams = [oracle_talker(ref, pc, 64, cp=True) for _ in range(B)]
    rng = np.random.default_rng(3)
    for p in range(5):
        x = rng.standard_normal((B, shape.cp_hidden)).astype(np.float32)
        got = cp.batch_step(x, np.full(B, p, np.int32))
        for b in range(B):
            want = np.array(x[b], copy=True)
            assert oracle.lib.qo_cp_pass(C.byref(streams[b][0]), want.ctypes.data, p) == 0
            assert rel_l2(got[b], want) <= 1e-3, (p, b, rel_l2(got[b], want))
    cp.free()


@need_ref
def test_cp_prefill2_vs_oracle_and_reference(oracle):
    """Two-position prefill (cp_prefill2, qwen_tts_code_predictor.c:816-902): the
    two-column pass against two sequential oracle passes at positions 0 and 1 (the
    reference's own definition: 'the same math', its matmat only reorders rounding),
    then whole frames with the prefill on against the compiled reference's
    qwen_cp_predict with QWEN_CP_PREFILL2=1 (its mode is probed once per thread, so the
    reference runs in a fresh thread)."""
    import os
    import threading
    from test_gpu_parity import _gpu_cp
    from oracle.oracle import oracle_talker
    print("[case] cp prefill2 int8", flush=True)
    ref, shape = _ref("mini", "int8")
    cp = _gpu_cp(ref, shape, hip.INT8)
    with pytest.raises(RuntimeError):
        cp.prefill2(np.zeros(shape.cp_hidden, np.float32), np.zeros(shape.cp_hidden, np.float32))   # not enabled
    cp.set_prefill2(1)
    rng = np.random.default_rng(21)
    for trial in range(3):
        x0 = rng.standard_normal(shape.cp_hidden).astype(np.float32)
        x1 = rng.standard_normal(shape.cp_hidden).astype(np.float32)
        g0, g1 = cp.prefill2(x0, x1)
        t, _ = oracle_talker(ref, hip.INT8, 64, cp=True)
        w0, w1 = np.array(x0, copy=True), np.array(x1, copy=True)
        assert oracle.lib.qo_cp_pass(C.byref(t), w0.ctypes.data, 0) == 0
        assert oracle.lib.qo_cp_pass(C.byref(t), w1.ctypes.data, 1) == 0
        for g, w in [(g0, w0), (g1, w1)]:
            assert np.abs(g - w).max() <= 2e-2 and rel_l2(g, w) <= 1e-3, (trial, rel_l2(g, w))
    frames = []
    for f in range(4):
        th = rng.standard_normal(shape.hidden).astype(np.float32)
        th /= np.sqrt((th ** 2).mean())
        frames.append((th, int(rng.integers(0, 2048))))
    got = [list(cp.frame(th, c0)) for th, c0 in frames]
    want = []
    old = os.environ.get("QWEN_CP_PREFILL2")
    os.environ["QWEN_CP_PREFILL2"] = "1"
    try:
        th_ = threading.Thread(target=lambda: want.extend(list(ref.cp_predict(th, c0)) for th, c0 in frames))
        th_.start()
        th_.join()
    finally:
        if old is None:
            del os.environ["QWEN_CP_PREFILL2"]
        else:
            os.environ["QWEN_CP_PREFILL2"] = old
    assert len(want) == len(frames)
    assert got == want, (got, want)
    cp.set_prefill2(0)                                  # back to sequential passes
    assert [list(cp.frame(th, c0)) for th, c0 in frames] == [list(ref.cp_predict(th, c0)) for th, c0 in frames]
    cp.free()


@need_ref
def test_cp_prefill2_needs_int8():
    from test_gpu_parity import _gpu_cp
    ref, shape = _ref("mini", "bf16")
    cp = _gpu_cp(ref, shape, hip.BF16)
    with pytest.raises(RuntimeError):
        cp.set_prefill2(1)
    cp.free()
