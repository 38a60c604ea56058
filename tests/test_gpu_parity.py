"""GPU parity: the HIP library (through its C ABI) against the reference engine built
from its own sources (oracle/_ref) and against the C restatement (oracle/).

Tolerances (north star): per-layer hidden states max-abs <= 2e-2 and rel-L2 <= 1e-3
of the reference CPU path; quantized weights and the KV append bit-exact; greedy codec
tokens identical.  Kernel-level checks are tighter (f64 brute force, rel 2e-5).
"""
import numpy as np
import pytest

from conftest import model_dir, need_ref, rel_l2

pytestmark = pytest.mark.gpu

from qwen3_tts_amd import hip, synth  # noqa: E402


def _ref(name, prec, threads=8):
    from oracle.oracle import RefModel
    d, shape, t = model_dir(name)
    return RefModel(d, shape, prec=prec, threads=threads), shape, t


def _gpu_talker(ref, shape, prec_code, kv_max=2048, nlayers=None):
    layers = hip.layers_from_ref(ref, prec_code)
    if nlayers is not None:
        layers = layers[:nlayers]
    cos, sin = ref.rope()
    return hip.Talker(shape, layers, ref.final_norm(), cos, sin, prec_code, kv_max)


# ---------------------------------------------------------------------------- kernels

MV_SHAPES = [(4096, 1024), (1024, 3072), (2048, 2048), (2048, 6144), (6144, 1024), (3072, 2048),
             (257, 320), (64, 96)]


@pytest.mark.parametrize("prec", ["bf16", "int8", "q4"])
@pytest.mark.parametrize("rows,cols", MV_SHAPES)
def test_op_matvec(oracle, prec, rows, cols):
    if prec == "q4" and cols % 32:
        pytest.skip("q4_0 needs cols % 32 == 0")
    print(f"[case] matvec {prec} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    y = np.empty(rows, np.float32)
    L = hip.lib()
    if prec == "bf16":
        hip.check(L.qwen_hip_op_matvec_bf16(y.ctypes.data, w.ctypes.data, x.ctypes.data, rows, cols), "mv")
        y64 = oracle.matvec(0, w, None, x, rows, cols, f64=True)
    elif prec == "int8":
        q, s = oracle.quantize_int8(w)
        hip.check(L.qwen_hip_op_matvec_int8(y.ctypes.data, q.ctypes.data, s.ctypes.data, x.ctypes.data, rows, cols), "mv")
        y64 = oracle.matvec(1, q, s, x, rows, cols, f64=True)
    else:
        b = oracle.quantize_q4_0(w)
        hip.check(L.qwen_hip_op_matvec_q4_0(y.ctypes.data, b.ctypes.data, x.ctypes.data, rows, cols), "mv")
        y64 = oracle.matvec(2, b, None, x, rows, cols, f64=True)
    err = np.abs(y - y64).max() / np.abs(y64).max()
    assert err < 2e-5, err


@pytest.mark.parametrize("seq_k", [1, 2, 17, 64, 300, 2048, 4096, 4097, 5000, 8192])
def test_op_attention(oracle, seq_k):
    print(f"[case] attention seq_k={seq_k}", flush=True)
    nh, nkv, hd = 16, 8, 128
    rng = np.random.default_rng(seq_k)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = synth.f32_to_bf16_rne(rng.standard_normal((seq_k, nkv * hd)).astype(np.float32))
    V = synth.f32_to_bf16_rne(rng.standard_normal((seq_k, nkv * hd)).astype(np.float32))
    out = np.empty(nh * hd, np.float32)
    sc = 1.0 / np.sqrt(hd)
    hip.check(hip.lib().qwen_hip_op_causal_attention_bf16kv(out.ctypes.data, q.ctypes.data, K.ctypes.data,
                                                            V.ctypes.data, 1, seq_k, nh, nkv, hd,
                                                            np.float32(sc), seq_k - 1), "attn")
    ref = oracle.attention(q, K, V, 1, seq_k, nh, nkv, hd, sc, seq_k - 1)
    assert rel_l2(out, ref) < 2e-5
    # all-equal keys reduce softmax to the mean of V (closed form)
    if seq_k > 1:
        K2 = np.tile(K[:1], (seq_k, 1))
        hip.check(hip.lib().qwen_hip_op_causal_attention_bf16kv(out.ctypes.data, q.ctypes.data, K2.ctypes.data,
                                                                V.ctypes.data, 1, seq_k, nh, nkv, hd,
                                                                np.float32(sc), seq_k - 1), "attn")
        vf = synth.bf16_to_f32(V).reshape(seq_k, nkv, hd).mean(0)
        expect = np.repeat(vf, nh // nkv, axis=0).reshape(-1)
        assert np.abs(out - expect).max() < 1e-4


def test_op_attention_causal_multiquery(oracle):
    nh, nkv, hd, sq, sk = 16, 8, 128, 5, 40
    rng = np.random.default_rng(5)
    q = rng.standard_normal(sq * nh * hd).astype(np.float32)
    K = synth.f32_to_bf16_rne(rng.standard_normal((sk, nkv * hd)).astype(np.float32))
    V = synth.f32_to_bf16_rne(rng.standard_normal((sk, nkv * hd)).astype(np.float32))
    out = np.empty(sq * nh * hd, np.float32)
    hip.check(hip.lib().qwen_hip_op_causal_attention_bf16kv(out.ctypes.data, q.ctypes.data, K.ctypes.data,
                                                            V.ctypes.data, sq, sk, nh, nkv, hd,
                                                            np.float32(0.0883883), 30), "attn")
    ref = oracle.attention(q, K, V, sq, sk, nh, nkv, hd, 0.0883883, 30)
    assert rel_l2(out, ref) < 2e-5


@need_ref
@pytest.mark.parametrize("rows,cols", [(64, 1024), (300, 2048), (7, 72)])
def test_quantize_int8_bitexact_vs_reference(rows, cols):
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    rng = np.random.default_rng(rows)
    w = synth.f32_to_bf16_rne((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    w[0, :5] = 0  # a few exact zeros
    q_ref = np.empty((rows, cols), np.int8); s_ref = np.empty(rows, np.float32)
    R.ref_quantize_int8(w.ctypes.data, rows, cols, q_ref.ctypes.data, s_ref.ctypes.data)
    q = np.empty_like(q_ref); s = np.empty_like(s_ref)
    hip.check(hip.lib().qwen_hip_op_quantize_int8(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data), "q8")
    assert np.array_equal(q, q_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


@need_ref
@pytest.mark.parametrize("dist", ["model", "unit", "tiny", "huge", "grid", "sparse", "heavy"])
def test_quantize_q4_vs_reference(dist):
    """The device q4_0 quantizer (k_quant_q4) bit-exact against the reference's
    qwen_quantize_bf16_to_q4_0 (nibbles and f16 scales) across weight distributions."""
    from oracle.oracle import RefModel
    R = RefModel.load_lib()
    rows, cols = 512, 1024
    rng = np.random.default_rng(3)
    x = {"model": lambda: rng.standard_normal((rows, cols)) * 0.02, "unit": lambda: rng.standard_normal((rows, cols)),
         "tiny": lambda: rng.standard_normal((rows, cols)) * 1e-6, "huge": lambda: rng.standard_normal((rows, cols)) * 1e3,
         "grid": lambda: rng.integers(-8, 9, (rows, cols)) * 0.01,
         "sparse": lambda: rng.standard_normal((rows, cols)) * (rng.random((rows, cols)) < 0.1),
         "heavy": lambda: rng.standard_t(2, (rows, cols)) * 0.02}[dist]()
    w = synth.f32_to_bf16_rne(x.astype(np.float32))
    ref = np.empty(rows * cols // 32 * 18, np.uint8)
    R.ref_quantize_q4_0(w.ctypes.data, rows, cols, ref.ctypes.data)
    got = np.empty_like(ref)
    hip.check(hip.lib().qwen_hip_op_quantize_q4_0(w.ctypes.data, rows, cols, got.ctypes.data), "q4")
    rb, gb = ref.reshape(-1, 18), got.reshape(-1, 18)
    assert np.array_equal(rb[:, 2:], gb[:, 2:]), "nibbles"
    bad = np.where(~(rb[:, :2] == gb[:, :2]).all(1))[0]
    assert len(bad) == 0, (len(bad), bad[:4], rb[bad[:2], :2], gb[bad[:2], :2])


# ------------------------------------------------------------------------- Talker step

@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "bf16"), ("mini", "int8"), ("mini", "int4"), ("mini17", "int4"),
                                       ("mini17", "int8"), ("mini17", "bf16")])
def test_talker_steps_vs_reference(name, prec):
    """mini17 runs the fused step at hidden 2048 (int8: MFMA tiles; int4: q4_0 tiles; bf16);
    mini bf16/int8 the fused step at hidden 1024; mini int4 the per-kernel path."""
    print(f"[case] talker {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    pc = hip.PREC[prec]
    g = _gpu_talker(ref, shape, pc)
    emb = ref.codec_emb()
    rng = np.random.default_rng(11)
    nsteps = 24
    worst = 0.0
    for pos in range(nsteps):
        e = synth.bf16_to_f32(emb[rng.integers(0, 2048)])
        res, h_ref = ref.step_layers(e)
        h = g.step(e, pos)
        assert np.abs(h - h_ref).max() <= 2e-2
        assert rel_l2(h, h_ref) <= 1e-3, (pos, rel_l2(h, h_ref))
        assert rel_l2(g.dec_x(), res[-1]) <= 1e-3
        worst = max(worst, rel_l2(h, h_ref))
        if pos == 0:
            # first step, layer 0: same input, so only f32 rounding differences
            # (summation order; the reference's rsqrt+Newton 1/sqrt) that straddle a
            # truncation boundary can differ.  Deeper layers inherit those one-ulp
            # flips through attention, so they are only held to the ulp bound below.
            kr, vr = ref.kv()
            kg, vg = g.download_kv(1)
            for a, b in [(kg, kr), (vg, vr)]:
                assert (a[0, 0] != b[0, 0]).mean() < 5e-3
    # KV: the device cache holds the truncated bf16 bits of its own k/v.  Layer 0's
    # k/v depend only on the (identical) input embedding, so every element is within
    # one bf16 ulp of the reference's.  Deeper layers see inputs that already differ at
    # ~1e-4 (one-ulp flips fed back through attention), so they are held to a row
    # rel-L2 bound in line with the hidden-state tolerance.
    kr, vr = ref.kv()
    kg, vg = g.download_kv(nsteps)
    rates = []
    for a, b in [(kg, kr), (vg, vr)]:
        a, b = a[:, :nsteps], b[:, :nsteps]
        rates.append(float((a != b).mean()))
        fa, fb = synth.bf16_to_f32(a), synth.bf16_to_f32(b)
        tol = 2.0 ** -7 * np.maximum(np.abs(fa[0]), np.abs(fb[0])) + 1e-6
        bad = np.argwhere(np.abs(fa[0] - fb[0]) > tol)
        assert len(bad) == 0, [(tuple(i), fa[0][tuple(i)], fb[0][tuple(i)]) for i in bad[:8]]
        num = np.linalg.norm((fa - fb).astype(np.float64), axis=-1)
        den = np.linalg.norm(fb.astype(np.float64), axis=-1)
        assert (num <= 1e-2 * den + 1e-6).all(), float((num / den).max())
    print(f"[result] talker {prec}: worst hidden rel-L2 {worst:.2e}, KV mismatch k {rates[0]:.4f} v {rates[1]:.4f}")
    g.free()


@need_ref
def test_talker_per_layer_residuals():
    ref, shape, _ = _ref("mini", "bf16")
    g1 = _gpu_talker(ref, shape, hip.BF16, nlayers=1)
    g2 = _gpu_talker(ref, shape, hip.BF16)
    emb = ref.codec_emb()
    for pos in range(6):
        e = synth.bf16_to_f32(emb[pos * 37])
        res, _ = ref.step_layers(e)
        g1.step(e, pos)
        g2.step(e, pos)
        for l, got in enumerate([g1.dec_x(), g2.dec_x()]):
            assert np.abs(got - res[l]).max() <= 2e-2
            assert rel_l2(got, res[l]) <= 1e-3


@need_ref
def test_upload_kv_roundtrip_and_resume():
    """Host prefill -> upload_kv -> device decode continues the reference trajectory."""
    ref, shape, _ = _ref("mini", "bf16")
    emb = ref.codec_emb()
    rng = np.random.default_rng(2)
    embeds = [synth.bf16_to_f32(emb[rng.integers(0, 2048)]) for _ in range(12)]
    for e in embeds[:8]:
        ref.step(e)
    g = _gpu_talker(ref, shape, hip.BF16)
    kr, vr = ref.kv()
    g.upload_kv(np.ascontiguousarray(kr), np.ascontiguousarray(vr), 8)
    kg, vg = g.download_kv(8)
    assert np.array_equal(kg[:, :8], kr[:, :8]) and np.array_equal(vg[:, :8], vr[:, :8])
    for i, e in enumerate(embeds[8:]):
        h_ref = ref.step(e)
        h = g.step(e, 8 + i)
        assert rel_l2(h, h_ref) <= 1e-3


@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "bf16"), ("mini", "int8"), ("mini17", "bf16"), ("mini17", "int8"),
                                       ("mini17", "int4")])
def test_fused_step_matches_kernel_sequence(name, prec):
    """The default step (one persistent kernel, or the captured graph where that is
    unavailable) against the plain launch sequence: same per-row arithmetic (int8: the
    same exact integer piece sums, MFMA in the fused step, v_dot4 in the matvec kernel),
    so the residual stream is bit-identical; the final RMSNorm reduces in a different
    order.  mini bf16 runs the role-specialised kernel's bf16 build: its projections sum
    the same exact products (bf16 weight x three exact bf16 pieces of the activation) in
    the MFMA's f32 order instead of the matvec kernel's, so the projections agree to f32
    rounding (mini17 int4 runs its q4_0 build, and the per-kernel q4_0 matvec k_mv_q4r
    states that build's arithmetic in its order, so that pair is bit-identical); a K/V element whose two f32 values straddle a bf16 truncation boundary
    (about 1 in 16000) then differs by one bf16 ulp, and that flip moves the residual
    stream by ~1e-4.  The two paths are held to the bounds the per-kernel path meets
    against the reference (rel-L2 1e-3 on the residual stream, K/V rows within rel-L2
    1e-2) and to few K/V flips."""
    print(f"[case] fused vs kernels {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    pc = hip.PREC[prec]
    exact = (name, prec) != ("mini", "bf16")
    worst = 0.0
    ga = _gpu_talker(ref, shape, pc)
    gb = _gpu_talker(ref, shape, pc)
    emb = ref.codec_emb()
    for pos in range(10):
        e = synth.bf16_to_f32(emb[pos])
        a = ga.step(e, pos, graph=True)
        b = gb.step(e, pos, graph=False)
        if exact:
            assert np.array_equal(ga.dec_x(), gb.dec_x()), pos
            assert rel_l2(a, b) < 1e-6, pos
        else:
            assert rel_l2(ga.dec_x(), gb.dec_x()) < 1e-3, (pos, rel_l2(ga.dec_x(), gb.dec_x()))
            assert rel_l2(a, b) < 1e-3, pos
        worst = max(worst, rel_l2(ga.dec_x(), gb.dec_x()))
    print(f"[result] fused vs kernels {name} {prec}: worst residual rel-L2 {worst:.2e}")
    ka, va = ga.download_kv(10)
    kb, vb = gb.download_kv(10)
    if exact:
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    else:
        _kv_close(ka[:, :10], kb[:, :10])
        _kv_close(va[:, :10], vb[:, :10])


def _kv_close(x, y):
    """bf16 caches of two paths whose projections differ only in f32 summation order:
    rows within rel-L2 1e-2, and at most 5 % of the elements differing."""
    fx, fy = synth.bf16_to_f32(x).astype(np.float64), synth.bf16_to_f32(y).astype(np.float64)
    num = np.linalg.norm(fx - fy, axis=-1)
    den = np.linalg.norm(fy, axis=-1)
    assert (num <= 1e-2 * den + 1e-6).all(), float((num / np.maximum(den, 1e-30)).max())
    assert (x != y).mean() < 0.05, float((x != y).mean())


@need_ref
def test_fused_step_long_context_matches_kernel_sequence():
    """Caches beyond 4096 positions: every attention chunk holds more than one 128-key
    LDS block (the second block is staged inside the phase).  Fused step == per-kernel
    sequence bit for bit, and the per-kernel step against the oracle's attention-level
    tolerance through the final hidden state."""
    print("[case] fused vs kernels, KV 5000", flush=True)
    ref, shape, _ = _ref("mini17", "int8")
    pc = hip.INT8
    kv_max, n0 = 6144, 5000
    ga = _gpu_talker(ref, shape, pc, kv_max=kv_max)
    gb = _gpu_talker(ref, shape, pc, kv_max=kv_max)
    rng = np.random.default_rng(11)
    L, kvd = shape.layers, shape.kv_dim
    kk = synth.f32_to_bf16_rne(rng.standard_normal((L, n0, kvd)).astype(np.float32))
    vv = synth.f32_to_bf16_rne((rng.standard_normal((L, n0, kvd)) * 0.5).astype(np.float32))
    for g in (ga, gb):
        g.upload_kv(kk, vv, n0)
    emb = ref.codec_emb()
    hs = []
    for i in range(3):
        e = synth.bf16_to_f32(emb[100 + i])
        a = ga.step(e, n0 + i, graph=True)
        b = gb.step(e, n0 + i, graph=False)
        assert np.array_equal(ga.dec_x(), gb.dec_x()), i
        assert rel_l2(a, b) < 1e-6, i
        hs.append(b)
    ka, va = ga.download_kv(n0 + 3)
    kb, vb = gb.download_kv(n0 + 3)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    assert np.array_equal(ka[:, :n0], kk) and np.array_equal(va[:, :n0], vv)
    # the same three steps through the oracle's decode over the same cache
    from oracle.oracle import Oracle, oracle_talker
    orc = Oracle()
    ot, keep = oracle_talker(ref, pc, kv_max)
    keep["kv_k"][:, :n0] = kk
    keep["kv_v"][:, :n0] = vv
    for i, h in enumerate(hs):
        h_o, _ = orc.talker_step(ot, synth.bf16_to_f32(emb[100 + i]), n0 + i)
        assert np.abs(h - h_o).max() <= 2e-2 and rel_l2(h, h_o) <= 1e-3, (i, rel_l2(h, h_o))


@need_ref
@pytest.mark.parametrize("prec", ["bf16", "int8", "int4"])
def test_dequant_bitexact(oracle, prec):
    ref, shape, _ = _ref("mini", prec)
    pc = hip.PREC[prec]
    g = _gpu_talker(ref, shape, pc)
    for which, nm in enumerate(["q", "k", "v", "o", "gate_up", "down"]):
        m = ref.layer_mat(1, nm)
        rows, cols = m["rows"], m["cols"]
        got = g.dequant(1, which, 0, 16, cols)
        if pc == hip.BF16:
            want = synth.bf16_to_f32(m["bf16"][:16])
        elif pc == hip.INT8:
            want = oracle.dequant_int8(np.ascontiguousarray(m["int8"][:16]), np.ascontiguousarray(m["scale"][:16]))
        else:
            want = oracle.dequant_q4_0(m["q4"][: 16 * cols // 32 * 18], 16, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), nm


@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "bf16"), ("mini", "int8"), ("mini17", "int4"), ("mini17", "int8"),
                                       ("mini17", "bf16")])
def test_greedy_tokens_match_reference(name, prec):
    print(f"[case] greedy {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    pc = hip.PREC[prec]
    g = _gpu_talker(ref, shape, pc)
    emb = ref.codec_emb()
    head = np.ascontiguousarray(ref.codec_head())
    e0 = synth.bf16_to_f32(emb[123])
    n = 64
    toks_ref = []
    e = e0
    for f in range(n):
        h = ref.step(e)
        t, _ = ref.codec_greedy(h, f)
        toks_ref.append(t)
        e = synth.bf16_to_f32(emb[t])
    toks, _ = g.greedy(head, np.ascontiguousarray(emb), e0, 0, 0, n)
    assert list(toks) == toks_ref


@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "int8"), ("mini17", "int8"), ("mini", "bf16"), ("mini17", "int4")])
def test_fused_greedy_one_launch_matches_step_launches(name, prec):
    """A greedy launch of 24 steps from position 0, which crosses 16 keys (so every one of
    its steps keeps the attention merge of the chunk partials), against the same steps as
    one launch each (up to 16 keys a launch has every key in chunk 0 and writes the
    attention output from that chunk, o * (1/l), without the merge): the same tokens, and
    the same hidden state and K/V to the bit."""
    print(f"[case] greedy one launch vs step launches {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    pc = hip.PREC[prec]
    ga, gb = _gpu_talker(ref, shape, pc), _gpu_talker(ref, shape, pc)
    emb = np.ascontiguousarray(ref.codec_emb())
    head = np.ascontiguousarray(ref.codec_head())
    e0 = synth.bf16_to_f32(emb[321])
    n = 24
    ta, ha = ga.greedy(head, emb, e0, 0, 10, n)
    tb, e = [], e0
    for i in range(n):
        t1, hb = gb.greedy(head, emb, e, i, 10 + i, 1)
        tb.append(int(t1[0]))
        e = synth.bf16_to_f32(emb[int(t1[0])])
    assert list(ta) == tb
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))
    ka, va = ga.download_kv(n)
    kb, vb = gb.download_kv(n)
    assert np.array_equal(ka[:, :n], kb[:, :n]) and np.array_equal(va[:, :n], vb[:, :n])
    ga.free(); gb.free()


@need_ref
@pytest.mark.parametrize("name,prec,top_p,text_len,warmup", [("mini", "int8", 1.0, 0, 0), ("mini17", "int4", 1.0, 0, 0),
                                                             ("mini", "int8", 0.8, 1, 3), ("mini17", "int8", 0.95, 2, 0)])
def test_sampled_loop_matches_reference(oracle, name, prec, top_p, text_len, warmup):
    """qwen_hip_talker_sample (step -> codec head -> rule + qwen_tts_sample -> next embed, all
    on the device) against the reference's step and codec head with the oracle sampler
    (pinned to the reference's qwen_tts_sample) at the reference's default settings, with
    top-p below 1, greedy warmup frames and the EOS boost of qwen_tts.c:1666-1675 (text_len
    1 or 2: the boost starts after frame 6 or 12 and ends the utterance within the run).
    A token may differ only where the draw lies within rounding of a cumulative boundary;
    the trajectories part there, so the comparison stops, but the first 8 tokens must
    agree.  Generation ends at the first EOS on both sides (qwen_tts.c:1716-1719) with the
    same LCG state.  At temperature 0 the loop gives the greedy loop's tokens and leaves
    the LCG state alone."""
    from conftest import draw_margin
    print(f"[case] sampled loop {name} {prec} top_p={top_p} text_len={text_len} warmup={warmup}", flush=True)
    ref, shape, _ = _ref(name, prec)
    pc = hip.PREC[prec]
    emb = ref.codec_emb()
    head = np.ascontiguousarray(ref.codec_head())
    embc = np.ascontiguousarray(emb)
    e0 = synth.bf16_to_f32(emb[321])
    prev0 = [5, 17, 5, 900]
    n = 32
    g = _gpu_talker(ref, shape, pc)
    toks, _, seed_dev = g.sample(head, embc, e0, 0, 0, n, 0.9, 50, top_p, 1.05, prev0, 777,
                                 greedy_warmup=warmup, text_len=text_len)
    seed, prev, e, same, ref_toks = 777, list(prev0), e0, 0, []
    expected, start = 3 * text_len, 6 * text_len
    parted = False
    for f in range(n):
        h = ref.step(e)
        _, lg = ref.codec_greedy(h, f)
        boost = min(np.float32(0.5) * np.float32(f - start), np.float32(10.0)) if expected > 0 and f > start else 0.0
        temp, tk = (0.0, 1) if f < warmup else (0.9, 50)
        t, seed, dist = oracle.sample(lg, temp, tk, top_p, 1.05, prev, seed, rule=(f, float(boost)))
        ref_toks.append(t)
        if f >= len(toks) or int(toks[f]) != t:
            assert dist is not None and draw_margin(dist, seed) < 1e-4, (f, toks[f:f + 1], t)
            parted = True
            break
        same += 1
        if t == 2150:
            break
        prev.append(t)
        e = synth.bf16_to_f32(emb[t])
    print(f"[result] sampled loop {name} {prec}: {same}/{len(toks)} tokens identical, reference {ref_toks[-4:]}")
    assert same >= min(8, len(ref_toks)), same
    if not parted:
        assert len(toks) == len(ref_toks) and seed_dev == seed
    if text_len:
        assert 2150 in ref_toks or parted, "the EOS boost should end the utterance within the run"
    g.free()
    # temperature 0: the greedy loop's tokens, LCG state untouched
    ga, gb = _gpu_talker(ref, shape, pc), _gpu_talker(ref, shape, pc)
    t_s, h_s, sd = ga.sample(head, embc, e0, 0, 0, 16, 0.0, 0, 1.0, 1.0, (), 99)
    t_g, h_g = gb.greedy(head, embc, e0, 0, 0, 16)
    assert list(t_s) == list(t_g) and sd == 99
    assert rel_l2(h_s, h_g) < 1e-5
    ga.free(); gb.free()


# ------------------------------------------------------------------------ Code Predictor

def _gpu_cp(ref, shape, prec_code):
    from qwen3_tts_amd.hip import CpDesc, Mat, Layer, TalkerDesc
    import ctypes as C
    s = shape
    keep = []
    layers = hip.layers_from_ref(ref, prec_code, cp=True)
    arr = (Layer * len(layers))()
    for l, ly in enumerate(layers):
        for nm in ["q", "k", "v", "o", "gate_up", "down"]:
            w, sc = ly[nm]
            keep += [w, sc]
            getattr(arr[l], nm).w = w.ctypes.data
            getattr(arr[l], nm).scale = None if sc is None else sc.ctypes.data
        for nm in ["input_norm", "post_attn_norm", "q_norm", "k_norm"]:
            keep.append(ly[nm]); setattr(arr[l], nm, ly[nm].ctypes.data)
    cos, sin = ref.cp_rope()
    fn = ref.cp_norm()
    keep += [arr, cos, sin, fn]
    td = TalkerDesc(hidden=s.cp_hidden, inter=s.cp_inter, n_heads=s.cp_heads, n_kv_heads=s.cp_kv_heads,
                    head_dim=s.cp_head_dim, n_layers=len(layers), kv_max=64, eps=s.eps, prec=prec_code,
                    quantize_to=-1, layers=arr, final_norm=fn.ctypes.data, rope_cos=cos.ctypes.data,
                    rope_sin=sin.ctypes.data, rope_len=cos.shape[0])
    d = CpDesc()
    d.cp = td
    d.codebook = s.codebook
    d.lm_prec = prec_code
    kind = {0: "bf16", 1: "int8", 2: "q4"}[prec_code]
    for gi in range(15):
        lm = ref.cp_lm_head(gi)
        keep.append(lm)
        d.lm_head[gi].w = lm[kind].ctypes.data
        d.lm_head[gi].scale = lm["scale"].ctypes.data if prec_code == 1 else None
        ce = ref.cp_codec_emb(gi); keep.append(ce)
        d.cp_codec_emb[gi] = ce.ctypes.data
    te = ref.codec_emb(); keep.append(te)
    d.talker_codec_emb = te.ctypes.data
    d.codec_vocab = s.codec_vocab
    d.talker_hidden = s.hidden
    d.emb_dim = s.hidden
    mtp = ref.cp_mtp()
    if mtp["bf16"] is not None:
        use8 = mtp["int8"] is not None
        d.mtp_prec = 1 if use8 else 0
        d.mtp.w = (mtp["int8"] if use8 else mtp["bf16"]).ctypes.data
        d.mtp.scale = mtp["scale"].ctypes.data if use8 else None
        d.mtp_bias = mtp["bias"].ctypes.data
        keep.append(mtp)
    return hip.CodePredictor(d, keep)


@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "bf16"), ("mini", "int8"), ("mini17", "bf16"), ("mini", "int4")])
def test_cp_frame_codes_match_reference(name, prec):
    print(f"[case] cp frame {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    cp = _gpu_cp(ref, shape, hip.PREC[prec])
    rng = np.random.default_rng(7)
    for f in range(4):
        th = rng.standard_normal(shape.hidden).astype(np.float32)
        th /= np.sqrt((th ** 2).mean())
        code0 = int(rng.integers(0, 2048))
        want = ref.cp_predict(th, code0)
        got = cp.frame(th, code0)
        assert list(got) == list(want), (f, got, want)


@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "int8"), ("mini17", "int8"), ("mini", "bf16"), ("mini17", "bf16")])
def test_cp_frame_fused_matches_launch_graph(name, prec):
    """CP layers of the 0.6B geometry (mini17: with the 1.7B Talker's mtp projection
    2048 -> 1024 in front of every pass): the frame as one launch of the role-specialised
    kernel and as the per-kernel launch graph give the same codes over frames back to back,
    the codes are the reference's qwen_cp_predict (the fused frame is the default), and the
    K/V of all 16 positions are the same bits with int8 weights.  With bf16 weights the
    fused frame's projections sum the same exact products in the MFMA's f32 order, so its
    K/V are held to rel-L2 1e-2 per row with few elements differing."""
    print(f"[case] fused CP frame {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    cp = _gpu_cp(ref, shape, hip.PREC[prec])
    assert cp.fused(True), f"the 0.6B {prec} CP should take the fused frame"
    rng = np.random.default_rng(11)
    for f in range(5):
        th = rng.standard_normal(shape.hidden).astype(np.float32)
        th /= np.sqrt((th ** 2).mean())
        code0 = int(rng.integers(0, 2048))
        assert cp.fused(True)
        a = list(cp.frame(th, code0))
        ka, va = cp.download_kv(16)
        assert not cp.fused(False)
        b = list(cp.frame(th, code0))
        kb, vb = cp.download_kv(16)
        assert a == b, (f, a, b)
        if prec == "int8":
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), f
        else:
            _kv_close(ka, kb)
            _kv_close(va, vb)
        assert a == list(ref.cp_predict(th, code0)), f
    cp.fused(True)


@need_ref
@pytest.mark.parametrize("name,prec", [("mini", "bf16"), ("mini", "int8"), ("mini17", "int4"), ("mini17", "int8")])
def test_load_file_matches_reference_loader(name, prec):
    """qwen_hip_talker_load_file (model.safetensors -> device, gate|up interleaved and
    quantized on the device) against the state built from the reference loader's own
    bytes (bf16 mmap, its host int8 / q4_0 quantizers): every matrix dequantises to the
    same bits, and steps give the same results bit for bit."""
    print(f"[case] load_file {name} {prec}", flush=True)
    ref, shape, _ = _ref(name, prec)
    d, _, _ = model_dir(name)
    pc = hip.PREC[prec]
    cos, sin = ref.rope()
    a = hip.Talker.from_file(d, shape, cos, sin, 256, quantize_to=-1 if prec == "bf16" else pc)
    b = _gpu_talker(ref, shape, pc, kv_max=256)
    for l in range(shape.layers):
        for which, nm in enumerate(["q", "k", "v", "o", "gate_up", "down"]):
            m = ref.layer_mat(l, nm)
            rows, cols = m["rows"], m["cols"]
            n = min(rows, 64)
            ga, gb = a.dequant(l, which, rows - n, n, cols), b.dequant(l, which, rows - n, n, cols)
            assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), (l, nm)
    emb = ref.codec_emb()
    for pos in range(4):
        e = synth.bf16_to_f32(emb[pos * 11])
        ha, hb = a.step(e, pos), b.step(e, pos)
        assert np.array_equal(ha, hb) and np.array_equal(a.dec_x(), b.dec_x()), pos
    a.free()
    b.free()
