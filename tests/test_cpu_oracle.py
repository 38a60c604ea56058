"""The oracle (oracle/qwen_oracle.c) pinned on the CPU.

Three independent pins, chosen so that a plausible slip in the restatement (a dropped
term, a wrong sign or index, a transposed operand, a different rounding rule) fails one:

* golden fixtures written by the reference's own C (tests/golden/make_golden.py);
* the compiled reference itself when oracle/_ref is built (``need_ref``);
* closed forms: float64 brute force, special cases that reduce to a textbook result
  (attention over one key is that key's value; equal scores give the mean of V),
  invariants of the quantizers.
No GPU is used here.
"""
import os

import numpy as np
import pytest

from conftest import draw_margin, need_oracle, need_ref, rel_l2, sample_cases

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = need_oracle


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bf16_to_f64(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def f32_to_bf16_rne(a):
    from qwen3_tts_amd import synth
    return synth.f32_to_bf16_rne(np.asarray(a, np.float32))


# ---------------------------------------------------------------------------------------
# conversions
# ---------------------------------------------------------------------------------------

def test_f16_to_f32_golden(oracle):
    g = gold("golden_convert.npz")
    got = np.array([oracle.lib.qo_f16_to_f32(int(h)) for h in g["halves"]], np.float32).view(np.uint32)
    assert np.array_equal(got, g["f16_to_f32"])


def test_f16_to_f32_exhaustive_closed_form(oracle):
    """Normals, zeros and infinities equal IEEE binary16; subnormals follow the
    reference's portable branch (qwen_tts_kernels.h:162-179), whose exponent
    112 - shift yields exactly half the IEEE value; NaN stays NaN."""
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.lib.qo_f16_to_f32(int(v)) for v in h], np.float32)
    ieee = h.astype(np.uint16).view(np.float16).astype(np.float32)
    exp = (h >> 10) & 0x1F
    mant = h & 0x3FF
    normal = (exp > 0) & (exp < 31)
    assert np.array_equal(got[normal], ieee[normal])
    zero = (exp == 0) & (mant == 0)
    assert np.array_equal(got[zero].view(np.uint32), ieee[zero].view(np.uint32))
    sub = (exp == 0) & (mant != 0)
    assert np.array_equal(got[sub], ieee[sub] * np.float32(0.5))
    inf = (exp == 31) & (mant == 0)
    assert np.array_equal(got[inf], ieee[inf])
    assert np.all(np.isnan(got[(exp == 31) & (mant != 0)]))


def test_f32_to_f16_golden(oracle):
    g = gold("golden_convert.npz")
    got = np.array([oracle.lib.qo_f32_to_f16(float(v)) for v in g["f32_in"]], np.uint16)
    assert np.array_equal(got, g["f32_to_f16"])


def test_f32_to_f16_against_ieee(oracle):
    """Within the normal binary16 range the reference's rounding equals IEEE
    round-to-nearest except on exact ties, where it rounds the magnitude up."""
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.normal(0, 1, 3000), rng.uniform(-6e4, 6e4, 1000)]).astype(np.float32)
    x = x[np.abs(x) >= 6.2e-5]
    got = np.array([oracle.lib.qo_f32_to_f16(float(v)) for v in x], np.uint16)
    ieee = x.astype(np.float16).view(np.uint16)
    diff = got != ieee
    # every difference must be an exact tie rounded away from zero by one unit
    for v, a, b in zip(x[diff], got[diff], ieee[diff]):
        lo = np.float16(v).astype(np.float64)
        assert abs(int(a) - int(b)) == 1
        up = np.array([max(a, b)], np.uint16).view(np.float16)[0].astype(np.float64)
        dn = np.array([min(a, b)], np.uint16).view(np.float16)[0].astype(np.float64)
        assert abs(float(v) - (up + dn) / 2) == 0.0, (v, lo)
        assert abs(np.array([a], np.uint16).view(np.float16)[0]) >= abs(np.array([b], np.uint16).view(np.float16)[0])


def test_bf16_truncation(oracle):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 10, 2000).astype(np.float32)
    got = np.array([oracle.lib.qo_f32_to_bf16_trunc(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, (x.view(np.uint32) >> 16).astype(np.uint16))
    back = np.array([oracle.lib.qo_bf16_to_f32(int(b)) for b in got], np.float32)
    assert np.array_equal(back.view(np.uint32), got.astype(np.uint32) << 16)


# ---------------------------------------------------------------------------------------
# quantizers
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["a", "b"])
def test_int8_quantizer_golden(oracle, tag):
    g = gold("golden_quant.npz")
    q, s = oracle.quantize_int8(g[f"i8_{tag}_w"])
    assert np.array_equal(s.view(np.uint32), g[f"i8_{tag}_s"].view(np.uint32))
    assert np.array_equal(q, g[f"i8_{tag}_q"])


def test_int8_quantizer_invariants(oracle):
    rng = np.random.default_rng(11)
    w = f32_to_bf16_rne(rng.normal(0, 0.03, (64, 512)))
    q, s = oracle.quantize_int8(w)
    v = bf16_to_f64(w)
    amax = np.abs(v).max(axis=1)
    # scale is amax/127 to within one f32 rounding of the reciprocal form
    assert np.allclose(s, amax / 127.0, rtol=2.5e-7, atol=0)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    arg = np.abs(v).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(64), arg]) == 127)
    err = np.abs(v - q.astype(np.float64) * s[:, None].astype(np.float64))
    assert np.all(err <= 0.5 * s[:, None] * (1 + 1e-5) + 1e-12)


def test_q4_quantizer_golden(oracle):
    g = gold("golden_quant.npz")
    b = oracle.quantize_q4_0(g["q4_w"])
    ref = g["q4_blocks"]
    # bit-exact: nibbles and f16 scales.  The reference build may vectorise the scale's
    # double sums in any order, but every term (v^2 * v * q, v^2 * q^2 of bf16 values and
    # q in [-8, 7]) is an exact double and the few-ulp rounding of the sum never reaches
    # the f16 rounding of the scale, so order does not show.
    assert np.array_equal(b[..., 2:], ref[..., 2:]), "nibbles"
    assert np.array_equal(b[..., :2], ref[..., :2]), "f16 scales"


def test_q4_quantizer_invariants(oracle):
    """q in [-8, 7]; the first largest |v| of a block maps to -8; the f16 scale is the
    weighted least-squares optimum sum(v^2 v q)/sum(v^2 q^2) up to f16 rounding."""
    rng = np.random.default_rng(12)
    w = f32_to_bf16_rne(rng.normal(0, 0.02, (32, 256)))
    b = oracle.quantize_q4_0(w)
    v = bf16_to_f64(w).reshape(32, 8, 32)
    qs = b[..., 2:]
    q = np.empty((32, 8, 32), np.int32)
    q[..., 0::2] = (qs & 0xF).astype(np.int32) - 8
    q[..., 1::2] = (qs >> 4).astype(np.int32) - 8
    assert q.min() >= -8 and q.max() <= 7
    first = np.abs(v).argmax(axis=2)
    assert np.all(np.take_along_axis(q, first[..., None], 2)[..., 0] == -8)
    opt = (v * v * v * q).sum(2) / (v * v * q * q).sum(2)
    sc = b[..., :2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    assert np.all(np.abs(sc - opt) <= np.abs(opt) * 2.0 ** -10)


def test_dequant_closed_form(oracle):
    rng = np.random.default_rng(13)
    w = f32_to_bf16_rne(rng.normal(0, 0.02, (16, 128)))
    q, s = oracle.quantize_int8(w)
    assert np.array_equal(oracle.dequant_int8(q, s), (q.astype(np.float32) * s[:, None]).astype(np.float32))
    b = oracle.quantize_q4_0(w)
    d = oracle.dequant_q4_0(b, 16, 128)
    sc = b[..., :2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float32)
    nib = np.empty((16, 4, 32), np.float32)
    nib[..., 0::2] = (b[..., 2:] & 0xF).astype(np.float32) - 8
    nib[..., 1::2] = (b[..., 2:] >> 4).astype(np.float32) - 8
    assert np.array_equal(d, (nib * sc[..., None]).reshape(16, 128))


# ---------------------------------------------------------------------------------------
# layer operations
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("prec", ["bf16", "int8", "q4"])
def test_matvec_golden_and_f64(oracle, prec):
    g = gold("golden_ops.npz")
    W, x = g["mv_W"], g["mv_x"]
    rows, cols = W.shape
    if prec == "bf16":
        y = oracle.matvec(0, W, None, x, rows, cols)
        wd = bf16_to_f64(W)
        yr = g["mv_y_bf16"]
    elif prec == "int8":
        q, s = oracle.quantize_int8(W)
        assert np.array_equal(q, g["mv_q8"])
        y = oracle.matvec(1, q, s, x, rows, cols)
        wd = q.astype(np.float64) * s[:, None].astype(np.float64)
        yr = g["mv_y_int8"]
    else:
        b = g["mv_q4"]
        y = oracle.matvec(2, b, None, x, rows, cols)
        wd = oracle.dequant_q4_0(b, rows, cols).astype(np.float64)
        yr = g["mv_y_q4"]
    exact = wd @ x.astype(np.float64)
    tol = 4e-6 * np.abs(wd) @ np.abs(x.astype(np.float64)) + 1e-7
    assert np.all(np.abs(y - exact) <= tol)
    assert np.all(np.abs(yr - exact) <= tol), "reference vs f64"


def test_attention_golden(oracle):
    g = gold("golden_ops.npz")
    sk = g["at_K"].shape[0]
    out = oracle.attention(g["at_Q"], g["at_K"], g["at_V"], 1, sk, 4, 2, 128, np.float32(1 / np.sqrt(128)), sk - 1)
    assert rel_l2(out, g["at_out"]) < 1e-6
    # float64 softmax brute force
    Q = g["at_Q"].reshape(4, 128).astype(np.float64)
    K = bf16_to_f64(g["at_K"]).reshape(sk, 2, 128)
    V = bf16_to_f64(g["at_V"]).reshape(sk, 2, 128)
    exp = np.empty((4, 128))
    for h in range(4):
        sc = K[:, h // 2] @ Q[h] / np.sqrt(128)
        p = np.exp(sc - sc.max())
        exp[h] = p @ V[:, h // 2] / p.sum()
    assert rel_l2(out, exp.ravel()) < 1e-6


def test_attention_special_cases(oracle):
    rng = np.random.default_rng(5)
    nh, nkv, hd = 4, 2, 128
    Q = rng.normal(0, 1, nh * hd).astype(np.float32)
    # one key: the output is that key's value, exactly
    K = f32_to_bf16_rne(rng.normal(0, 1, (1, nkv * hd)))
    V = f32_to_bf16_rne(rng.normal(0, 1, (1, nkv * hd)))
    out = oracle.attention(Q, K, V, 1, 1, nh, nkv, hd, np.float32(1 / np.sqrt(hd)), 0).reshape(nh, hd)
    v = bf16_to_f64(V).reshape(nkv, hd)
    for h in range(nh):
        assert np.array_equal(out[h], v[h // 2].astype(np.float32))
    # identical keys: all scores equal, the output is the mean of V
    n = 50
    K = np.repeat(K, n, axis=0)
    V = f32_to_bf16_rne(rng.normal(0, 1, (n, nkv * hd)))
    out = oracle.attention(Q, K, V, 1, n, nh, nkv, hd, np.float32(1 / np.sqrt(hd)), n - 1).reshape(nh, hd)
    mean = bf16_to_f64(V).reshape(n, nkv, hd).mean(0)
    for h in range(nh):
        assert np.allclose(out[h], mean[h // 2], rtol=1e-5, atol=1e-6)
    # causal mask: query at offset 0 over 50 keys sees key 0 only
    out0 = oracle.attention(Q, K, V, 1, n, nh, nkv, hd, np.float32(1 / np.sqrt(hd)), 0).reshape(nh, hd)
    v0 = bf16_to_f64(V[:1]).reshape(nkv, hd)
    for h in range(nh):
        assert np.array_equal(out0[h], v0[h // 2].astype(np.float32))


def test_rms_norm_golden_and_closed_form(oracle):
    g = gold("golden_ops.npz")
    y = oracle.rms_norm(g["rn_x"], g["rn_w"], 1e-6)
    assert rel_l2(y, g["rn_y"]) < 1e-6
    x = g["rn_x"].astype(np.float64)
    exp = x / np.sqrt((x * x).mean() + 1e-6) * g["rn_w"].astype(np.float64)
    assert np.allclose(y, exp, rtol=2e-6, atol=1e-7)


def test_swiglu_golden_and_closed_form(oracle):
    g = gold("golden_ops.npz")
    y = oracle.swiglu(g["sw_in"])
    assert np.allclose(y, g["sw_out"], rtol=2e-6, atol=1e-7)
    gu = g["sw_in"].astype(np.float64)
    exp = gu[0::2] / (1 + np.exp(-gu[0::2])) * gu[1::2]
    assert np.allclose(y, exp, rtol=2e-6, atol=1e-7)


def test_rope_closed_form(oracle):
    """NeoX split-half rotation: (x1, x2) -> (x1 c - x2 s, x2 c + x1 s) per frequency,
    i.e. multiplication of x1 + i x2 by e^{i angle}; position 0 (cos 1, sin 0) is exact."""
    import ctypes as C
    rng = np.random.default_rng(9)
    nh, hd = 3, 128
    x = rng.normal(0, 1, nh * hd).astype(np.float32)
    ang = rng.uniform(-np.pi, np.pi, (2, hd // 2))
    cos = np.cos(ang).astype(np.float32)
    sin = np.sin(ang).astype(np.float32)
    cos[0] = 1.0; sin[0] = 0.0
    for pos in (0, 1):
        y = x.copy()
        oracle.lib.qo_rope_neox(y.ctypes.data_as(C.c_void_p), nh, hd, cos.ctypes.data_as(C.c_void_p),
                                sin.ctypes.data_as(C.c_void_p), pos)
        z = x.reshape(nh, 2, hd // 2).astype(np.float64)
        c = z[:, 0] + 1j * z[:, 1]
        r = c * (cos[pos].astype(np.float64) + 1j * sin[pos].astype(np.float64))
        exp = np.stack([r.real, r.imag], 1).ravel()
        if pos == 0:
            assert np.array_equal(y, x)
        assert np.allclose(y, exp, rtol=1e-6, atol=1e-6)


def test_per_head_norm_closed_form(oracle):
    import ctypes as C
    rng = np.random.default_rng(10)
    nh, hd = 5, 128
    x = rng.normal(0, 2, nh * hd).astype(np.float32)
    w = (1 + rng.normal(0, 0.1, hd)).astype(np.float32)
    y = x.copy()
    oracle.lib.qo_rms_norm_per_head(y.ctypes.data_as(C.c_void_p), w.ctypes.data_as(C.c_void_p), nh, hd,
                                    C.c_float(1e-6))
    z = x.reshape(nh, hd).astype(np.float64)
    exp = z / np.sqrt((z * z).mean(1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.allclose(y, exp.ravel(), rtol=2e-6, atol=1e-7)


def test_argmax_lowest_index_on_ties(oracle):
    v = np.array([1.0, 3.0, -2.0, 3.0, 3.0], np.float32)
    assert oracle.lib.qo_argmax(v.ctypes.data, v.size) == 1
    v = np.full(7, -5.0, np.float32)
    assert oracle.lib.qo_argmax(v.ctypes.data, v.size) == 0


def _greedy(oracle, logits, frame):
    """Run the codec-head greedy rule with a head whose first column holds `logits` and a
    hidden state e_0, so head . hidden reproduces them exactly (bf16-representable)."""
    vocab, D = logits.size, 8
    head = np.zeros((vocab, D), np.uint16)
    head[:, 0] = f32_to_bf16_rne(logits)
    hid = np.zeros(D, np.float32); hid[0] = 1.0
    return oracle.lib.qo_codec_greedy(head.ctypes.data, hid.ctypes.data, vocab, D, frame, None)


def test_codec_greedy_rules(oracle):
    """qwen_tts.c:1652-1694 + qwen_tts_sampling.c:165-181: clip to [-100, 100];
    tokens 2048..3071 except EOS 2150 are masked; EOS is masked on frames 0 and 1;
    ties resolve to the lowest index."""
    base = np.full(3072, -1.0, np.float32)
    lg = base.copy(); lg[2500] = 50.0; lg[17] = 5.0
    assert _greedy(oracle, lg, 5) == 17                       # masked control token
    lg = base.copy(); lg[2150] = 50.0; lg[900] = 5.0
    assert _greedy(oracle, lg, 0) == 900                      # EOS masked on frame 0
    assert _greedy(oracle, lg, 1) == 900                      # ... and frame 1
    assert _greedy(oracle, lg, 2) == 2150                     # allowed from frame 2
    lg = base.copy(); lg[700] = 150.0; lg[300] = 120.0
    assert _greedy(oracle, lg, 3) == 300                      # both clip to 100: lowest index
    lg = base.copy(); lg[1000] = 7.0; lg[999] = 7.0
    assert _greedy(oracle, lg, 3) == 999


# ---------------------------------------------------------------------------------------
# whole decode step and Code-Predictor frame against the reference's outputs
# ---------------------------------------------------------------------------------------

def _tiny_tensors():
    from qwen3_tts_amd import synth
    if not hasattr(_tiny_tensors, "t"):
        _tiny_tensors.t = synth.generate(synth.SHAPES["tiny"], 0x5EED0001, 0.1, threads=8)
    return _tiny_tensors.t


def test_synthetic_weights_are_the_fixture_weights():
    import hashlib
    t = _tiny_tensors()
    h = hashlib.sha256()
    for k in sorted(t):
        h.update(k.encode())
        h.update(np.ascontiguousarray(t[k]).tobytes())
    assert h.hexdigest() == str(gold("golden_tiny_bf16.npz")["weights_sha256"])


@pytest.mark.parametrize("prec", ["bf16", "int8", "int4"])
def test_talker_steps_golden(oracle, prec):
    from oracle.oracle import talker_from_tensors
    from qwen3_tts_amd import synth
    g = gold(f"golden_tiny_{prec}.npz")
    s = synth.SHAPES["tiny"]
    t = _tiny_tensors()
    ot, keep = talker_from_tensors(oracle, t, s, prec, 64, g["rope_cos"], g["rope_sin"])
    emb = t["talker.model.codec_embedding.weight"]
    for i, tok in enumerate(g["tokens"]):
        h, dx = oracle.talker_step(ot, synth.bf16_to_f32(emb[tok]), i)
        assert np.abs(h - g["hidden"][i]).max() <= 2e-2 and rel_l2(h, g["hidden"][i]) <= 1e-3, i
        assert rel_l2(dx, g["dec_x"][i]) <= 1e-3, i
    n = len(g["tokens"])
    kk, vv = keep["kv_k"][:, :n], keep["kv_v"][:, :n]
    vk = bf16_to_f64(kk) - bf16_to_f64(g["kv_k"])
    vv_ = bf16_to_f64(vv) - bf16_to_f64(g["kv_v"])
    # truncation to bf16 can flip one unit where the f32 values differ in the last bits
    assert (kk != g["kv_k"]).mean() < 0.02 and (vv != g["kv_v"]).mean() < 0.02
    assert np.abs(vk).max() < 0.05 and np.abs(vv_).max() < 0.05


@pytest.mark.parametrize("prec", ["bf16", "int8", "int4"])
def test_cp_frames_golden(oracle, prec):
    from oracle.oracle import cp_frame_from_tensors
    from qwen3_tts_amd import synth
    g = gold(f"golden_tiny_{prec}.npz")
    s = synth.SHAPES["tiny"]
    f, keep = cp_frame_from_tensors(oracle, _tiny_tensors(), s, prec, g["cp_rope_cos"], g["cp_rope_sin"])
    for i in range(g["frame_codes"].shape[0]):
        codes = oracle.cp_frame(f, g["frame_hidden"][i], int(g["frame_code0"][i]))
        assert np.array_equal(codes, g["frame_codes"][i]), (i, codes, g["frame_codes"][i])


# ---------------------------------------------------------------------------------------
# against the compiled reference directly (in this container)
# ---------------------------------------------------------------------------------------

@need_ref
def test_quantizers_vs_reference_random(oracle):
    import ctypes as C
    from oracle.oracle import RefModel
    L = RefModel.load_lib()
    rng = np.random.default_rng(21)
    for rows, cols in [(33, 1024), (7, 200), (5, 3072)]:
        w = f32_to_bf16_rne(rng.normal(0, 0.02, (rows, cols)))
        q, s = oracle.quantize_int8(w)
        qr = np.empty_like(q); sr = np.empty_like(s)
        L.ref_quantize_int8(w.ctypes.data_as(C.c_void_p), rows, cols, qr.ctypes.data_as(C.c_void_p),
                            sr.ctypes.data_as(C.c_void_p))
        assert np.array_equal(q, qr) and np.array_equal(s, sr)
        if cols % 32 == 0:
            b = oracle.quantize_q4_0(w)
            br = np.empty_like(b)
            L.ref_quantize_q4_0(w.ctypes.data_as(C.c_void_p), rows, cols, br.ctypes.data_as(C.c_void_p))
            assert np.array_equal(b, br)


@need_ref
@pytest.mark.parametrize("variant", ["", "_avx512"])
def test_q4_quantizer_bitexact_across_distributions(oracle, variant):
    """The q4_0 restatement against both reference builds on weight distributions that
    stress the quantizer: the model's N(0, 0.02), unit and extreme magnitudes (f16
    subnormal and large scales), exact grid values (rounding ties), sparse blocks (zeros,
    vmax of either sign) and heavy tails (wide dynamic range inside a block)."""
    import ctypes as C
    from oracle.oracle import RefModel
    L = RefModel.load_lib(variant)
    rng = np.random.default_rng(9)
    cases = [rng.standard_normal((512, 1024)) * 0.02, rng.standard_normal((128, 1024)),
             rng.standard_normal((64, 1024)) * 1e-6, rng.standard_normal((64, 1024)) * 1e3,
             rng.integers(-8, 9, (64, 1024)) * 0.01, rng.standard_normal((64, 1024)) * (rng.random((64, 1024)) < 0.1),
             rng.standard_t(2, (64, 1024)) * 0.02]
    for x in cases:
        w = f32_to_bf16_rne(x.astype(np.float32))
        rows, cols = w.shape
        b = oracle.quantize_q4_0(w)
        br = np.empty_like(b)
        L.ref_quantize_q4_0(w.ctypes.data_as(C.c_void_p), rows, cols, br.ctypes.data_as(C.c_void_p))
        assert np.array_equal(b, br)


@need_ref
def test_gate_up_interleave_matches_reference_loader():
    from conftest import model_dir
    from oracle.oracle import RefModel
    from qwen3_tts_amd import synth
    d, shape, t = model_dir("tiny")
    ref = RefModel(d, shape, prec="bf16", threads=1)
    for l in range(shape.layers):
        p = f"talker.model.layers.{l}."
        gu = synth.interleave_gate_up(t[p + "mlp.gate_proj.weight"], t[p + "mlp.up_proj.weight"])
        assert np.array_equal(ref.layer_mat(l, "gate_up")["bf16"], gu)


# ---------------------------------------------------------------------------------------
# Talker prefill (qwen_talker_prefill, t.c:730-1038)
# ---------------------------------------------------------------------------------------

def _kv_close(a, b):
    """bf16 K/V rows: truncation can flip one unit where the f32 values differ in the
    last bits (different summation order); nothing else may differ."""
    d = np.abs(bf16_to_f64(a) - bf16_to_f64(b))
    return (a != b).mean() < 0.02 and d.max() < 0.05


def test_prefill_golden(oracle):
    from oracle.oracle import talker_from_tensors
    from qwen3_tts_amd import synth
    g = gold("golden_tiny_prefill.npz")
    s = synth.SHAPES["tiny"]
    ot, keep = talker_from_tensors(oracle, _tiny_tensors(), s, "bf16", 64, g["rope_cos"], g["rope_sin"])
    dx = oracle.talker_prefill(ot, g["embeds"])
    n = g["embeds"].shape[0]
    assert rel_l2(dx, g["dec_x_bf16"]) <= 1e-4 and np.abs(dx - g["dec_x_bf16"]).max() <= 2e-3
    assert _kv_close(keep["kv_k"][:, :n], g["kv_k_bf16"]) and _kv_close(keep["kv_v"][:, :n], g["kv_v_bf16"])
    # the reference's prefill reads the bf16 weights whatever the decode precision
    assert np.array_equal(g["dec_x_bf16"], g["dec_x_int8"]) and np.array_equal(g["kv_k_bf16"], g["kv_k_int8"])


def test_prefill_layer0_kv_equals_decode_steps(oracle):
    """Position s of a prefill and decode step s see the same layer-0 input and do the
    same arithmetic up to the KV append, so layer 0's K/V rows agree bit for bit; deeper
    layers differ only through the attention (f32 K/V in the prefill, bf16 cache in the
    decode), which the dec_x tolerance bounds."""
    from oracle.oracle import talker_from_tensors
    from qwen3_tts_amd import synth
    g = gold("golden_tiny_prefill.npz")
    s = synth.SHAPES["tiny"]
    t = _tiny_tensors()
    e = g["embeds"][:12]
    op, kp = talker_from_tensors(oracle, t, s, "bf16", 64, g["rope_cos"], g["rope_sin"])
    od, kd = talker_from_tensors(oracle, t, s, "bf16", 64, g["rope_cos"], g["rope_sin"])
    dx_p = oracle.talker_prefill(op, e)
    for i in range(e.shape[0]):
        _, dx_d = oracle.talker_step(od, e[i], i)
    assert np.array_equal(kp["kv_k"][0, :12], kd["kv_k"][0, :12]) and np.array_equal(kp["kv_v"][0, :12], kd["kv_v"][0, :12])
    assert rel_l2(dx_p, dx_d) <= 2e-2


def test_attention_f32_matches_bf16_twin_on_bf16_values(oracle):
    """On K/V that are exactly bf16, the f32-K/V attention equals the bf16-cache one."""
    from qwen3_tts_amd import synth
    rng = np.random.default_rng(3)
    nh, nkv, hd, sq = 4, 2, 128, 9
    q = rng.standard_normal(sq * nh * hd).astype(np.float32)
    kb = synth.f32_to_bf16_rne(rng.standard_normal((sq, nkv * hd)).astype(np.float32))
    vb = synth.f32_to_bf16_rne(rng.standard_normal((sq, nkv * hd)).astype(np.float32))
    a = oracle.attention(q, kb, vb, sq, sq, nh, nkv, hd, 0.0883883, 0)
    b = oracle.attention_f32(q, bf16_to_f64(kb).astype(np.float32), bf16_to_f64(vb).astype(np.float32),
                             sq, sq, nh, nkv, hd, 0.0883883, 0)
    assert np.array_equal(a, b)


@need_ref
def test_prefill_vs_reference_live(oracle):
    """The oracle prefill against the compiled reference's, at another length and on
    other inputs than the fixture."""
    from conftest import model_dir
    from oracle.oracle import RefModel, oracle_talker
    d, shape, t = model_dir("tiny")
    ref = RefModel(d, shape, prec="bf16", threads=4)
    rng = np.random.default_rng(11)
    e = rng.normal(0, 0.7, (37, shape.hidden)).astype(np.float32)
    dx_r = ref.prefill(e)
    kr, vr = ref.kv()
    ot, keep = oracle_talker(ref, 0, 64)
    dx_o = oracle.talker_prefill(ot, e)
    assert rel_l2(dx_o, dx_r) <= 1e-4
    assert _kv_close(keep["kv_k"][:, :37], np.array(kr[:, :37])) and _kv_close(keep["kv_v"][:, :37], np.array(vr[:, :37]))


# --------------------------------------------------------------------------- sampling

def _ref_sample(L, case):
    lg = np.array(case["logits"], np.float32, copy=True)
    if case["rule"] is not None:
        pytest.skip("rule cases are checked on the oracle only")
    pv = np.ascontiguousarray(case["prev"], np.int32)
    sd = np.array([case["seed"]], np.uint32)
    t = L.ref_sample(lg.ctypes.data, lg.size, case["temp"], case["top_k"], case["top_p"], case["rep"],
                     pv.ctypes.data if pv.size else None, pv.size, sd.ctypes.data)
    return t, int(sd[0])


@need_ref
def test_sample_oracle_matches_reference(oracle):
    """qo_sample against the compiled reference's qwen_tts_sample (built -O3 -ffast-math,
    so its loops may be vectorised): the same LCG state always, the same token unless
    the draw lies within rounding of a cumulative boundary."""
    from oracle.oracle import RefModel
    L = RefModel.load_lib()
    n = diff = 0
    for case in sample_cases(600, 5):
        t_ref, s_ref = _ref_sample(L, case)
        t, s, dist = oracle.sample(case["logits"], case["temp"], case["top_k"], case["top_p"], case["rep"],
                                   case["prev"], case["seed"])
        n += 1
        assert s == s_ref
        if t != t_ref:
            diff += 1
            assert dist is not None and draw_margin(dist, s) < 1e-5, (case["temp"], case["top_k"], case["top_p"])
    assert diff <= n // 100, diff


def test_sample_oracle_closed_forms(oracle):
    rng = np.random.default_rng(3)
    for _ in range(50):
        V = int(rng.integers(2, 3000))
        lg = (rng.standard_normal(V) * 2).astype(np.float32)
        am = int(np.argmax(lg))
        sd = int(rng.integers(0, 2 ** 32))
        # greedy: argmax, state untouched
        assert oracle.sample(lg, 0.0, 0, 1.0, 1.0, (), sd)[:2] == (am, sd)
        # top-k 1 and a vanishing top-p leave only the maximum; the state advances once
        adv = (sd * 1103515245 + 12345) & 0xFFFFFFFF
        assert oracle.sample(lg, 0.9, 1, 1.0, 1.0, (), sd)[:2] == (am, adv)
        assert oracle.sample(lg, 0.9, 0, 1e-6, 1.0, (), sd)[:2] == (am, adv)
        # a large repetition penalty on a positive maximum hands greedy the runner-up
        lp = lg.copy(); lp[am] = abs(lp[am]) + 1.0
        second = int(np.argsort(-lp, kind="stable")[1])
        assert oracle.sample(lp, 0.0, 0, 1.0, 1e6, np.array([am], np.int32), sd)[0] == second
    # the draw follows the distribution: 4 tokens, many seeds
    lg = np.log(np.array([0.1, 0.2, 0.3, 0.4], np.float32))
    cnt = np.zeros(4)
    sd = 1
    for _ in range(20000):
        t, sd, _ = oracle.sample(lg, 1.0, 0, 1.0, 1.0, (), sd)
        cnt[t] += 1
    assert np.abs(cnt / cnt.sum() - [0.1, 0.2, 0.3, 0.4]).max() < 0.02
    # codec-head rule: specials masked, EOS masked before frame 2, boosted after
    lg = np.zeros(3072, np.float32); lg[2500] = 50; lg[2150] = 40; lg[7] = 30
    assert oracle.sample(lg, 0.0, 0, 1.0, 1.0, (), 1, rule=(0, 0.0))[0] == 7
    assert oracle.sample(lg, 0.0, 0, 1.0, 1.0, (), 1, rule=(5, 0.0))[0] == 2150
    lg[7] = 45
    assert oracle.sample(lg, 0.0, 0, 1.0, 1.0, (), 1, rule=(5, 0.0))[0] == 7
    assert oracle.sample(lg, 0.0, 0, 1.0, 1.0, (), 1, rule=(5, 6.0))[0] == 2150
