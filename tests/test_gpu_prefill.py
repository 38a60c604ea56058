"""GPU parity of the Talker prefill (qwen_talker_prefill, qwen_tts_talker.c:730-1038).

The projection GEMM against an f64 product (the three exact bf16 planes make it an f32
sum of exact products, so it is held to f32 accuracy); the whole prefill against the
compiled reference's outputs (golden fixture, tiny model) and against the oracle's
prefill at the 0.6B/1.7B layer shapes; the decode continuing from a device prefill
against the oracle continuing from its own.
"""
import numpy as np
import pytest

from conftest import model_dir, rel_l2

pytestmark = pytest.mark.gpu

from qwen3_tts_amd import hip, synth  # noqa: E402


def _gemm(W, X, epi, Y0=None):
    S, K = X.shape
    N = W.shape[0]
    ny = N // 2 if epi == 2 else N
    Y = np.zeros((S, ny), np.float32) if Y0 is None else np.array(Y0, np.float32, copy=True)
    hip.check(hip.lib().qwen_hip_op_prefill_gemm(Y.ctypes.data, np.ascontiguousarray(W).ctypes.data,
                                                 np.ascontiguousarray(X, np.float32).ctypes.data, S, N, K, epi),
              "prefill_gemm")
    return Y


@pytest.mark.parametrize("S,N,K", [(1, 64, 64), (17, 128, 256), (24, 1024, 256), (64, 4096, 2048),
                                   (100, 2048, 6144), (257, 192, 320), (200, 12288, 2048),
                                   (512, 8192, 256)])
def test_op_prefill_gemm(S, N, K):
    print(f"[case] prefill gemm S={S} N={N} K={K}", flush=True)
    rng = np.random.default_rng(S * 131 + N + K)
    W = synth.f32_to_bf16_rne((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    X = rng.standard_normal((S, K)).astype(np.float32)
    W64 = synth.bf16_to_f32(W).astype(np.float64)
    ref = X.astype(np.float64) @ W64.T
    Y = _gemm(W, X, 0)
    assert np.abs(Y - ref).max() <= 2e-6 * np.abs(ref).max() * np.sqrt(K / 64)
    Y0 = rng.standard_normal((S, N)).astype(np.float32)
    Yr = _gemm(W, X, 1, Y0)
    assert np.abs(Yr - (Y0 + ref)).max() <= 2e-6 * np.abs(ref).max() * np.sqrt(K / 64) + 1e-6
    g, u = ref[:, 0::2], ref[:, 1::2]
    sw = g / (1.0 + np.exp(-g)) * u
    Ys = _gemm(W, X, 2)
    assert np.abs(Ys - sw).max() <= 1e-5 * max(np.abs(sw).max(), 1e-3)


def test_op_prefill_gemm_planes_are_exact():
    """A weight of 1.0 at column k picks x[k] out exactly: the three bf16 planes sum to
    the f32 activation bit for bit (a two-plane split would lose the low 8 bits)."""
    K, N, S = 128, 64, 5
    W = np.zeros((N, K), np.uint16)
    for n in range(N):
        W[n, (7 * n) % K] = 0x3F80   # bf16 1.0
    rng = np.random.default_rng(9)
    X = (rng.standard_normal((S, K)) * np.exp(rng.uniform(-20, 20, (S, K)))).astype(np.float32)
    Y = _gemm(W, X, 0)
    assert np.array_equal(Y, X[:, (7 * np.arange(N)) % K])


@pytest.mark.parametrize("S,nh,nkv", [(1, 16, 8), (37, 16, 8), (100, 4, 2), (300, 16, 8), (1000, 16, 8)])
def test_op_prefill_attention(oracle, S, nh, nkv):
    """The tiled causal attention against the oracle's f32 attention (qwen_causal_attention
    restated): the VALU kernel's 16-query workgroups (S = 1, 37, 100) and the matrix-core
    kernel (S = 300, 1000)."""
    print(f"[case] prefill attention S={S} nh={nh} nkv={nkv}", flush=True)
    rng = np.random.default_rng(S + nh)
    ld = (nh + 2 * nkv) * 128
    qkv = (rng.standard_normal((S, ld)) * 1.5).astype(np.float32)
    out = np.empty((S, nh * 128), np.float32)
    sc = np.float32(1.0 / np.sqrt(128.0))
    hip.check(hip.lib().qwen_hip_op_prefill_attention(out.ctypes.data, qkv.ctypes.data, S, nh, nkv, sc), "pf_attn")
    q = np.ascontiguousarray(qkv[:, :nh * 128]); k = np.ascontiguousarray(qkv[:, nh * 128:(nh + nkv) * 128])
    v = np.ascontiguousarray(qkv[:, (nh + nkv) * 128:])
    ref = oracle.attention_f32(q, k, v, S, S, nh, nkv, 128, float(sc), 0).reshape(S, nh * 128)
    assert rel_l2(out, ref) < 2e-6 and np.abs(out - ref).max() < 1e-5


def _tiny_talker(prec_code, quantize_to=-1, kv_max=64):
    from test_cpu_oracle import gold
    d, shape, t = model_dir("tiny")
    g = gold("golden_tiny_prefill.npz")
    layers = hip.layers_from_tensors(t, shape)
    fn = synth.bf16_to_f32(t["talker.model.norm.weight"])
    return hip.Talker(shape, layers, fn, g["rope_cos"], g["rope_sin"], prec_code, kv_max, quantize_to=quantize_to), g, t


def _kv_close(a, b):
    d = np.abs(synth.bf16_to_f32(a).astype(np.float64) - synth.bf16_to_f32(b))
    return (a != b).mean() < 0.02 and d.max() < 0.05


@pytest.mark.parametrize("quant", [-1, hip.INT8])
def test_prefill_matches_reference_golden(quant):
    """The device prefill against the compiled reference's prefill (tiny model, 24
    positions): dec_x and every layer's K/V rows.  An int8 state prefills with the bf16
    weights, like the reference, so it gives the bf16 state's result bit for bit."""
    print(f"[case] prefill golden quant={quant}", flush=True)
    tk, g, _ = _tiny_talker(hip.BF16, quant)
    dx = tk.prefill(g["embeds"])
    n = g["embeds"].shape[0]
    assert rel_l2(dx, g["dec_x_bf16"]) <= 1e-5 and np.abs(dx - g["dec_x_bf16"]).max() <= 1e-4
    k, v = tk.download_kv(n)
    assert _kv_close(k[:, :n], g["kv_k_bf16"]) and _kv_close(v[:, :n], g["kv_v_bf16"])
    if quant != -1:
        tb, _, _ = _tiny_talker(hip.BF16, -1)
        dxb = tb.prefill(g["embeds"])
        kb, vb = tb.download_kv(n)
        assert np.array_equal(dx, dxb) and np.array_equal(k[:, :n], kb[:, :n]) and np.array_equal(v[:, :n], vb[:, :n])
        tb.free()
    tk.free()


def test_prefill_async_replays_reproduce_the_prefill():
    """The benchmark entry qwen_hip_talker_prefill_async replays the last prefill from its
    kept embeddings: after the cache rows are overwritten with zeros, two replays write
    back exactly the first prefill's K/V rows and dec_x."""
    print("[case] prefill async replay", flush=True)
    tk, g, _ = _tiny_talker(hip.BF16, -1)
    dx = tk.prefill(g["embeds"])
    n = g["embeds"].shape[0]
    k, v = tk.download_kv(n)
    tk.upload_kv(np.zeros_like(k[:, :n]), np.zeros_like(v[:, :n]), n)
    z, _ = tk.download_kv(n)
    assert not z[:, :n].any()
    hip.check(hip.lib().qwen_hip_talker_prefill_async(tk.h, n, 2), "prefill_async")
    hip.check(hip.lib().qwen_hip_talker_sync(tk.h), "sync")
    k2, v2 = tk.download_kv(n)
    assert np.array_equal(k2[:, :n], k[:, :n]) and np.array_equal(v2[:, :n], v[:, :n])
    assert np.array_equal(tk.dec_x(), dx)
    tk.free()


@pytest.mark.parametrize("name,seq", [("mini", 100), ("mini17", 40), ("mini", 240)])
def test_prefill_matches_oracle_layer_shapes(oracle, name, seq):
    """The 0.6B / 1.7B layer shapes (2 layers) against the oracle prefill, then one decode
    step from each side's KV.  100 and 40 positions run the VALU attention, 240 the
    matrix-core one (64 workgroups), with 16 padding rows in the O projection's planes."""
    from oracle.oracle import talker_from_tensors
    print(f"[case] prefill oracle {name} seq={seq}", flush=True)
    d, shape, t = model_dir(name)
    cos, sin = synth.rope_tables(shape.head_dim, shape.rope_theta, 256)
    layers = hip.layers_from_tensors(t, shape)
    fn = synth.bf16_to_f32(t["talker.model.norm.weight"])
    tk = hip.Talker(shape, layers, fn, cos, sin, hip.BF16, 256)
    ot, keep = talker_from_tensors(oracle, t, shape, "bf16", 256, cos, sin)
    rng = np.random.default_rng(seq)
    e = rng.normal(0, 0.5, (seq, shape.hidden)).astype(np.float32)
    dx = tk.prefill(e)
    dx_o = oracle.talker_prefill(ot, e)
    assert rel_l2(dx, dx_o) <= 1e-4, rel_l2(dx, dx_o)
    k, v = tk.download_kv(seq)
    assert _kv_close(k[:, :seq], keep["kv_k"][:, :seq]) and _kv_close(v[:, :seq], keep["kv_v"][:, :seq])
    # the decode continues from the prefilled cache
    x = rng.normal(0, 0.5, shape.hidden).astype(np.float32)
    h = tk.step(x, seq)
    h_o, _ = oracle.talker_step(ot, x, seq)
    assert rel_l2(h, h_o) <= 1e-3
    tk.free()


def test_prefill_argument_errors_leave_state_usable():
    tk, g, _ = _tiny_talker(hip.BF16, -1, kv_max=64)
    L = hip.lib()
    e = np.zeros((65, tk.H), np.float32)
    assert L.qwen_hip_talker_prefill(tk.h, None, e.ctypes.data, 65) != 0      # beyond the rope table (64)
    assert L.qwen_hip_talker_prefill(tk.h, None, None, 4) != 0               # no inputs
    dx = tk.prefill(g["embeds"])
    assert rel_l2(dx, g["dec_x_bf16"]) <= 1e-5
    tk.free()
