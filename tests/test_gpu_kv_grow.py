"""Device KV capacity growth (qwen_hip_talker_grow_kv, the reference's kv_cache_grow,
qwen_tts_talker.c:257-280): the capacity doubles when a step needs a position past it, the
cache is copied on the device, and the decode goes on with a fused kernel.

Parity is against states that never grow: a state whose cache starts at the grown capacity
runs the same kernels on the same cache, so tokens and hidden states are equal to the bit.
Across 4096 positions the role-specialised kernel hands over to the single-role one; the
continuation is then checked against a fresh single-role state given the same cache rows."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from qwen3_tts_amd import hip, synth  # noqa: E402

_W = {}


def _weights():
    if "t" not in _W:
        s = synth.SHAPES["mini17"]
        t = synth.generate(s, 0x5EED0007, 0.1, threads=8, only=lambda n: not n.startswith("talker.code_predictor."))
        _W["t"] = (s, t, hip.layers_from_tensors(t, s))
    return _W["t"]


def _state(kv_max):
    s, t, layers = _weights()
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, 8192)
    fnorm = synth.bf16_to_f32(t["talker.model.norm.weight"])
    return hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, kv_max, quantize_to=hip.INT8)


def _heads():
    _, t, _ = _weights()
    return (np.ascontiguousarray(t["talker.codec_head.weight"]),
            np.ascontiguousarray(t["talker.model.codec_embedding.weight"]))


def test_kv_grow_greedy_tokens_unchanged():
    """Greedy loop: 50 steps in a 64-position cache, then 150 more (the cache grows to 256
    before the launch), equal to the bit to 200 steps in a 256-position cache."""
    print("[case] kv grow: greedy 64 -> 256 positions, mini17 int8", flush=True)
    L = hip.lib()
    head, emb = _heads()
    e0 = synth.bf16_to_f32(emb[321])
    b = _state(256)
    want, hb = b.greedy(head, emb, e0, 0, 0, 200)
    b.free()
    a = _state(64)
    assert L.qwen_hip_talker_fused_kernel(a.h) == 2 and L.qwen_hip_talker_kv_max(a.h) == 64
    t1, _ = a.greedy(head, emb, e0, 0, 0, 50)
    t2, ha = a.greedy(head, emb, synth.bf16_to_f32(emb[t1[-1]]), 50, 50, 150)
    assert L.qwen_hip_talker_kv_max(a.h) == 256 and L.qwen_hip_talker_fused_kernel(a.h) == 2
    a.free()
    assert list(t1) + list(t2) == list(want)
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))


def test_kv_grow_single_steps_bitwise():
    """Host-driven steps (qwen_hip_talker_step grows first, as qwen_talker_step does): a
    32-position cache stepped to position 99 grows 32 -> 64 -> 128; every step's hidden
    state equals a 128-position state's to the bit."""
    print("[case] kv grow: single steps 32 -> 128 positions, mini17 int8", flush=True)
    L = hip.lib()
    head, emb = _heads()
    a, b = _state(32), _state(128)
    rng = np.random.default_rng(5)
    caps = []
    try:
        for pos in range(100):
            e = synth.bf16_to_f32(emb[int(rng.integers(0, 2048))])
            ha, hb = a.step(e, pos), b.step(e, pos)
            assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32)), pos
            caps.append(L.qwen_hip_talker_kv_max(a.h))
    finally:
        a.free(); b.free()
    assert caps[31] == 32 and caps[32] == 64 and caps[64] == 128


def test_kv_grow_across_4096_hands_over_to_single_role_kernel():
    """A 4096-position cache filled to 4090 (upload), 4 greedy steps on the role-specialised
    kernel, then 8 more: the cache grows to 8192 and the single-role persistent kernel takes
    over.  The grown cache holds the same bits (download), and the 8 steps equal those of a
    fresh 8192-position state given that cache."""
    print("[case] kv grow: 4096 -> 8192 positions, role kernel -> single-role kernel", flush=True)
    L = hip.lib()
    s, _, _ = _weights()
    head, emb = _heads()
    rng = np.random.default_rng(9)
    n0 = 4090
    kvk = synth.f32_to_bf16_rne(rng.normal(0, 1.0, (s.layers, n0, s.kv_dim)).astype(np.float32))
    kvv = synth.f32_to_bf16_rne(rng.normal(0, 0.1, (s.layers, n0, s.kv_dim)).astype(np.float32))
    e0 = synth.bf16_to_f32(emb[77])
    a = _state(4096)
    try:
        assert L.qwen_hip_talker_fused_kernel(a.h) == 2
        a.upload_kv(kvk, kvv, n0)
        t1, _ = a.greedy(head, emb, e0, n0, 0, 4)
        before = a.download_kv(n0 + 4)
        e1 = synth.bf16_to_f32(emb[t1[-1]])
        t2, ha = a.greedy(head, emb, e1, n0 + 4, 4, 8)
        assert L.qwen_hip_talker_kv_max(a.h) == 8192 and L.qwen_hip_talker_fused_kernel(a.h) == 1
        after = a.download_kv(n0 + 4)
    finally:
        a.free()
    assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])
    b = _state(8192)
    try:
        assert L.qwen_hip_talker_fused_kernel(b.h) == 1
        b.upload_kv(np.ascontiguousarray(before[0]), np.ascontiguousarray(before[1]), n0 + 4)
        w2, hb = b.greedy(head, emb, e1, n0 + 4, 4, 8)
    finally:
        b.free()
    assert list(t2) == list(w2)
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))


def test_kv_grow_limits():
    L = hip.lib()
    a = _state(64)
    try:
        assert L.qwen_hip_talker_grow_kv(a.h, 10) == 0 and L.qwen_hip_talker_kv_max(a.h) == 64
        assert L.qwen_hip_talker_grow_kv(a.h, 8193) == -1
        assert "8192" in hip.last_error()
        assert L.qwen_hip_talker_grow_kv(a.h, 100) == 0 and L.qwen_hip_talker_kv_max(a.h) == 128
    finally:
        a.free()
