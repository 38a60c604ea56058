"""Write the golden fixtures under tests/golden/ from the compiled reference.

    python tests/golden/make_golden.py        # needs oracle/_ref/libqwen_ref.so (make -C oracle ref)
    python tests/golden/make_golden.py --only-prefill   # just golden_tiny_prefill.npz

The reference commits no vectors for the decode path (its tests need real weights), so
these fixtures are the reference's own outputs on seeded synthetic inputs, produced by
the reference C sources compiled by oracle/Makefile (ref_harness.c drives them):

  golden_convert.npz  f16 -> f32 of every subnormal/special half (qwen_tts_kernels.h:162-179),
                      f32 -> f16 of edge values (qwen_tts_kernels.h:180-201)
  golden_quant.npz    int8 row quantizer (qwen_tts_kernels.c:2143-2238) and q4_0 weighted-LSQ
                      quantizer (qwen_tts_kernels.c:2662-2726) on crafted matrices
  golden_ops.npz      matvec bf16/int8/q4_0 129x320 (k.c:1091, :2548, :3195), causal
                      attention over a bf16 KV (k.c:3704-3846), rms_norm (k.c:292), swiglu
  golden_tiny_<p>.npz the "tiny" synthetic model (seed 0x5EED0001): 8 Talker decode steps
                      (qwen_talker_step, t.c:537-699) and 3 Code-Predictor frames
                      (qwen_cp_predict, cp.c:926-1045) per precision p in bf16/int8/int4
  golden_tiny_prefill.npz  the same model's Talker prefill (qwen_talker_prefill,
                      t.c:730-1038) of 24 positions: the inputs, every layer's K/V rows and
                      dec_x, with the reference loaded as bf16 and as int8 (its prefill reads
                      the bf16 weights either way)

Only data is written (inputs, expected outputs, a hash of the synthetic weights); the
tests regenerate the weights from the seed with qwen3_tts_amd.synth and run the oracle.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import conftest  # noqa: E402  (imports the package as qwen3_tts_amd)
from oracle.oracle import RefModel, _p  # noqa: E402
from qwen3_tts_amd import synth  # noqa: E402

SEED_W = 0x5EED0001
TINY_STEPS = 8
TINY_FRAMES = 3


def tensor_hash(tens) -> str:
    h = hashlib.sha256()
    for k in sorted(tens):
        h.update(k.encode())
        h.update(np.ascontiguousarray(tens[k]).tobytes())
    return h.hexdigest()


def bf16(a):
    return synth.f32_to_bf16_rne(np.asarray(a, np.float32))


def convert_fixture(L):
    halves = [h for h in range(65536) if (h & 0x7C00) == 0 or (h & 0x7C00) == 0x7C00]
    halves += list(range(0x0400, 0x0410)) + [0x3C00, 0xBC00, 0x7BFF, 0xFBFF]
    halves = np.array(sorted(set(halves)), np.uint16)
    f16_f32 = np.array([L.ref_f16_to_f32(int(h)) for h in halves], np.float32)

    rng = np.random.default_rng(0x601D0001)
    vals = [0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65519.0, 65520.0, 65536.0, 1e-8, 5.96e-8,
            2.98e-8, 2.9802322e-08, 6.1035156e-05, 6.097555e-05, 1.0, -1.0]
    # exact ties: halfway between adjacent halves, normal and subnormal
    for h in list(range(0x0001, 0x0400, 37)) + list(range(0x0400, 0x7BFF, 509)):
        a = float(np.array([h], np.uint16).view(np.float16)[0])
        b = float(np.array([h + 1], np.uint16).view(np.float16)[0])
        vals += [(a + b) / 2, -(a + b) / 2]
    vals += list(rng.normal(0, 1, 1500)) + list(rng.normal(0, 3e-5, 500)) + list(rng.uniform(-7e4, 7e4, 300))
    f32_in = np.array(vals, np.float32)
    f32_f16 = np.array([L.ref_f32_to_f16(float(v)) for v in f32_in], np.uint16)
    return dict(halves=halves, f16_to_f32=f16_f32.view(np.uint32), f32_in=f32_in, f32_to_f16=f32_f16)


def quant_fixture(L):
    rng = np.random.default_rng(0x601D0002)
    # int8, body-only width (320 = 40 x 8) with special rows
    w = rng.normal(0, 0.02, (40, 320)).astype(np.float32)
    w[0] = 0.0                                   # zero row: scale 0, q 0
    w[1] = 0.0; w[1, 17] = -0.5                   # single value
    w[2] = np.arange(320) % 9 - 4.0; w[2, 0] = 127.0   # amax 127: v*inv lands on integers
    w[3] = (np.arange(320) % 11 - 5) + 0.5; w[3, 5] = 127.0  # .5 ties
    w8a = bf16(w)
    # int8 with a tail (37 = 4 x 8 + 5): the reference rounds the tail with roundf
    w = rng.normal(0, 0.02, (8, 37)).astype(np.float32)
    w[0] = (np.arange(37) % 7 - 3) + 0.5; w[0, 0] = 127.0
    w8b = bf16(w)
    out = {}
    for tag, src in (("a", w8a), ("b", w8b)):
        r, c = src.shape
        q = np.empty((r, c), np.int8); s = np.empty(r, np.float32)
        L.ref_quantize_int8(_p(src), r, c, _p(q), _p(s))
        out[f"i8_{tag}_w"] = src; out[f"i8_{tag}_q"] = q; out[f"i8_{tag}_s"] = s
    # q4_0 with crafted blocks
    w = rng.normal(0, 0.02, (24, 256)).astype(np.float32)
    w[0, :32] = 0.0                               # zero block
    w[1, :32] = 0.01; w[1, 3] = -0.04; w[1, 9] = 0.04   # |max| tie: first index wins
    w[2, 32:64] = np.linspace(-0.08, 0.08, 32)
    w[3] = rng.standard_t(2, 256) * 0.01          # heavy tails
    w4 = bf16(w)
    blocks = np.empty((24, 256 // 32, 18), np.uint8)
    L.ref_quantize_q4_0(_p(w4), 24, 256, _p(blocks))
    out["q4_w"] = w4; out["q4_blocks"] = blocks
    return out


def ops_fixture(L):
    rng = np.random.default_rng(0x601D0003)
    rows, cols = 129, 320
    W = bf16(rng.normal(0, 0.02, (rows, cols)))
    x = rng.normal(0, 1, cols).astype(np.float32)
    out = {"mv_W": W, "mv_x": x}
    y = np.empty(rows, np.float32)
    L.ref_matvec_bf16(_p(y), _p(W), _p(x), rows, cols); out["mv_y_bf16"] = y.copy()
    q = np.empty((rows, cols), np.int8); s = np.empty(rows, np.float32)
    L.ref_quantize_int8(_p(W), rows, cols, _p(q), _p(s))
    L.ref_matvec_int8(_p(y), _p(q), _p(s), _p(x), rows, cols); out["mv_y_int8"] = y.copy()
    out["mv_q8"] = q; out["mv_s8"] = s
    blocks = np.empty((rows, cols // 32, 18), np.uint8)
    L.ref_quantize_q4_0(_p(W), rows, cols, _p(blocks))
    L.ref_matvec_q4_0(_p(y), _p(blocks), _p(x), rows, cols); out["mv_y_q4"] = y.copy()
    out["mv_q4"] = blocks
    # attention: 4 heads over 2 kv heads, head_dim 128, 37 keys, one query at offset 36
    nh, nkv, hd, sk = 4, 2, 128, 37
    Q = rng.normal(0, 1, nh * hd).astype(np.float32)
    K = bf16(rng.normal(0, 1, (sk, nkv * hd)))
    V = bf16(rng.normal(0, 1, (sk, nkv * hd)))
    o = np.empty(nh * hd, np.float32)
    sc = np.float32(1.0 / np.sqrt(hd))
    L.ref_attention_bf16kv(_p(o), _p(Q), _p(K), _p(V), 1, sk, nh, nkv, hd, float(sc), sk - 1)
    out.update(at_Q=Q, at_K=K, at_V=V, at_out=o)
    # rms norm and swiglu
    xr = rng.normal(0, 2, 1024).astype(np.float32)
    wr = (1 + rng.normal(0, 0.1, 1024)).astype(np.float32)
    yr = np.empty(1024, np.float32)
    L.ref_rms_norm(_p(yr), _p(xr), _p(wr), 1, 1024, 1e-6)
    out.update(rn_x=xr, rn_w=wr, rn_y=yr)
    gu = rng.normal(0, 3, 2 * 512).astype(np.float32)
    g2 = gu.copy()
    L.ref_swiglu(_p(g2), 512)
    out.update(sw_in=gu, sw_out=g2[:512].copy())
    return out


def tiny_fixture(prec, d, shape, tens):
    ref = RefModel(d, shape, prec=prec, threads=1)
    rng = np.random.default_rng(0x5EED0002)
    toks = rng.integers(0, 2048, TINY_STEPS).astype(np.int32)
    emb = ref.codec_emb()
    hid = np.empty((TINY_STEPS, shape.hidden), np.float32)
    dx = np.empty_like(hid)
    for i, t in enumerate(toks):
        e = synth.bf16_to_f32(emb[t])
        hid[i] = ref.step(e)
        dx[i] = ref.dec_x()
    kk, vv = ref.kv()
    cos, sin = ref.rope()
    ccos, csin = ref.cp_rope()
    fr_h = rng.normal(0, 1, (TINY_FRAMES, shape.hidden)).astype(np.float32)
    fr_c = rng.integers(0, 2048, TINY_FRAMES).astype(np.int32)
    codes = np.stack([ref.cp_predict(fr_h[i], int(fr_c[i])) for i in range(TINY_FRAMES)])
    return dict(tokens=toks, hidden=hid, dec_x=dx, kv_k=np.array(kk[:, :TINY_STEPS]), kv_v=np.array(vv[:, :TINY_STEPS]),
                rope_cos=np.array(cos[:64]), rope_sin=np.array(sin[:64]),
                cp_rope_cos=np.array(ccos[:16]), cp_rope_sin=np.array(csin[:16]),
                frame_hidden=fr_h, frame_code0=fr_c, frame_codes=codes,
                weights_sha256=np.array(tensor_hash(tens)))


PREFILL_SEQ = 24


def prefill_fixture(d, shape):
    rng = np.random.default_rng(0x5EED0003)
    out = {}
    for prec in ("bf16", "int8"):
        ref = RefModel(d, shape, prec=prec, threads=1)
        if prec == "bf16":
            emb = ref.codec_emb()
            toks = rng.integers(0, 2048, PREFILL_SEQ // 2)
            e = np.concatenate([synth.bf16_to_f32(emb[toks]),
                                rng.normal(0, 0.5, (PREFILL_SEQ - toks.size, shape.hidden))]).astype(np.float32)
            out["embeds"] = e
        dx = ref.prefill(out["embeds"])
        assert ref.kv_len == PREFILL_SEQ
        kk, vv = ref.kv()
        out[f"dec_x_{prec}"] = dx
        out[f"kv_k_{prec}"] = np.array(kk[:, :PREFILL_SEQ])
        out[f"kv_v_{prec}"] = np.array(vv[:, :PREFILL_SEQ])
    cos, sin = ref.rope()
    out["rope_cos"] = np.array(cos[:64]); out["rope_sin"] = np.array(sin[:64])
    return out


def main():
    L = RefModel.load_lib()
    if "--only-prefill" in sys.argv:
        shape = synth.SHAPES["tiny"]
        tens = synth.generate(shape, SEED_W, 0.1, threads=8)
        with tempfile.TemporaryDirectory() as td:
            d = os.path.join(td, "tiny")
            synth.write_model_dir(d, shape, SEED_W, 0.1, tensors=tens)
            np.savez_compressed(os.path.join(HERE, "golden_tiny_prefill.npz"), **prefill_fixture(d, shape))
        return
    np.savez_compressed(os.path.join(HERE, "golden_convert.npz"), **convert_fixture(L))
    np.savez_compressed(os.path.join(HERE, "golden_quant.npz"), **quant_fixture(L))
    np.savez_compressed(os.path.join(HERE, "golden_ops.npz"), **ops_fixture(L))
    shape = synth.SHAPES["tiny"]
    tens = synth.generate(shape, SEED_W, 0.1, threads=8)
    with tempfile.TemporaryDirectory() as td:
        d = os.path.join(td, "tiny")
        synth.write_model_dir(d, shape, SEED_W, 0.1, tensors=tens)
        for prec in ("bf16", "int8", "int4"):
            np.savez_compressed(os.path.join(HERE, f"golden_tiny_{prec}.npz"), **tiny_fixture(prec, d, shape, tens))
        np.savez_compressed(os.path.join(HERE, "golden_tiny_prefill.npz"), **prefill_fixture(d, shape))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
