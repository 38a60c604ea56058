"""Seeded synthetic Qwen3-TTS Talker + Code-Predictor weights in the reference layout.

The reference has no real weights offline, so every parity test and benchmark runs on
random-init weights of the real architecture.  This module produces them:

* linear / embedding weights ~ N(0, 0.02), rounded f32 -> bf16 round-to-nearest-even
  (the conversion a checkpoint writer applies; ingot ``src/dtype.c:277-284``);
* RMSNorm gains: 1.0 (HF init) by default, or ``1 + N(0, gain_jitter)`` so that tests
  can tell one norm vector from another;
* tensor names and shapes of the reference loader (``qwen_tts_talker.c:330-376``,
  ``qwen_tts_code_predictor.c:404-486``), gate|up kept as two tensors (the loader
  interleaves them, ``qwen_tts_talker.c:378-388``).

Every tensor gets its own generator seeded by ``(seed, tensor-index)`` so generation
can run on a thread pool and still be bit-identical run to run and box to box.

``write_model_dir`` writes ``model.safetensors`` (hand-rolled writer: 8-byte header
length, JSON header, raw little-endian payload) for the reference loader to mmap.
"""
from __future__ import annotations

import json
import os
import struct
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, asdict

import numpy as np


@dataclass(frozen=True)
class ModelShape:
    """Talker + CP dimensions (``qwen_tts.h:82-119``)."""
    hidden: int = 1024
    layers: int = 28
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    inter: int = 3072
    codec_vocab: int = 3072
    codebook: int = 2048
    text_hidden: int = 2048
    cp_hidden: int = 1024
    cp_layers: int = 5
    cp_heads: int = 16
    cp_kv_heads: int = 8
    cp_head_dim: int = 128
    cp_inter: int = 3072
    eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def q_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    def as_cfg(self):
        return asdict(self)


SHAPE_06B = ModelShape()
SHAPE_17B = ModelShape(hidden=2048, inter=6144)
# Small shape used by golden fixtures and quick parity tests: same head geometry
# (head_dim 128, GQA 2:1) and the same vocab rules, far fewer bytes.
SHAPE_TINY = ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, inter=512,
                        text_hidden=64, cp_hidden=256, cp_layers=2, cp_heads=4, cp_kv_heads=2,
                        cp_head_dim=128, cp_inter=512)
# Two-layer models with the real per-layer dimensions (so the tuned kernels run) for
# fast parity runs: "mini" = 0.6B layer geometry, "mini17" = 1.7B layer geometry
# (hidden 2048, so the CP gets its small_to_mtp_projection).
SHAPE_MINI = ModelShape(layers=2, cp_layers=2)
SHAPE_MINI17 = ModelShape(hidden=2048, inter=6144, layers=2, cp_layers=2)
SHAPES = {"0.6B": SHAPE_06B, "1.7B": SHAPE_17B, "tiny": SHAPE_TINY, "mini": SHAPE_MINI,
          "mini17": SHAPE_MINI17}


def f32_to_bf16_rne(a: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def tensor_specs(s: ModelShape):
    """Ordered list of (name, shape, kind) where kind is 'w' (N(0,.02)), 'n' (norm gain),
    'z' (zeros) or 'b' (bias, N(0,.02))."""
    out = []
    out.append(("talker.model.text_embedding.weight", (16, s.text_hidden), "z"))
    out.append(("talker.codec_head.weight", (s.codec_vocab, s.hidden), "w"))
    out.append(("talker.model.codec_embedding.weight", (s.codec_vocab, s.hidden), "w"))
    out.append(("talker.model.norm.weight", (s.hidden,), "n"))
    for i in range(s.layers):
        p = f"talker.model.layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (s.q_dim, s.hidden), "w"),
            (p + "self_attn.k_proj.weight", (s.kv_dim, s.hidden), "w"),
            (p + "self_attn.v_proj.weight", (s.kv_dim, s.hidden), "w"),
            (p + "self_attn.o_proj.weight", (s.hidden, s.q_dim), "w"),
            (p + "self_attn.q_norm.weight", (s.head_dim,), "n"),
            (p + "self_attn.k_norm.weight", (s.head_dim,), "n"),
            (p + "input_layernorm.weight", (s.hidden,), "n"),
            (p + "post_attention_layernorm.weight", (s.hidden,), "n"),
            (p + "mlp.gate_proj.weight", (s.inter, s.hidden), "w"),
            (p + "mlp.up_proj.weight", (s.inter, s.hidden), "w"),
            (p + "mlp.down_proj.weight", (s.hidden, s.inter), "w"),
        ]
    cq = s.cp_heads * s.cp_head_dim
    ckv = s.cp_kv_heads * s.cp_head_dim
    emb_dim = s.hidden  # CP codec embeddings live in the Talker hidden size
    out.append(("talker.code_predictor.model.norm.weight", (s.cp_hidden,), "n"))
    for i in range(s.cp_layers):
        p = f"talker.code_predictor.model.layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (cq, s.cp_hidden), "w"),
            (p + "self_attn.k_proj.weight", (ckv, s.cp_hidden), "w"),
            (p + "self_attn.v_proj.weight", (ckv, s.cp_hidden), "w"),
            (p + "self_attn.o_proj.weight", (s.cp_hidden, cq), "w"),
            (p + "self_attn.q_norm.weight", (s.cp_head_dim,), "n"),
            (p + "self_attn.k_norm.weight", (s.cp_head_dim,), "n"),
            (p + "input_layernorm.weight", (s.cp_hidden,), "n"),
            (p + "post_attention_layernorm.weight", (s.cp_hidden,), "n"),
            (p + "mlp.gate_proj.weight", (s.cp_inter, s.cp_hidden), "w"),
            (p + "mlp.up_proj.weight", (s.cp_inter, s.cp_hidden), "w"),
            (p + "mlp.down_proj.weight", (s.cp_hidden, s.cp_inter), "w"),
        ]
    for g in range(15):
        out.append((f"talker.code_predictor.lm_head.{g}.weight", (s.codebook, s.cp_hidden), "w"))
        out.append((f"talker.code_predictor.model.codec_embedding.{g}.weight",
                    (s.codebook, emb_dim), "w"))
    if s.hidden != s.cp_hidden:
        out.append(("talker.code_predictor.small_to_mtp_projection.weight",
                    (s.cp_hidden, s.hidden), "w"))
        out.append(("talker.code_predictor.small_to_mtp_projection.bias", (s.cp_hidden,), "b"))
    return out


def _gen_one(seed: int, idx: int, shape, kind: str, gain_jitter: float) -> np.ndarray:
    n = int(np.prod(shape))
    if kind == "z":
        return np.zeros(shape, dtype=np.uint16)
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed & 0xFFFFFFFF, idx])))
    if kind == "n":
        if gain_jitter == 0.0:
            return f32_to_bf16_rne(np.ones(n, dtype=np.float32)).reshape(shape)
        g = 1.0 + gain_jitter * rng.standard_normal(n, dtype=np.float32)
        return f32_to_bf16_rne(g).reshape(shape)
    a = rng.standard_normal(n, dtype=np.float32)
    a *= np.float32(0.02)
    return f32_to_bf16_rne(a).reshape(shape)


def generate(shape: ModelShape, seed: int = 0x5EED0001, gain_jitter: float = 0.0,
             threads: int = 8, only=None) -> dict:
    """Return {name: uint16 bf16-bit array}.  ``only`` optionally filters names."""
    specs = tensor_specs(shape)
    jobs = [(i, n, shp, k) for i, (n, shp, k) in enumerate(specs) if only is None or only(n)]
    out = {}
    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        futs = {ex.submit(_gen_one, seed, i, shp, k, gain_jitter): n for (i, n, shp, k) in jobs}
        for f, n in futs.items():
            out[n] = f.result()
    return out


def write_safetensors(path: str, tensors: dict, metadata=None):
    """Minimal safetensors writer: all tensors stored as BF16 (uint16 bit patterns)."""
    header = {}
    off = 0
    names = list(tensors.keys())
    for n in names:
        a = tensors[n]
        nb = a.size * 2
        header[n] = {"dtype": "BF16", "shape": list(a.shape), "data_offsets": [off, off + nb]}
        off += nb
    if metadata:
        header["__metadata__"] = {k: str(v) for k, v in metadata.items()}
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for n in names:
            f.write(np.ascontiguousarray(tensors[n], dtype=np.uint16).tobytes())


def write_model_dir(d: str, shape: ModelShape, seed: int = 0x5EED0001, gain_jitter: float = 0.0,
                    threads: int = 8, tensors=None):
    os.makedirs(d, exist_ok=True)
    if tensors is None:
        tensors = generate(shape, seed, gain_jitter, threads)
    write_safetensors(os.path.join(d, "model.safetensors"), tensors,
                      {"seed": seed, "gain_jitter": gain_jitter})
    with open(os.path.join(d, "shape.json"), "w") as f:
        json.dump({"shape": shape.as_cfg(), "seed": seed, "gain_jitter": gain_jitter}, f)
    return tensors


def interleave_gate_up(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """Rows [g0, u0, g1, u1, ...] (``qwen_tts_talker.c:378-388``)."""
    inter, h = gate.shape
    gu = np.empty((2 * inter, h), dtype=gate.dtype)
    gu[0::2] = gate
    gu[1::2] = up
    return gu


def rope_tables(head_dim: int, theta: float, npos: int):
    """NeoX cos/sin tables the way the Talker loader builds them
    (``qwen_tts_talker.c:478-495``): inv_freq[i] = 1/powf(theta, 2i/hd) in f32,
    angle = (float)pos * inv_freq[i].  numpy's float32 pow/cos/sin are not glibc's,
    so these tables are an approximation used only where the bits do not matter
    (benchmark weights); parity runs take the reference loader's own tables."""
    half = head_dim // 2
    i = np.arange(half, dtype=np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta), (2 * i).astype(np.float32) / np.float32(head_dim))).astype(np.float32)
    pos = np.arange(npos, dtype=np.float32)[:, None]
    ang = (pos * inv[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
