"""Seeded synthetic speech-decoder weights (the 12 Hz codec's decoder) in the reference layout.

The reference loads its speech decoder from the speech tokenizer's safetensors as F32
tensors (``qwen_tts_speech_decoder.c:372-578``, every tensor through ``get_f32``); this
module writes a file of the same names, shapes and dtype with random-init values scaled
so that activations stay O(1) through the whole network (weights ~ N(0, 1/fan_in),
small biases, layer scales and ConvNeXt gammas ~0.1, snake log-parameters ~N(0, 0.2)).
The architecture constants are the ones the reference's decode hard-codes
(``qwen_tts_speech_decoder.c:585-587``, ``:757-762``, ``:1158-1159``): codebook dim 256,
16 codebooks of 2048 entries, VQ hidden 512, latent 1024, an 8-layer pre-transformer of
width 512 (16 heads of 64, SwiGLU 1024), two ConvNeXt upsamplers (x2 each), then
1536 -> 768 -> 384 -> 192 -> 96 channels at upsampling rates 8, 5, 4, 3.

Each tensor has its own generator seeded by ``(seed, tensor-index)``, so files are
bit-identical run to run.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

CB_DIM, CB_SIZE, N_CB = 256, 2048, 16
VQ_HIDDEN, LATENT, DEC_HIDDEN, DEC_INTER = 512, 1024, 512, 1024
N_HEADS, HEAD_DIM, WINDOW, N_LAYERS = 16, 64, 72, 8
UP_RATES = (8, 5, 4, 3)
UP_CH = (768, 384, 192, 96)
INIT_CH = 1536
DILATIONS = (1, 3, 9)
ROPE_THETA = 10000.0
EPS = 1e-5
SAMPLES_PER_FRAME = 4 * 8 * 5 * 4 * 3          # 1920


def sd_specs():
    """[(name, shape, kind, scale)] in file order; kind: w (N(0, scale)), b (N(0, scale)),
    c (constant scale, +-10 % jitter), g (1 + N(0, scale)), u (cluster usage), e (EMA sums)."""
    out = []
    out.append(("decoder.quantizer.rvq_first.vq.layers.0._codebook.embedding_sum", (CB_SIZE, CB_DIM), "e", 1.0))
    out.append(("decoder.quantizer.rvq_first.vq.layers.0._codebook.cluster_usage", (CB_SIZE,), "u", 0.3))
    for k in range(15):
        out.append((f"decoder.quantizer.rvq_rest.vq.layers.{k}._codebook.embedding_sum", (CB_SIZE, CB_DIM), "e", 1.0))
        out.append((f"decoder.quantizer.rvq_rest.vq.layers.{k}._codebook.cluster_usage", (CB_SIZE,), "u", 0.3))
    out.append(("decoder.quantizer.rvq_first.output_proj.weight", (VQ_HIDDEN, CB_DIM), "w", CB_DIM ** -0.5))
    out.append(("decoder.quantizer.rvq_rest.output_proj.weight", (VQ_HIDDEN, CB_DIM), "w", (15 * CB_DIM) ** -0.5))
    out.append(("decoder.pre_conv.conv.weight", (LATENT, VQ_HIDDEN, 3), "w", (3 * VQ_HIDDEN) ** -0.5))
    out.append(("decoder.pre_conv.conv.bias", (LATENT,), "b", 0.02))
    pt = "decoder.pre_transformer"
    out.append((f"{pt}.input_proj.weight", (DEC_HIDDEN, LATENT), "w", LATENT ** -0.5))
    out.append((f"{pt}.input_proj.bias", (DEC_HIDDEN,), "b", 0.02))
    qd = N_HEADS * HEAD_DIM
    for i in range(N_LAYERS):
        p = f"{pt}.layers.{i}"
        out.append((f"{p}.input_layernorm.weight", (DEC_HIDDEN,), "g", 0.1))
        out.append((f"{p}.self_attn.q_proj.weight", (qd, DEC_HIDDEN), "w", DEC_HIDDEN ** -0.5))
        out.append((f"{p}.self_attn.k_proj.weight", (qd, DEC_HIDDEN), "w", DEC_HIDDEN ** -0.5))
        out.append((f"{p}.self_attn.v_proj.weight", (qd, DEC_HIDDEN), "w", DEC_HIDDEN ** -0.5))
        out.append((f"{p}.self_attn.o_proj.weight", (DEC_HIDDEN, qd), "w", qd ** -0.5))
        out.append((f"{p}.self_attn_layer_scale.scale", (DEC_HIDDEN,), "c", 0.1))
        out.append((f"{p}.post_attention_layernorm.weight", (DEC_HIDDEN,), "g", 0.1))
        out.append((f"{p}.mlp.gate_proj.weight", (DEC_INTER, DEC_HIDDEN), "w", DEC_HIDDEN ** -0.5))
        out.append((f"{p}.mlp.up_proj.weight", (DEC_INTER, DEC_HIDDEN), "w", DEC_HIDDEN ** -0.5))
        out.append((f"{p}.mlp.down_proj.weight", (DEC_HIDDEN, DEC_INTER), "w", DEC_INTER ** -0.5))
        out.append((f"{p}.mlp_layer_scale.scale", (DEC_HIDDEN,), "c", 0.1))
    out.append((f"{pt}.norm.weight", (DEC_HIDDEN,), "g", 0.1))
    out.append((f"{pt}.output_proj.weight", (LATENT, DEC_HIDDEN), "w", DEC_HIDDEN ** -0.5))
    out.append((f"{pt}.output_proj.bias", (LATENT,), "b", 0.02))
    for b in range(2):
        p = f"decoder.upsample.{b}"
        out.append((f"{p}.0.conv.weight", (LATENT, LATENT, 2), "w", LATENT ** -0.5))
        out.append((f"{p}.0.conv.bias", (LATENT,), "b", 0.02))
        out.append((f"{p}.1.dwconv.conv.weight", (LATENT, 1, 7), "w", 7 ** -0.5))
        out.append((f"{p}.1.dwconv.conv.bias", (LATENT,), "b", 0.02))
        out.append((f"{p}.1.pwconv1.weight", (4 * LATENT, LATENT), "w", LATENT ** -0.5))
        out.append((f"{p}.1.pwconv1.bias", (4 * LATENT,), "b", 0.02))
        out.append((f"{p}.1.pwconv2.weight", (LATENT, 4 * LATENT), "w", (4 * LATENT) ** -0.5))
        out.append((f"{p}.1.pwconv2.bias", (LATENT,), "b", 0.02))
        out.append((f"{p}.1.norm.weight", (LATENT,), "g", 0.1))
        out.append((f"{p}.1.norm.bias", (LATENT,), "b", 0.02))
        out.append((f"{p}.1.gamma", (LATENT,), "c", 0.1))
    out.append(("decoder.decoder.0.conv.weight", (INIT_CH, LATENT, 7), "w", (7 * LATENT) ** -0.5))
    out.append(("decoder.decoder.0.conv.bias", (INIT_CH,), "b", 0.02))
    cin = INIT_CH
    for b in range(4):
        p = f"decoder.decoder.{b + 1}.block"
        r, c = UP_RATES[b], UP_CH[b]
        out.append((f"{p}.0.alpha", (cin,), "b", 0.2))
        out.append((f"{p}.0.beta", (cin,), "b", 0.2))
        out.append((f"{p}.1.conv.weight", (cin, c, 2 * r), "w", (2 * cin) ** -0.5))
        out.append((f"{p}.1.conv.bias", (c,), "b", 0.02))
        for ri in range(2, 5):
            out.append((f"{p}.{ri}.act1.alpha", (c,), "b", 0.2))
            out.append((f"{p}.{ri}.act1.beta", (c,), "b", 0.2))
            out.append((f"{p}.{ri}.conv1.conv.weight", (c, c, 7), "w", 0.5 * (7 * c) ** -0.5))
            out.append((f"{p}.{ri}.conv1.conv.bias", (c,), "b", 0.02))
            out.append((f"{p}.{ri}.act2.alpha", (c,), "b", 0.2))
            out.append((f"{p}.{ri}.act2.beta", (c,), "b", 0.2))
            out.append((f"{p}.{ri}.conv2.conv.weight", (c, c, 1), "w", 0.5 * c ** -0.5))
            out.append((f"{p}.{ri}.conv2.conv.bias", (c,), "b", 0.02))
        cin = c
    out.append(("decoder.decoder.5.alpha", (cin,), "b", 0.2))
    out.append(("decoder.decoder.5.beta", (cin,), "b", 0.2))
    out.append(("decoder.decoder.6.conv.weight", (1, cin, 7), "w", 0.1 * (7 * cin) ** -0.5))
    out.append(("decoder.decoder.6.conv.bias", (1,), "b", 0.02))
    return out


def _gen(seed, idx, shape, kind, scale):
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed & 0xFFFFFFFF, 0x5D, idx])))
    n = int(np.prod(shape))
    if kind == "c":
        a = np.float32(scale) * (1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32))
    elif kind == "g":
        a = 1.0 + np.float32(scale) * rng.standard_normal(n, dtype=np.float32)
    elif kind == "u":
        a = np.exp(np.float32(scale) * rng.standard_normal(n, dtype=np.float32)) * np.float32(4.0)
    else:   # w, b, e
        a = rng.standard_normal(n, dtype=np.float32) * np.float32(scale)
    return np.ascontiguousarray(a.astype(np.float32).reshape(shape))


def generate_sd(seed: int = 0x5EED0D0C) -> dict:
    """{name: f32 array}; 'e' sums are scaled by their codebook's cluster usage so that
    the dequantised codebook (sum / max(usage, 1e-5)) is ~N(0, 1)."""
    out = {}
    for i, (name, shp, kind, sc) in enumerate(sd_specs()):
        out[name] = _gen(seed, i, shp, kind, sc)
    for name in list(out):
        if name.endswith("embedding_sum"):
            u = out[name.replace("embedding_sum", "cluster_usage")]
            out[name] = np.ascontiguousarray((out[name] * u[:, None]).astype(np.float32))
    return out


def write_safetensors_f32(path: str, tensors: dict):
    header, off = {}, 0
    for n, a in tensors.items():
        header[n] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + a.size * 4]}
        off += a.size * 4
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path + ".tmp", "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for a in tensors.values():
            f.write(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    os.replace(path + ".tmp", path)


def write_sd(d: str, seed: int = 0x5EED0D0C, tensors=None) -> str:
    """Writes <d>/speech_decoder.safetensors (once); returns its path."""
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, "speech_decoder.safetensors")
    if not os.path.exists(path):
        write_safetensors_f32(path, tensors if tensors is not None else generate_sd(seed))
    return path


def rope_tables_sd(n: int):
    """The pre-transformer's NeoX tables as the reference loader builds them
    (qwen_tts_speech_decoder.c:455-463: angle = pos / powf(theta, 2i/hd)), in float64."""
    i = np.arange(HEAD_DIM // 2, dtype=np.float64)
    ang = np.arange(n, dtype=np.float64)[:, None] / np.power(ROPE_THETA, 2.0 * i / HEAD_DIM)[None, :]
    return np.cos(ang), np.sin(ang)
