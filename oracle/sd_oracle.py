"""Float64 numpy restatement of the reference's one-shot speech decoder (TEST
INFRASTRUCTURE ONLY: imported by tests/ to check the device decoder stage by stage).

Follows ``qwen_speech_decoder_decode`` (qwen_tts_speech_decoder.c:579-1290) step by step,
in float64 on the reference's own formulas; the compiled reference (oracle/_ref,
ref_sd_decode) pins it end to end (tests/test_cpu_sd.py).  Layout as the reference:
transformer activations [T][C], conv activations channel-first [C][T].
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

CB_SIZE, N_HEADS, HEAD_DIM, WINDOW, N_LAYERS = 2048, 16, 64, 72, 8
UP_RATES, DILATIONS = (8, 5, 4, 3), (1, 3, 9)
ROPE_THETA, EPS = 10000.0, 1e-5


def _f(t, name):
    return np.asarray(t[name], np.float64)


def codebooks(t):
    """sd.c:383-405: codebook = embedding_sum / max(cluster_usage, 1e-5)."""
    out = []
    for k in range(16):
        p = ("decoder.quantizer.rvq_first.vq.layers.0._codebook" if k == 0
             else f"decoder.quantizer.rvq_rest.vq.layers.{k - 1}._codebook")
        es, cu = _f(t, p + ".embedding_sum"), _f(t, p + ".cluster_usage")
        out.append(es / np.maximum(cu, 1e-5)[:, None])
    return out


def vq(t, codes):
    """sd.c:599-660: codebook 0 through rvq_first's projection, the sum of codebooks
    1..15 through rvq_rest's; codes outside [0, 2048) contribute nothing."""
    cbs = codebooks(t)
    n = codes.shape[0]
    first = np.zeros((n, 256)); rest = np.zeros((n, 256))
    for f in range(n):
        c0 = int(codes[f, 0])
        if 0 <= c0 < CB_SIZE:
            first[f] = cbs[0][c0]
        for k in range(1, 16):
            c = int(codes[f, k])
            if 0 <= c < CB_SIZE:
                rest[f] += cbs[k][c]
    return (first @ _f(t, "decoder.quantizer.rvq_first.output_proj.weight").T +
            rest @ _f(t, "decoder.quantizer.rvq_rest.output_proj.weight").T)


def conv1d(x, w, b, dilation=1):
    """Causal conv (sd.c:98-119): x [Cin][T], w [Cout][Cin][k], pad_left (k-1)*dilation."""
    cout, cin, k = w.shape
    T = x.shape[1]
    pad = (k - 1) * dilation
    xp = np.concatenate([np.zeros((cin, pad)), x], axis=1)
    out = np.zeros((cout, T)) if b is None else np.repeat(b[:, None], T, axis=1).astype(np.float64)
    for j in range(k):
        out = out + w[:, :, j] @ xp[:, j * dilation:j * dilation + T]
    return out


def conv_transpose1d(x, w, b, stride):
    """Causal transposed conv (sd.c:122-160): x [Cin][T], w [Cin][Cout][k]; output
    position t*stride + j gets x[:, t] . w[:, :, j]; the right tail past T*stride is
    dropped (out_len = T*stride, sd.c:88-91)."""
    cin, cout, k = w.shape
    T = x.shape[1]
    L = T * stride
    out = np.zeros((cout, L + k))
    for j in range(k):
        out[:, j:j + T * stride:stride] += w[:, :, j].T @ x
    out = out[:, :L]
    if b is not None:
        out += b[:, None]
    return out


def rms_norm(x, w):
    """qwen_rms_norm (k.c:292-382), rows of x."""
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + EPS)
    return x * inv * w


def rope_tables(n):
    """sd.c:455-463: angle = pos / theta^(2i/hd)."""
    i = np.arange(HEAD_DIM // 2, dtype=np.float64)
    ang = np.arange(n, dtype=np.float64)[:, None] / np.power(ROPE_THETA, 2.0 * i / HEAD_DIM)[None, :]
    return np.cos(ang), np.sin(ang)


def rope(x, cos, sin):
    """NeoX split-half rotation per head (sd.c:790-860), x [T][16*64]."""
    T = x.shape[0]
    h = x.reshape(T, N_HEADS, HEAD_DIM)
    a, b = h[..., :HEAD_DIM // 2], h[..., HEAD_DIM // 2:]
    c, s = cos[:T, None, :], sin[:T, None, :]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1).reshape(T, -1)


def attention_windowed(q, k, v, window=WINDOW):
    """qwen_causal_attention_windowed (k.c:3579-3700) with seq_q == seq_k, q_offset 0:
    query i attends keys [max(0, i+1-window), i]."""
    T = q.shape[0]
    qh = q.reshape(T, N_HEADS, HEAD_DIM); kh = k.reshape(T, N_HEADS, HEAD_DIM); vh = v.reshape(T, N_HEADS, HEAD_DIM)
    out = np.zeros_like(qh)
    scale = 1.0 / np.sqrt(HEAD_DIM)
    for i in range(T):
        j0 = max(0, i + 1 - window)
        s = np.einsum("hd,jhd->hj", qh[i], kh[j0:i + 1]) * scale
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[i] = np.einsum("hj,jhd->hd", p, vh[j0:i + 1])
    return out.reshape(T, -1)


def snake(x, la, lb):
    """qwen_snake_activation (k.c:4472-4600): x + exp(-beta) sin^2(exp(alpha) x), per channel."""
    return x + np.exp(-lb)[:, None] * np.sin(np.exp(la)[:, None] * x) ** 2


def gelu(x):
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def pre_transformer(t, h):
    """sd.c:757-1002 (8 layers) + final norm and output projection (sd.c:1012-1044); h [T][512]."""
    pt = "decoder.pre_transformer"
    cos, sin = rope_tables(h.shape[0])
    for i in range(N_LAYERS):
        p = f"{pt}.layers.{i}"
        xn = rms_norm(h, _f(t, f"{p}.input_layernorm.weight"))
        q = rope(xn @ _f(t, f"{p}.self_attn.q_proj.weight").T, cos, sin)
        k = rope(xn @ _f(t, f"{p}.self_attn.k_proj.weight").T, cos, sin)
        v = xn @ _f(t, f"{p}.self_attn.v_proj.weight").T
        a = attention_windowed(q, k, v)
        h = h + (a @ _f(t, f"{p}.self_attn.o_proj.weight").T) * _f(t, f"{p}.self_attn_layer_scale.scale")
        xn = rms_norm(h, _f(t, f"{p}.post_attention_layernorm.weight"))
        g = xn @ _f(t, f"{p}.mlp.gate_proj.weight").T
        u = xn @ _f(t, f"{p}.mlp.up_proj.weight").T
        m = g / (1.0 + np.exp(-g)) * u
        h = h + (m @ _f(t, f"{p}.mlp.down_proj.weight").T) * _f(t, f"{p}.mlp_layer_scale.scale")
    h = rms_norm(h, _f(t, f"{pt}.norm.weight"))
    return h @ _f(t, f"{pt}.output_proj.weight").T + _f(t, f"{pt}.output_proj.bias")


def convnext(t, b, sig):
    """sd.c:1062-1158: transposed conv x2, depthwise conv k=7, LayerNorm over channels
    (mean and E[x^2] - mean^2 per time step, eps 1e-5), pw1 + GELU, pw2, gamma, residual."""
    p = f"decoder.upsample.{b}"
    sig = conv_transpose1d(sig, _f(t, f"{p}.0.conv.weight"), _f(t, f"{p}.0.conv.bias"), 2)
    res = sig
    dw = _f(t, f"{p}.1.dwconv.conv.weight")[:, 0, :]
    T = sig.shape[1]
    xp = np.concatenate([np.zeros((sig.shape[0], 6)), sig], axis=1)
    d = np.repeat(_f(t, f"{p}.1.dwconv.conv.bias")[:, None], T, axis=1)
    for j in range(7):
        d = d + dw[:, j:j + 1] * xp[:, j:j + T]
    mean = d.mean(axis=0, keepdims=True)
    var = (d * d).mean(axis=0, keepdims=True) - mean * mean
    x = (d - mean) / np.sqrt(var + 1e-5) * _f(t, f"{p}.1.norm.weight")[:, None] + _f(t, f"{p}.1.norm.bias")[:, None]
    y = gelu(_f(t, f"{p}.1.pwconv1.weight") @ x + _f(t, f"{p}.1.pwconv1.bias")[:, None])
    y = _f(t, f"{p}.1.pwconv2.weight") @ y + _f(t, f"{p}.1.pwconv2.bias")[:, None]
    return res + y * _f(t, f"{p}.1.gamma")[:, None]


def conv_decoder(t, sig):
    """sd.c:1160-1282: initial conv k=7, four upsample blocks (snake, transposed conv,
    three residual units snake / conv k=7 dilated / snake / conv k=1), final snake,
    conv to one channel, clamp to [-1, 1]."""
    sig = conv1d(sig, _f(t, "decoder.decoder.0.conv.weight"), _f(t, "decoder.decoder.0.conv.bias"))
    for b in range(4):
        p = f"decoder.decoder.{b + 1}.block"
        sig = snake(sig, _f(t, f"{p}.0.alpha"), _f(t, f"{p}.0.beta"))
        sig = conv_transpose1d(sig, _f(t, f"{p}.1.conv.weight"), _f(t, f"{p}.1.conv.bias"), UP_RATES[b])
        for r in range(3):
            q = f"{p}.{r + 2}"
            x = snake(sig, _f(t, f"{q}.act1.alpha"), _f(t, f"{q}.act1.beta"))
            x = conv1d(x, _f(t, f"{q}.conv1.conv.weight"), _f(t, f"{q}.conv1.conv.bias"), DILATIONS[r])
            x = snake(x, _f(t, f"{q}.act2.alpha"), _f(t, f"{q}.act2.beta"))
            sig = sig + conv1d(x, _f(t, f"{q}.conv2.conv.weight"), _f(t, f"{q}.conv2.conv.bias"))
    sig = snake(sig, _f(t, "decoder.decoder.5.alpha"), _f(t, "decoder.decoder.5.beta"))
    audio = conv1d(sig, _f(t, "decoder.decoder.6.conv.weight"), _f(t, "decoder.decoder.6.conv.bias"))[0]
    return np.clip(audio, -1.0, 1.0)


def decode(t, codes, stages=None):
    """codes int [n][16] -> audio float64 [1920 n].  ``stages`` (a dict) receives the
    intermediate tensors: vq [n][512], pre_conv [n][1024] (time-major), hidden [n][512]
    (input projection), latent [n][1024] (after the pre-transformer), convnext [T][1024]
    (after both upsamplers, time-major), audio_raw (before the clamp)."""
    codes = np.asarray(codes)
    v = vq(t, codes)
    x = conv1d(v.T, _f(t, "decoder.pre_conv.conv.weight"), _f(t, "decoder.pre_conv.conv.bias"))
    h = x.T @ _f(t, "decoder.pre_transformer.input_proj.weight").T + _f(t, "decoder.pre_transformer.input_proj.bias")
    lat = pre_transformer(t, h)
    sig = lat.T
    for b in range(2):
        sig = convnext(t, b, sig)
    audio = conv_decoder(t, sig)
    if stages is not None:
        stages.update(vq=v, pre_conv=x.T, hidden=h, latent=lat, convnext=sig.T)
    return audio
