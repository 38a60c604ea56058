"""ctypes bindings for the CPU checkers (TEST INFRASTRUCTURE ONLY).

* ``Oracle``  — this repo's C restatement, ``oracle/liboracle.so`` (qwen_oracle.c).
* ``RefModel`` — the reference engine built from /root/reference sources into
  ``oracle/_ref/libqwen_ref.so`` (ref_harness.c): the reference's own loader,
  quantizers, qwen_talker_step and qwen_cp_predict.

Only tests/, ``__graft_entry__.smoke`` and bench.py's cpu_baseline leg import this.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32P = C.POINTER(C.c_float)
U16P = C.POINTER(C.c_uint16)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class OMat(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scale", C.c_void_p)]


class OLayer(C.Structure):
    _fields_ = [("q", OMat), ("k", OMat), ("v", OMat), ("o", OMat), ("gate_up", OMat),
                ("down", OMat), ("input_norm", C.c_void_p), ("post_attn_norm", C.c_void_p),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class OTalker(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_heads", C.c_int),
                ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("n_layers", C.c_int),
                ("kv_max", C.c_int), ("eps", C.c_float), ("prec", C.c_int),
                ("layers", C.POINTER(OLayer)), ("final_norm", C.c_void_p),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("rope_len", C.c_int),
                ("kv_k", C.c_void_p), ("kv_v", C.c_void_p)]


class OCpFrame(C.Structure):
    _fields_ = [("cp", C.POINTER(OTalker)), ("lm_head", C.c_void_p * 15),
                ("lm_scale", C.c_void_p * 15), ("lm_prec", C.c_int),
                ("cp_emb", C.c_void_p * 15), ("talker_codec_emb", C.c_void_p),
                ("talker_hidden", C.c_int), ("emb_dim", C.c_int), ("codebook", C.c_int),
                ("codec_vocab", C.c_int), ("mtp_w", C.c_void_p), ("mtp_scale", C.c_void_p),
                ("mtp_prec", C.c_int), ("mtp_bias", C.c_void_p)]


class Oracle:
    """The C restatement.  Arrays are numpy; results returned as numpy."""

    def __init__(self, path=None):
        path = path or os.path.join(HERE, "liboracle.so")
        self.lib = L = C.CDLL(path)
        vp, i, f = C.c_void_p, C.c_int, C.c_float
        L.qo_bf16_to_f32.argtypes = [C.c_uint16]; L.qo_bf16_to_f32.restype = f
        L.qo_f32_to_bf16_trunc.argtypes = [f]; L.qo_f32_to_bf16_trunc.restype = C.c_uint16
        L.qo_f16_to_f32.argtypes = [C.c_uint16]; L.qo_f16_to_f32.restype = f
        L.qo_f32_to_f16.argtypes = [f]; L.qo_f32_to_f16.restype = C.c_uint16
        L.qo_quantize_int8.argtypes = [vp, i, i, vp, vp]
        L.qo_quantize_q4_0.argtypes = [vp, i, i, vp]
        L.qo_dequant_int8.argtypes = [vp, vp, i, i, vp]
        L.qo_dequant_q4_0.argtypes = [vp, i, i, vp]
        L.qo_matvec.argtypes = [i, vp, vp, vp, vp, i, i]
        L.qo_matvec_f64.argtypes = [i, vp, vp, vp, vp, i, i]
        L.qo_rms_norm.argtypes = [vp, vp, vp, i, f]
        L.qo_rms_norm_per_head.argtypes = [vp, vp, i, i, f]
        L.qo_rope_neox.argtypes = [vp, i, i, vp, vp, i]
        L.qo_swiglu.argtypes = [vp, i]
        L.qo_attention_bf16kv.argtypes = [vp, vp, vp, vp, i, i, i, i, i, f, i]
        L.qo_argmax.argtypes = [vp, i]; L.qo_argmax.restype = i
        L.qo_codec_greedy.argtypes = [vp, vp, i, i, i, vp]; L.qo_codec_greedy.restype = i
        L.qo_talker_step.argtypes = [C.POINTER(OTalker), vp, i, vp, vp, vp]
        L.qo_talker_step.restype = i
        L.qo_cp_pass.argtypes = [C.POINTER(OTalker), vp, i]; L.qo_cp_pass.restype = i
        L.qo_talker_prefill.argtypes = [C.POINTER(OTalker), vp, i, vp]; L.qo_talker_prefill.restype = i
        L.qo_attention_f32.argtypes = [vp, vp, vp, vp, i, i, i, i, i, f, i]
        L.qo_sample.argtypes = [vp, i, f, i, f, f, vp, i, vp]; L.qo_sample.restype = i
        L.qo_codec_rule.argtypes = [vp, i, i, f]
        L.qo_cp_frame.argtypes = [C.POINTER(OCpFrame), vp, i, vp]; L.qo_cp_frame.restype = i

    # -- scalar / array helpers
    def quantize_int8(self, w_bf16):
        rows, cols = w_bf16.shape
        q = np.empty((rows, cols), np.int8); s = np.empty(rows, np.float32)
        self.lib.qo_quantize_int8(_p(np.ascontiguousarray(w_bf16)), rows, cols, _p(q), _p(s))
        return q, s

    def quantize_q4_0(self, w_bf16):
        rows, cols = w_bf16.shape
        b = np.empty((rows, cols // 32, 18), np.uint8)
        self.lib.qo_quantize_q4_0(_p(np.ascontiguousarray(w_bf16)), rows, cols, _p(b))
        return b

    def dequant_q4_0(self, blocks, rows, cols):
        out = np.empty((rows, cols), np.float32)
        self.lib.qo_dequant_q4_0(_p(np.ascontiguousarray(blocks)), rows, cols, _p(out))
        return out

    def dequant_int8(self, q, s):
        rows, cols = q.shape
        out = np.empty((rows, cols), np.float32)
        self.lib.qo_dequant_int8(_p(q), _p(s), rows, cols, _p(out))
        return out

    def matvec(self, prec, W, scale, x, rows, cols, f64=False):
        x = np.ascontiguousarray(x, np.float32)
        if f64:
            y = np.empty(rows, np.float64)
            self.lib.qo_matvec_f64(prec, _p(y), _p(np.ascontiguousarray(W)), _p(scale), _p(x), rows, cols)
        else:
            y = np.empty(rows, np.float32)
            self.lib.qo_matvec(prec, _p(y), _p(np.ascontiguousarray(W)), _p(scale), _p(x), rows, cols)
        return y

    def rms_norm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32); out = np.empty_like(x)
        self.lib.qo_rms_norm(_p(out), _p(x), _p(np.ascontiguousarray(w, np.float32)), x.size, eps)
        return out

    def attention(self, Q, K, V, seq_q, seq_k, nh, nkv, hd, scale, q_off):
        out = np.empty(seq_q * nh * hd, np.float32)
        self.lib.qo_attention_bf16kv(_p(out), _p(np.ascontiguousarray(Q, np.float32)),
                                     _p(np.ascontiguousarray(K)), _p(np.ascontiguousarray(V)),
                                     seq_q, seq_k, nh, nkv, hd, scale, q_off)
        return out

    def talker_step(self, t, embed, pos):
        """One oracle decode step on OTalker t: (hidden f32[H], dec_x f32[H])."""
        h = np.empty(t.hidden, np.float32); dx = np.empty(t.hidden, np.float32)
        rc = self.lib.qo_talker_step(C.byref(t), _p(np.ascontiguousarray(embed, np.float32)), pos, _p(h), _p(dx), None)
        if rc != 0:
            raise RuntimeError("qo_talker_step failed")
        return h, dx

    def talker_prefill(self, t, embeds):
        """Oracle prefill of embeds f32[seq][H] on OTalker t (bf16 weights): fills the
        cache rows [0, seq) of t's KV arrays; returns dec_x f32[H]."""
        e = np.ascontiguousarray(embeds, np.float32)
        dx = np.empty(t.hidden, np.float32)
        rc = self.lib.qo_talker_prefill(C.byref(t), _p(e), e.shape[0], _p(dx))
        if rc != 0:
            raise RuntimeError("qo_talker_prefill failed")
        return dx

    def attention_f32(self, Q, K, V, seq_q, seq_k, nh, nkv, hd, scale, q_off):
        out = np.empty(seq_q * nh * hd, np.float32)
        self.lib.qo_attention_f32(_p(out), _p(np.ascontiguousarray(Q, np.float32)), _p(np.ascontiguousarray(K, np.float32)),
                                  _p(np.ascontiguousarray(V, np.float32)), seq_q, seq_k, nh, nkv, hd, scale, q_off)
        return out

    def sample(self, logits, temp, top_k, top_p, rep=1.0, prev=(), seed=12345, rule=None):
        """qwen_tts_sample restated; rule = (frame, eos_boost) applies the codec-head rule
        first.  Returns (token, new seed, final distribution or None when greedy)."""
        lg = np.array(logits, np.float32, copy=True)
        if rule is not None:
            self.lib.qo_codec_rule(_p(lg), lg.size, int(rule[0]), float(rule[1]))
        pv = np.ascontiguousarray(prev, np.int32)
        sd = np.array([seed], np.uint32)
        t = self.lib.qo_sample(_p(lg), lg.size, temp, top_k, top_p, rep, _p(pv) if pv.size else None, pv.size, _p(sd))
        return t, int(sd[0]), (None if temp < 1e-6 else lg)

    def cp_frame(self, f, talker_hidden, code0):
        """16 CP passes + 15 argmax codes on OCpFrame f."""
        out = np.empty(15, np.int32)
        rc = self.lib.qo_cp_frame(C.byref(f), _p(np.ascontiguousarray(talker_hidden, np.float32)), code0, _p(out))
        if rc != 0:
            raise RuntimeError("qo_cp_frame failed")
        return out

    def swiglu(self, gu):
        gu = np.array(gu, np.float32, copy=True)
        self.lib.qo_swiglu(_p(gu), gu.size // 2)
        return gu[: gu.size // 2].copy()


class RefModel:
    """The reference engine (its loader, quantizers, step and CP frame)."""

    CFG_ORDER = ["hidden", "layers", "heads", "kv_heads", "head_dim", "inter", "codec_vocab",
                 "codebook", "text_hidden", "cp_hidden", "cp_layers", "cp_heads", "cp_kv_heads",
                 "cp_head_dim", "cp_inter"]

    @staticmethod
    def lib_path(variant=""):
        return os.path.join(HERE, "_ref", f"libqwen_ref{variant}.so")

    @staticmethod
    def load_lib(variant=""):
        L = C.CDLL(RefModel.lib_path(variant))
        vp, i, f = C.c_void_p, C.c_int, C.c_float
        L.ref_open.argtypes = [C.c_char_p, C.POINTER(C.c_int), f, f, i, i, i]
        L.ref_open.restype = vp
        for n, rt in [("ref_kv_len", i), ("ref_kv_max", i), ("ref_rope_len", i),
                      ("ref_cp_kv_max", i), ("ref_cp_emb_dim", i)]:
            getattr(L, n).argtypes = [vp]; getattr(L, n).restype = rt
        for n in ["ref_kv_k", "ref_kv_v", "ref_rope_cos", "ref_rope_sin", "ref_talker_norm",
                  "ref_codec_head", "ref_codec_emb", "ref_cp_norm", "ref_cp_kv_k", "ref_cp_kv_v",
                  "ref_cp_rope_cos", "ref_cp_rope_sin", "ref_cp_dec_x"]:
            getattr(L, n).argtypes = [vp]; getattr(L, n).restype = vp
        L.ref_set_kv_len.argtypes = [vp, i]
        L.ref_kv_reserve.argtypes = [vp, i]; L.ref_kv_reserve.restype = i
        L.ref_ctx.argtypes = [vp]; L.ref_ctx.restype = vp
        L.ref_set_threads.argtypes = [i]
        L.ref_talker_step.argtypes = [vp, vp, vp]; L.ref_talker_step.restype = i
        L.ref_talker_prefill.argtypes = [vp, vp, i]; L.ref_talker_prefill.restype = i
        L.ref_talker_step_layers.argtypes = [vp, vp, vp, vp]; L.ref_talker_step_layers.restype = i
        L.ref_get_dec_x.argtypes = [vp, vp]
        L.ref_layer_ptr.argtypes = [vp, i, i, i, i]; L.ref_layer_ptr.restype = vp
        L.ref_cp_predict.argtypes = [vp, vp, i, vp]; L.ref_cp_predict.restype = i
        L.ref_cp_lm_head.argtypes = [vp, i, i]; L.ref_cp_lm_head.restype = vp
        L.ref_cp_codec_emb.argtypes = [vp, i]; L.ref_cp_codec_emb.restype = vp
        L.ref_cp_mtp.argtypes = [vp, i]; L.ref_cp_mtp.restype = vp
        L.ref_codec_greedy.argtypes = [vp, vp, i, vp]; L.ref_codec_greedy.restype = i
        L.ref_quantize_int8.argtypes = [vp, i, i, vp, vp]
        L.ref_quantize_q4_0.argtypes = [vp, i, i, vp]
        L.ref_matvec_bf16.argtypes = [vp, vp, vp, i, i]
        L.ref_matmat_bf16.argtypes = [vp, vp, vp, i, i, i]
        L.ref_matvec_int8.argtypes = [vp, vp, vp, vp, i, i]
        L.ref_matvec_q4_0.argtypes = [vp, vp, vp, i, i]
        L.ref_attention_bf16kv.argtypes = [vp, vp, vp, vp, i, i, i, i, i, f, i]
        L.ref_rms_norm.argtypes = [vp, vp, vp, i, i, f]
        L.ref_swiglu.argtypes = [vp, i]
        L.ref_rms_norm_per_head.argtypes = [vp, vp, i, i, i, f]
        L.ref_argmax_matvec_bf16.argtypes = [vp, vp, i, i]; L.ref_argmax_matvec_bf16.restype = i
        L.ref_sample.argtypes = [vp, i, f, i, f, f, vp, i, vp]; L.ref_sample.restype = i
        L.ref_argmax_matvec_int8.argtypes = [vp, vp, vp, i, i]; L.ref_argmax_matvec_int8.restype = i
        L.ref_argmax_matvec_q4_0.argtypes = [vp, vp, i, i]; L.ref_argmax_matvec_q4_0.restype = i
        L.ref_f32_to_f16.argtypes = [f]; L.ref_f32_to_f16.restype = C.c_uint16
        L.ref_f16_to_f32.argtypes = [C.c_uint16]; L.ref_f16_to_f32.restype = f
        L.ref_time_talker_steps.argtypes = [vp, vp, i, vp]; L.ref_time_talker_steps.restype = C.c_double
        L.ref_time_talker_steps_each.argtypes = [vp, vp, i, vp, vp]
        L.ref_build_info.restype = C.c_char_p
        return L

    def __init__(self, model_dir, shape, prec="bf16", threads=1, variant=""):
        self.lib = self.load_lib(variant)
        self.shape = s = shape
        cfg = (C.c_int * 15)(*[getattr(s, k) for k in self.CFG_ORDER])
        self.prec = prec
        self.h = self.lib.ref_open(model_dir.encode(), cfg, s.eps, s.rope_theta,
                                   1 if prec == "int8" else 0, 1 if prec == "int4" else 0, threads)
        if not self.h:
            raise RuntimeError("reference load failed")

    # -- raw views of reference-owned memory
    def _view(self, ptr, dtype, count):
        if not ptr:
            return None
        buf = (C.c_byte * (count * np.dtype(dtype).itemsize)).from_address(ptr)
        return np.frombuffer(buf, dtype=dtype, count=count)

    def step(self, embed):
        out = np.empty(self.shape.hidden, np.float32)
        rc = self.lib.ref_talker_step(self.h, _p(np.ascontiguousarray(embed, np.float32)), _p(out))
        assert rc == 0
        return out

    def prefill(self, embeds):
        """The reference prefill of embeds f32[seq][H]; kv_len becomes seq."""
        e = np.ascontiguousarray(embeds, np.float32)
        rc = self.lib.ref_talker_prefill(self.h, _p(e), e.shape[0])
        assert rc == 0
        return self.dec_x()

    def step_layers(self, embed):
        s = self.shape
        res = np.empty((s.layers, s.hidden), np.float32)
        out = np.empty(s.hidden, np.float32)
        rc = self.lib.ref_talker_step_layers(self.h, _p(np.ascontiguousarray(embed, np.float32)), _p(res), _p(out))
        assert rc == 0
        return res, out

    def dec_x(self):
        out = np.empty(self.shape.hidden, np.float32)
        self.lib.ref_get_dec_x(self.h, _p(out))
        return out

    @property
    def kv_len(self):
        return self.lib.ref_kv_len(self.h)

    @kv_len.setter
    def kv_len(self, n):
        self.lib.ref_set_kv_len(self.h, n)

    def kv_reserve(self, n):
        """Grow the reference KV cache to at least n positions (views from kv() go stale)."""
        assert self.lib.ref_kv_reserve(self.h, n) == 0

    def set_kv(self, k, v, n):
        """Positions [0, n) of the reference cache <- k, v [layers][>= n][kv_dim]; kv_len = n."""
        self.kv_reserve(n + 1)
        rk, rv = self.kv()
        rk[:, :n] = k[:, :n]
        rv[:, :n] = v[:, :n]
        self.kv_len = n

    def kv(self):
        s = self.shape
        kvm = self.lib.ref_kv_max(self.h)
        n = s.layers * kvm * s.kv_dim
        k = self._view(self.lib.ref_kv_k(self.h), np.uint16, n).reshape(s.layers, kvm, s.kv_dim)
        v = self._view(self.lib.ref_kv_v(self.h), np.uint16, n).reshape(s.layers, kvm, s.kv_dim)
        return k, v

    def rope(self):
        n = self.lib.ref_rope_len(self.h)
        half = self.shape.head_dim // 2
        return (self._view(self.lib.ref_rope_cos(self.h), np.float32, n * half).reshape(n, half),
                self._view(self.lib.ref_rope_sin(self.h), np.float32, n * half).reshape(n, half))

    def cp_rope(self):
        n = self.lib.ref_cp_kv_max(self.h)
        half = self.shape.cp_head_dim // 2
        return (self._view(self.lib.ref_cp_rope_cos(self.h), np.float32, n * half).reshape(n, half),
                self._view(self.lib.ref_cp_rope_sin(self.h), np.float32, n * half).reshape(n, half))

    def layer_mat(self, layer, which, cp=False):
        """which: 'q','k','v','o','gate_up','down' -> dict of views by precision."""
        s = self.shape
        idx = ["q", "k", "v", "o", "gate_up", "down"].index(which)
        H = s.cp_hidden if cp else s.hidden
        F = s.cp_inter if cp else s.inter
        nh, nkv, hd = (s.cp_heads, s.cp_kv_heads, s.cp_head_dim) if cp else (s.heads, s.kv_heads, s.head_dim)
        rows, cols = {"q": (nh * hd, H), "k": (nkv * hd, H), "v": (nkv * hd, H),
                      "o": (H, nh * hd), "gate_up": (2 * F, H), "down": (H, F)}[which]
        out = {"rows": rows, "cols": cols}
        cpf = 1 if cp else 0
        out["bf16"] = self._view(self.lib.ref_layer_ptr(self.h, cpf, layer, idx, 0), np.uint16, rows * cols)
        out["int8"] = self._view(self.lib.ref_layer_ptr(self.h, cpf, layer, idx, 1), np.int8, rows * cols)
        out["scale"] = self._view(self.lib.ref_layer_ptr(self.h, cpf, layer, idx, 2), np.float32, rows)
        out["q4"] = self._view(self.lib.ref_layer_ptr(self.h, cpf, layer, idx, 3), np.uint8, rows * cols // 32 * 18)
        for k in ("bf16", "int8"):
            if out[k] is not None:
                out[k] = out[k].reshape(rows, cols)
        return out

    def layer_norm(self, layer, which, cp=False):
        s = self.shape
        H = s.cp_hidden if cp else s.hidden
        hd = s.cp_head_dim if cp else s.head_dim
        idx = {"input": 10, "post": 11, "q": 12, "k": 13}[which]
        n = H if which in ("input", "post") else hd
        return self._view(self.lib.ref_layer_ptr(self.h, 1 if cp else 0, layer, idx, 0), np.float32, n)

    def final_norm(self):
        return self._view(self.lib.ref_talker_norm(self.h), np.float32, self.shape.hidden)

    def cp_norm(self):
        return self._view(self.lib.ref_cp_norm(self.h), np.float32, self.shape.cp_hidden)

    def codec_head(self):
        s = self.shape
        return self._view(self.lib.ref_codec_head(self.h), np.uint16, s.codec_vocab * s.hidden).reshape(s.codec_vocab, s.hidden)

    def codec_emb(self):
        s = self.shape
        return self._view(self.lib.ref_codec_emb(self.h), np.uint16, s.codec_vocab * s.hidden).reshape(s.codec_vocab, s.hidden)

    def cp_lm_head(self, g):
        s = self.shape
        n = s.codebook * s.cp_hidden
        return {"bf16": self._view(self.lib.ref_cp_lm_head(self.h, g, 0), np.uint16, n),
                "int8": self._view(self.lib.ref_cp_lm_head(self.h, g, 1), np.int8, n),
                "scale": self._view(self.lib.ref_cp_lm_head(self.h, g, 2), np.float32, s.codebook),
                "q4": self._view(self.lib.ref_cp_lm_head(self.h, g, 3), np.uint8, n // 32 * 18)}

    def cp_codec_emb(self, g):
        s = self.shape
        E = self.lib.ref_cp_emb_dim(self.h)
        return self._view(self.lib.ref_cp_codec_emb(self.h, g), np.uint16, s.codebook * E).reshape(s.codebook, E)

    def cp_mtp(self):
        s = self.shape
        n = s.cp_hidden * s.hidden
        return {"bf16": self._view(self.lib.ref_cp_mtp(self.h, 0), np.uint16, n),
                "int8": self._view(self.lib.ref_cp_mtp(self.h, 1), np.int8, n),
                "scale": self._view(self.lib.ref_cp_mtp(self.h, 2), np.float32, s.cp_hidden),
                "bias": self._view(self.lib.ref_cp_mtp(self.h, 3), np.float32, s.cp_hidden)}

    def cp_kv(self):
        s = self.shape
        kvm = self.lib.ref_cp_kv_max(self.h)
        kvd = s.cp_kv_heads * s.cp_head_dim
        n = s.cp_layers * kvm * kvd
        return (self._view(self.lib.ref_cp_kv_k(self.h), np.uint16, n).reshape(s.cp_layers, kvm, kvd),
                self._view(self.lib.ref_cp_kv_v(self.h), np.uint16, n).reshape(s.cp_layers, kvm, kvd))

    def cp_dec_x(self):
        """The CP residual after the last pass of the last qwen_cp_predict (ctx->cp_dec_x)."""
        return self._view(self.lib.ref_cp_dec_x(self.h), np.float32, self.shape.cp_hidden).copy()

    def cp_predict(self, talker_hidden, code0):
        out = (C.c_int * 15)()
        rc = self.lib.ref_cp_predict(self.h, _p(np.ascontiguousarray(talker_hidden, np.float32)), code0, out)
        assert rc == 0
        return np.array(list(out), np.int32)

    def codec_greedy(self, hidden, frame):
        lg = np.empty(self.shape.codec_vocab, np.float32)
        t = self.lib.ref_codec_greedy(self.h, _p(np.ascontiguousarray(hidden, np.float32)), frame, _p(lg))
        return t, lg


def oracle_talker(ref: RefModel, prec_code: int, kv_max: int, cp=False):
    """Build an OTalker over the reference-loaded weights (so both checkers see the
    same bytes).  Returns (struct, keepalive)."""
    s = ref.shape
    nl = s.cp_layers if cp else s.layers
    layers = (OLayer * nl)()
    keep = []
    kind = {0: "bf16", 1: "int8", 2: "q4"}[prec_code]
    for l in range(nl):
        ly = layers[l]
        for nm in ["q", "k", "v", "o", "gate_up", "down"]:
            m = ref.layer_mat(l, nm, cp=cp)
            arr = m[kind]
            keep.append(arr)
            getattr(ly, nm).w = arr.ctypes.data
            getattr(ly, nm).scale = m["scale"].ctypes.data if prec_code == 1 else None
        for nm, key in [("input_norm", "input"), ("post_attn_norm", "post"), ("q_norm", "q"), ("k_norm", "k")]:
            a = ref.layer_norm(l, key, cp=cp)
            keep.append(a)
            setattr(ly, nm, a.ctypes.data)
    if cp:
        cos, sin = ref.cp_rope()
        H, F, nh, nkv, hd = s.cp_hidden, s.cp_inter, s.cp_heads, s.cp_kv_heads, s.cp_head_dim
        fn = ref.cp_norm()
    else:
        cos, sin = ref.rope()
        H, F, nh, nkv, hd = s.hidden, s.inter, s.heads, s.kv_heads, s.head_dim
        fn = ref.final_norm()
    kvk = np.zeros((nl, kv_max, nkv * hd), np.uint16)
    kvv = np.zeros((nl, kv_max, nkv * hd), np.uint16)
    keep += [cos, sin, fn, kvk, kvv, layers]
    t = OTalker(hidden=H, inter=F, n_heads=nh, n_kv_heads=nkv, head_dim=hd, n_layers=nl,
                kv_max=kv_max, eps=s.eps, prec=prec_code, layers=layers, final_norm=fn.ctypes.data,
                rope_cos=cos.ctypes.data, rope_sin=sin.ctypes.data, rope_len=cos.shape[0],
                kv_k=kvk.ctypes.data, kv_v=kvv.ctypes.data)
    return t, {"keep": keep, "kv_k": kvk, "kv_v": kvv}


_PREC_CODE = {"bf16": 0, "int8": 1, "int4": 2}


def _quantized(orc: Oracle, w_bf16, prec):
    """(weight bytes, scale) of one matrix in the reference's host encoding, made by the
    oracle's own quantizers (qwen_tts_kernels.c:2143-2238, :2662-2726)."""
    if prec == "bf16":
        return np.ascontiguousarray(w_bf16), None
    if prec == "int8":
        return orc.quantize_int8(w_bf16)
    return orc.quantize_q4_0(w_bf16), None


def talker_from_tensors(orc: Oracle, tens, shape, prec, kv_max, rope_cos, rope_sin, cp=False):
    """An OTalker over synthetic tensors {reference name: bf16 array}, quantized by the
    oracle itself, with the given RoPE tables.  Mirrors the reference loader: gate|up
    rows interleaved (qwen_tts_talker.c:378-388), norm gains bf16 -> f32.
    Returns (struct, keepalive dict with the KV arrays)."""
    s = shape
    nl = s.cp_layers if cp else s.layers
    pre = "talker.code_predictor.model.layers." if cp else "talker.model.layers."
    layers = (OLayer * nl)()
    keep = []
    b2f = lambda a: (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    for l in range(nl):
        p = f"{pre}{l}."
        gu = np.empty((2 * tens[p + "mlp.gate_proj.weight"].shape[0], tens[p + "mlp.gate_proj.weight"].shape[1]),
                      np.uint16)
        gu[0::2] = tens[p + "mlp.gate_proj.weight"]
        gu[1::2] = tens[p + "mlp.up_proj.weight"]
        mats = {"q": tens[p + "self_attn.q_proj.weight"], "k": tens[p + "self_attn.k_proj.weight"],
                "v": tens[p + "self_attn.v_proj.weight"], "o": tens[p + "self_attn.o_proj.weight"],
                "gate_up": gu, "down": tens[p + "mlp.down_proj.weight"]}
        ly = layers[l]
        for nm, w in mats.items():
            wq, sc = _quantized(orc, w, prec)
            keep += [wq, sc]
            getattr(ly, nm).w = wq.ctypes.data
            getattr(ly, nm).scale = sc.ctypes.data if sc is not None else None
        for fld, key in [("input_norm", "input_layernorm.weight"), ("post_attn_norm", "post_attention_layernorm.weight"),
                         ("q_norm", "self_attn.q_norm.weight"), ("k_norm", "self_attn.k_norm.weight")]:
            a = np.ascontiguousarray(b2f(tens[p + key]))
            keep.append(a)
            setattr(ly, fld, a.ctypes.data)
    if cp:
        H, F, nh, nkv, hd = s.cp_hidden, s.cp_inter, s.cp_heads, s.cp_kv_heads, s.cp_head_dim
        fn = np.ascontiguousarray(b2f(tens["talker.code_predictor.model.norm.weight"]))
    else:
        H, F, nh, nkv, hd = s.hidden, s.inter, s.heads, s.kv_heads, s.head_dim
        fn = np.ascontiguousarray(b2f(tens["talker.model.norm.weight"]))
    cos = np.ascontiguousarray(rope_cos, np.float32)
    sin = np.ascontiguousarray(rope_sin, np.float32)
    kvk = np.zeros((nl, kv_max, nkv * hd), np.uint16)
    kvv = np.zeros((nl, kv_max, nkv * hd), np.uint16)
    keep += [cos, sin, fn, kvk, kvv, layers]
    t = OTalker(hidden=H, inter=F, n_heads=nh, n_kv_heads=nkv, head_dim=hd, n_layers=nl,
                kv_max=kv_max, eps=s.eps, prec=_PREC_CODE[prec], layers=layers, final_norm=fn.ctypes.data,
                rope_cos=cos.ctypes.data, rope_sin=sin.ctypes.data, rope_len=cos.shape[0],
                kv_k=kvk.ctypes.data, kv_v=kvv.ctypes.data)
    return t, {"keep": keep, "kv_k": kvk, "kv_v": kvv}


def cp_frame_from_tensors(orc: Oracle, tens, shape, prec, cp_cos, cp_sin):
    """An OCpFrame over synthetic tensors (CP layers, 15 lm heads in the CP precision,
    bf16 codec embeddings; no small_to_mtp_projection when the Talker and CP hidden
    sizes agree, qwen_tts_code_predictor.c:907-924).  Returns (struct, keepalive)."""
    s = shape
    cpt, keep = talker_from_tensors(orc, tens, s, prec, 64, cp_cos, cp_sin, cp=True)
    keep = {"cp": cpt, "inner": keep, "arrs": []}
    f = OCpFrame()
    f.cp = C.pointer(cpt)
    f.lm_prec = _PREC_CODE[prec]
    for g in range(15):
        wq, sc = _quantized(orc, tens[f"talker.code_predictor.lm_head.{g}.weight"], prec)
        e = np.ascontiguousarray(tens[f"talker.code_predictor.model.codec_embedding.{g}.weight"])
        keep["arrs"] += [wq, sc, e]
        f.lm_head[g] = wq.ctypes.data
        f.lm_scale[g] = sc.ctypes.data if sc is not None else None
        f.cp_emb[g] = e.ctypes.data
    te = np.ascontiguousarray(tens["talker.model.codec_embedding.weight"])
    keep["arrs"].append(te)
    f.talker_codec_emb = te.ctypes.data
    f.talker_hidden = s.hidden
    f.emb_dim = s.hidden
    f.codebook = s.codebook
    f.codec_vocab = s.codec_vocab
    if "talker.code_predictor.small_to_mtp_projection.weight" in tens:
        raise NotImplementedError("mtp projection: build the frame from RefModel instead")
    f.mtp_w = None
    return f, keep


class RefSpeechDecoder:
    """The reference's own speech decoder (qwen_speech_decoder_load + the one-shot
    qwen_speech_decoder_decode, qwen_tts_speech_decoder.c:372-1290) from oracle/_ref, over
    an F32 safetensors file of the decoder's tensors."""

    def __init__(self, path, threads=8, variant=""):
        L = C.CDLL(RefModel.lib_path(variant))
        vp, i = C.c_void_p, C.c_int
        L.ref_sd_open.argtypes = [C.c_char_p, i]; L.ref_sd_open.restype = vp
        L.ref_sd_decode.argtypes = [vp, vp, i, vp, i]; L.ref_sd_decode.restype = i
        L.ref_time_sd_decode.argtypes = [vp, vp, i]; L.ref_time_sd_decode.restype = C.c_double
        L.ref_sd_stream_new.argtypes = []; L.ref_sd_stream_new.restype = vp
        L.ref_sd_stream_decode.argtypes = [vp, vp, vp, i, vp, i]; L.ref_sd_stream_decode.restype = i
        L.ref_sd_stream_free.argtypes = [vp]
        self.L = L
        self.h = L.ref_sd_open(str(path).encode(), threads)
        if not self.h:
            raise RuntimeError("reference speech decoder load failed")

    def decode(self, codes):
        codes = np.ascontiguousarray(codes, np.int32)
        n = codes.shape[0]
        out = np.empty(n * 1920, np.float32)
        ns = self.L.ref_sd_decode(self.h, codes.ctypes.data, n, out.ctypes.data, out.size)
        if ns < 0:
            raise RuntimeError("reference decode failed")
        return out[:ns]

    def stream_decode(self, chunks):
        """The reference's exact streaming decode over successive chunks of codes (one
        fresh stream state); returns the concatenated audio."""
        st = self.L.ref_sd_stream_new()
        out = []
        try:
            for codes in chunks:
                codes = np.ascontiguousarray(codes, np.int32)
                buf = np.empty(codes.shape[0] * 1920, np.float32)
                ns = self.L.ref_sd_stream_decode(self.h, st, codes.ctypes.data, codes.shape[0], buf.ctypes.data, buf.size)
                if ns < 0:
                    raise RuntimeError("reference streaming decode failed")
                out.append(buf[:ns])
        finally:
            self.L.ref_sd_stream_free(st)
        return np.concatenate(out)

    def time_decode(self, codes):
        codes = np.ascontiguousarray(codes, np.int32)
        return self.L.ref_time_sd_decode(self.h, codes.ctypes.data, codes.shape[0])
