"""ctypes binding of libqwen_tts_hip.so (the C ABI declared in include/qwen_tts_hip.h).

The library is loaded from this package directory; there is no fallback: if the
shared object is missing or no GPU is present the calls fail loudly.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqwen_tts_hip.so")

BF16, INT8, Q4_0 = 0, 1, 2
PREC = {"bf16": BF16, "int8": INT8, "int4": Q4_0, "q4_0": Q4_0}

# every symbol the header declares (checked by the CPU test suite)
EXPORTS = [
    "qwen_hip_talker_init", "qwen_hip_talker_step", "qwen_hip_talker_get_dec_x",
    "qwen_hip_talker_upload_kv", "qwen_hip_talker_free", "qwen_hip_talker_download_kv",
    "qwen_hip_talker_greedy", "qwen_hip_talker_greedy_async", "qwen_hip_talker_sync",
    "qwen_hip_talker_stream", "qwen_hip_talker_fused", "qwen_hip_talker_fused_kernel", "qwen_hip_talker_grow_kv", "qwen_hip_talker_kv_max", "qwen_hip_talker_step_nograph", "qwen_hip_talker_launch_kernel", "qwen_hip_cp_init", "qwen_hip_cp_step", "qwen_hip_cp_download_kv",
    "qwen_hip_cp_frame", "qwen_hip_cp_frame_async", "qwen_hip_cp_sync", "qwen_hip_cp_stream", "qwen_hip_cp_fused",
    "qwen_hip_cp_free", "qwen_hip_available", "qwen_hip_init", "qwen_hip_free", "qwen_hip_matvec_bf16",
    "qwen_hip_matmat_bf16", "qwen_hip_op_matvec_int8", "qwen_hip_op_matvec_q4_0",
    "qwen_hip_op_matvec_bf16", "qwen_hip_op_causal_attention_bf16kv", "qwen_hip_op_rms_norm",
    "qwen_hip_op_rms_norm_per_head", "qwen_hip_op_swiglu", "qwen_hip_op_argmax_matvec",
    "qwen_hip_op_sample", "qwen_hip_op_codec_sample", "qwen_hip_talker_sample",
    "qwen_hip_op_quantize_int8", "qwen_hip_op_quantize_q4_0", "qwen_hip_talker_dequant",
    "qwen_hip_last_error", "qwen_hip_talker_batch_init", "qwen_hip_talker_batch_step", "qwen_hip_talker_batch_step_layers",
    "qwen_hip_talker_batch_upload_slot", "qwen_hip_talker_batch_free", "qwen_hip_talker_batch_download_slot",
    "qwen_hip_talker_batch_step_async", "qwen_hip_talker_batch_sync", "qwen_hip_talker_batch_stream",
    "qwen_hip_batch_fold_pieces",
    "qwen_hip_cp_batch_init", "qwen_hip_cp_batch_step", "qwen_hip_cp_batch_free", "qwen_hip_op_matmat_int8", "qwen_hip_op_matmat_q4_0",
    "qwen_hip_cp_set_prefill2", "qwen_hip_cp_prefill2",
    "qwen_hip_talker_prefill", "qwen_hip_talker_prefill_async", "qwen_hip_op_prefill_gemm",
    "qwen_hip_op_prefill_attention", "qwen_hip_talker_step_layers", "qwen_hip_op_matmat_int8_noalloc",
    "qwen_hip_generate", "qwen_hip_talker_load_file",
    "qwen_hip_sd_init", "qwen_hip_sd_load_file", "qwen_hip_sd_decode", "qwen_hip_sd_decode_device",
    "qwen_hip_sd_latent", "qwen_hip_sd_stream", "qwen_hip_sd_free", "qwen_hip_op_sd_conv",
    "qwen_hip_op_sd_conv_transpose", "qwen_hip_sd_stream_new", "qwen_hip_sd_stream_decode",
    "qwen_hip_sd_stream_reset", "qwen_hip_sd_stream_free",
]

SD_GET_FN = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_char_p, C.c_longlong)
SD_SAMPLES_PER_FRAME = 1920


class Mat(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scale", C.c_void_p)]


class Layer(C.Structure):
    _fields_ = [("q", Mat), ("k", Mat), ("v", Mat), ("o", Mat), ("gate_up", Mat), ("down", Mat),
                ("input_norm", C.c_void_p), ("post_attn_norm", C.c_void_p),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class TalkerDesc(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("n_layers", C.c_int), ("kv_max", C.c_int), ("eps", C.c_float),
                ("prec", C.c_int), ("quantize_to", C.c_int), ("layers", C.POINTER(Layer)),
                ("final_norm", C.c_void_p), ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
                ("rope_len", C.c_int)]


class CpDesc(C.Structure):
    _fields_ = [("cp", TalkerDesc), ("codebook", C.c_int), ("lm_prec", C.c_int), ("lm_head", Mat * 15),
                ("cp_codec_emb", C.c_void_p * 15), ("talker_codec_emb", C.c_void_p),
                ("codec_vocab", C.c_int), ("talker_hidden", C.c_int), ("emb_dim", C.c_int),
                ("mtp_prec", C.c_int), ("mtp", Mat), ("mtp_bias", C.c_void_p)]


class SampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("rep_penalty", C.c_float),
                ("greedy_warmup", C.c_int), ("text_len", C.c_int)]


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built: run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        vp, i, f = C.c_void_p, C.c_int, C.c_float
        L.qwen_hip_talker_init.argtypes = [C.POINTER(TalkerDesc)]; L.qwen_hip_talker_init.restype = vp
        L.qwen_hip_talker_load_file.argtypes = [C.c_char_p, C.POINTER(TalkerDesc)]
        L.qwen_hip_talker_load_file.restype = vp
        L.qwen_hip_talker_step.argtypes = [vp, vp, vp, i]; L.qwen_hip_talker_step.restype = i
        L.qwen_hip_talker_step_nograph.argtypes = [vp, vp, vp, i]; L.qwen_hip_talker_step_nograph.restype = i
        L.qwen_hip_talker_step_layers.argtypes = [vp, vp, vp, vp, i]; L.qwen_hip_talker_step_layers.restype = i
        L.qwen_hip_talker_get_dec_x.argtypes = [vp, vp]
        L.qwen_hip_talker_upload_kv.argtypes = [vp, vp, vp, i, i]; L.qwen_hip_talker_upload_kv.restype = i
        L.qwen_hip_talker_prefill.argtypes = [vp, vp, vp, i]; L.qwen_hip_talker_prefill.restype = i
        L.qwen_hip_talker_prefill_async.argtypes = [vp, i, i]; L.qwen_hip_talker_prefill_async.restype = i
        L.qwen_hip_op_prefill_gemm.argtypes = [vp, vp, vp, i, i, i, i]; L.qwen_hip_op_prefill_gemm.restype = i
        L.qwen_hip_op_prefill_attention.argtypes = [vp, vp, i, i, i, C.c_float]
        L.qwen_hip_op_prefill_attention.restype = i
        L.qwen_hip_talker_download_kv.argtypes = [vp, vp, vp, i, i]; L.qwen_hip_talker_download_kv.restype = i
        L.qwen_hip_talker_free.argtypes = [vp]
        L.qwen_hip_talker_greedy.argtypes = [vp, vp, vp, i, vp, i, i, i, vp, vp]
        L.qwen_hip_talker_greedy.restype = i
        L.qwen_hip_talker_greedy_async.argtypes = [vp, i]; L.qwen_hip_talker_greedy_async.restype = i
        L.qwen_hip_talker_sync.argtypes = [vp]; L.qwen_hip_talker_sync.restype = i
        L.qwen_hip_talker_stream.argtypes = [vp]; L.qwen_hip_talker_stream.restype = vp
        L.qwen_hip_talker_fused.argtypes = [vp]; L.qwen_hip_talker_fused.restype = i
        L.qwen_hip_talker_fused_kernel.argtypes = [vp]; L.qwen_hip_talker_fused_kernel.restype = i
        L.qwen_hip_talker_grow_kv.argtypes = [vp, i]; L.qwen_hip_talker_grow_kv.restype = i
        L.qwen_hip_talker_kv_max.argtypes = [vp]; L.qwen_hip_talker_kv_max.restype = i
        L.qwen_hip_talker_launch_kernel.argtypes = [vp, i, i, i]; L.qwen_hip_talker_launch_kernel.restype = i
        L.qwen_hip_talker_dequant.argtypes = [vp, i, i, i, i, vp]; L.qwen_hip_talker_dequant.restype = i
        L.qwen_hip_cp_init.argtypes = [C.POINTER(CpDesc)]; L.qwen_hip_cp_init.restype = vp
        L.qwen_hip_cp_step.argtypes = [vp, vp, i]; L.qwen_hip_cp_step.restype = i
        L.qwen_hip_cp_download_kv.argtypes = [vp, vp, vp, i, i]; L.qwen_hip_cp_download_kv.restype = i
        L.qwen_hip_cp_frame.argtypes = [vp, vp, i, vp]; L.qwen_hip_cp_frame.restype = i
        L.qwen_hip_cp_frame_async.argtypes = [vp, i]; L.qwen_hip_cp_frame_async.restype = i
        L.qwen_hip_cp_sync.argtypes = [vp]; L.qwen_hip_cp_sync.restype = i
        L.qwen_hip_cp_fused.argtypes = [vp, i]; L.qwen_hip_cp_fused.restype = i
        L.qwen_hip_cp_stream.argtypes = [vp]; L.qwen_hip_cp_stream.restype = vp
        L.qwen_hip_cp_free.argtypes = [vp]
        L.qwen_hip_available.restype = i
        L.qwen_hip_init.restype = vp
        L.qwen_hip_free.argtypes = [vp]
        L.qwen_hip_matvec_bf16.argtypes = [vp, vp, vp, vp, i, i]
        L.qwen_hip_matmat_bf16.argtypes = [vp, vp, vp, vp, i, i, i]
        L.qwen_hip_op_matvec_int8.argtypes = [vp, vp, vp, vp, i, i]; L.qwen_hip_op_matvec_int8.restype = i
        L.qwen_hip_op_matvec_q4_0.argtypes = [vp, vp, vp, i, i]; L.qwen_hip_op_matvec_q4_0.restype = i
        L.qwen_hip_op_matvec_bf16.argtypes = [vp, vp, vp, i, i]; L.qwen_hip_op_matvec_bf16.restype = i
        L.qwen_hip_op_causal_attention_bf16kv.argtypes = [vp, vp, vp, vp, i, i, i, i, i, f, i]
        L.qwen_hip_op_causal_attention_bf16kv.restype = i
        L.qwen_hip_op_rms_norm.argtypes = [vp, vp, vp, i, i, f]; L.qwen_hip_op_rms_norm.restype = i
        L.qwen_hip_op_rms_norm_per_head.argtypes = [vp, vp, i, i, i, f]; L.qwen_hip_op_rms_norm_per_head.restype = i
        L.qwen_hip_op_swiglu.argtypes = [vp, vp, i]; L.qwen_hip_op_swiglu.restype = i
        L.qwen_hip_op_argmax_matvec.argtypes = [i, vp, vp, vp, i, i]; L.qwen_hip_op_argmax_matvec.restype = i
        L.qwen_hip_op_sample.argtypes = [vp, i, f, i, f, f, vp, i, vp]; L.qwen_hip_op_sample.restype = i
        L.qwen_hip_talker_sample.argtypes = [vp, vp, vp, i, vp, i, i, i, C.POINTER(SampleParams), vp, i, vp, vp, vp]
        L.qwen_hip_talker_sample.restype = i
        L.qwen_hip_generate.argtypes = [vp, vp, vp, vp, i, vp, vp, i, i, i, C.POINTER(SampleParams), vp, i, vp, vp, vp]
        L.qwen_hip_generate.restype = i
        L.qwen_hip_op_codec_sample.argtypes = [vp, i, i, f, f, i, f, f, vp, i, vp]
        L.qwen_hip_op_codec_sample.restype = i
        L.qwen_hip_op_quantize_int8.argtypes = [vp, i, i, vp, vp]; L.qwen_hip_op_quantize_int8.restype = i
        L.qwen_hip_op_quantize_q4_0.argtypes = [vp, i, i, vp]; L.qwen_hip_op_quantize_q4_0.restype = i
        L.qwen_hip_last_error.restype = C.c_char_p
        L.qwen_hip_talker_batch_init.argtypes = [vp, i]; L.qwen_hip_talker_batch_init.restype = vp
        L.qwen_hip_talker_batch_step.argtypes = [vp, vp, vp, vp]; L.qwen_hip_talker_batch_step.restype = i
        L.qwen_hip_talker_batch_step_layers.argtypes = [vp, vp, vp, vp, vp]; L.qwen_hip_talker_batch_step_layers.restype = i
        L.qwen_hip_talker_batch_upload_slot.argtypes = [vp, i, vp, vp, i, i]
        L.qwen_hip_talker_batch_upload_slot.restype = i
        L.qwen_hip_talker_batch_download_slot.argtypes = [vp, i, vp, vp, i, i]
        L.qwen_hip_talker_batch_download_slot.restype = i
        L.qwen_hip_talker_batch_free.argtypes = [vp]
        L.qwen_hip_talker_batch_step_async.argtypes = [vp, i]; L.qwen_hip_talker_batch_step_async.restype = i
        L.qwen_hip_talker_batch_sync.argtypes = [vp]; L.qwen_hip_talker_batch_sync.restype = i
        L.qwen_hip_talker_batch_stream.argtypes = [vp]; L.qwen_hip_talker_batch_stream.restype = vp
        L.qwen_hip_batch_fold_pieces.argtypes = [vp, i]; L.qwen_hip_batch_fold_pieces.restype = i
        L.qwen_hip_cp_batch_init.argtypes = [vp, i]; L.qwen_hip_cp_batch_init.restype = vp
        L.qwen_hip_cp_batch_step.argtypes = [vp, vp, vp]; L.qwen_hip_cp_batch_step.restype = i
        L.qwen_hip_cp_batch_free.argtypes = [vp]
        L.qwen_hip_cp_set_prefill2.argtypes = [vp, i]; L.qwen_hip_cp_set_prefill2.restype = i
        L.qwen_hip_cp_prefill2.argtypes = [vp, vp, vp]; L.qwen_hip_cp_prefill2.restype = i
        L.qwen_hip_op_matmat_int8.argtypes = [vp, vp, vp, vp, i, i, i]; L.qwen_hip_op_matmat_int8.restype = i
        L.qwen_hip_op_matmat_q4_0.argtypes = [vp, vp, vp, i, i, i]; L.qwen_hip_op_matmat_q4_0.restype = i
        L.qwen_hip_op_matmat_int8_noalloc.argtypes = [vp, vp, vp, vp, i, i, i, vp]
        L.qwen_hip_op_matmat_int8_noalloc.restype = i
        L.qwen_hip_sd_init.argtypes = [SD_GET_FN, vp]; L.qwen_hip_sd_init.restype = vp
        L.qwen_hip_sd_load_file.argtypes = [C.c_char_p]; L.qwen_hip_sd_load_file.restype = vp
        L.qwen_hip_sd_decode.argtypes = [vp, vp, i, vp, i]; L.qwen_hip_sd_decode.restype = i
        L.qwen_hip_sd_decode_device.argtypes = [vp, vp, i, vp]; L.qwen_hip_sd_decode_device.restype = i
        L.qwen_hip_sd_latent.argtypes = [vp, vp, i, vp]; L.qwen_hip_sd_latent.restype = i
        L.qwen_hip_sd_stream.argtypes = [vp]; L.qwen_hip_sd_stream.restype = vp
        L.qwen_hip_sd_free.argtypes = [vp]
        L.qwen_hip_op_sd_conv.argtypes = [vp, vp, vp, vp, i, i, i, i, i, i]; L.qwen_hip_op_sd_conv.restype = i
        L.qwen_hip_op_sd_conv_transpose.argtypes = [vp, vp, vp, vp, i, i, i, i, i, i]
        L.qwen_hip_op_sd_conv_transpose.restype = i
        L.qwen_hip_sd_stream_new.argtypes = [vp]; L.qwen_hip_sd_stream_new.restype = vp
        L.qwen_hip_sd_stream_decode.argtypes = [vp, vp, i, vp, i]; L.qwen_hip_sd_stream_decode.restype = i
        L.qwen_hip_sd_stream_reset.argtypes = [vp]; L.qwen_hip_sd_stream_reset.restype = i
        L.qwen_hip_sd_stream_free.argtypes = [vp]
        _lib = L
    return _lib


def last_error():
    return lib().qwen_hip_last_error().decode(errors="replace")


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {last_error()}")


class Talker:
    """Resident Talker (or any stack of layers) on the GPU.

    ``layers`` is a list of dicts {q,k,v,o,gate_up,down: (w, scale|None),
    input_norm, post_attn_norm, q_norm, k_norm}; arrays are numpy (host)."""

    def __init__(self, shape, layers, final_norm, rope_cos, rope_sin, prec, kv_max,
                 quantize_to=-1, cp=False):
        s = shape
        self.keep = []
        nl = len(layers)
        arr = (Layer * nl)()
        for l, ly in enumerate(layers):
            for nm in ["q", "k", "v", "o", "gate_up", "down"]:
                w, sc = ly[nm]
                self.keep += [w, sc]
                getattr(arr[l], nm).w = w.ctypes.data
                getattr(arr[l], nm).scale = None if sc is None else sc.ctypes.data
            for nm in ["input_norm", "post_attn_norm", "q_norm", "k_norm"]:
                a = np.ascontiguousarray(ly[nm], np.float32)
                self.keep.append(a)
                setattr(arr[l], nm, a.ctypes.data)
        fn = np.ascontiguousarray(final_norm, np.float32)
        rc_, rs_ = np.ascontiguousarray(rope_cos, np.float32), np.ascontiguousarray(rope_sin, np.float32)
        self.keep += [fn, rc_, rs_, arr]
        H, F = (s.cp_hidden, s.cp_inter) if cp else (s.hidden, s.inter)
        nh, nkv, hd = (s.cp_heads, s.cp_kv_heads, s.cp_head_dim) if cp else (s.heads, s.kv_heads, s.head_dim)
        self.H = H
        self.desc = TalkerDesc(hidden=H, inter=F, n_heads=nh, n_kv_heads=nkv, head_dim=hd, n_layers=nl,
                               kv_max=kv_max, eps=s.eps, prec=prec, quantize_to=quantize_to, layers=arr,
                               final_norm=fn.ctypes.data, rope_cos=rc_.ctypes.data, rope_sin=rs_.ctypes.data,
                               rope_len=rc_.shape[0])
        self.kv_max = kv_max
        self.kvd = nkv * hd
        self.nl = nl
        self.h = lib().qwen_hip_talker_init(C.byref(self.desc))
        if not self.h:
            raise RuntimeError("qwen_hip_talker_init failed: " + last_error())

    @classmethod
    def from_file(cls, model_path, shape, rope_cos, rope_sin, kv_max, quantize_to=-1):
        """A Talker state loaded by qwen_hip_talker_load_file (file -> device, no host copy)."""
        self = cls.__new__(cls)
        s = shape
        rc_, rs_ = np.ascontiguousarray(rope_cos, np.float32), np.ascontiguousarray(rope_sin, np.float32)
        self.keep = [rc_, rs_]
        self.H = s.hidden
        self.desc = TalkerDesc(hidden=s.hidden, inter=s.inter, n_heads=s.heads, n_kv_heads=s.kv_heads,
                               head_dim=s.head_dim, n_layers=s.layers, kv_max=kv_max, eps=s.eps, prec=BF16,
                               quantize_to=quantize_to, layers=None, final_norm=None, rope_cos=rc_.ctypes.data,
                               rope_sin=rs_.ctypes.data, rope_len=rc_.shape[0])
        self.kv_max, self.kvd, self.nl = kv_max, s.kv_heads * s.head_dim, s.layers
        self.h = lib().qwen_hip_talker_load_file(model_path.encode(), C.byref(self.desc))
        if not self.h:
            raise RuntimeError("qwen_hip_talker_load_file failed: " + last_error())
        return self

    def step(self, embed, pos, graph=True):
        out = np.empty(self.H, np.float32)
        e = np.ascontiguousarray(embed, np.float32)
        fn = lib().qwen_hip_talker_step if graph else lib().qwen_hip_talker_step_nograph
        check(fn(self.h, _p(e), _p(out), pos), "talker_step")
        return out

    def step_layers(self, embed, pos):
        """One step; returns (residual after every layer [n_layers][H], final-normed hidden)."""
        res = np.empty((self.nl, self.H), np.float32)
        out = np.empty(self.H, np.float32)
        e = np.ascontiguousarray(embed, np.float32)
        check(lib().qwen_hip_talker_step_layers(self.h, _p(e), _p(res), _p(out), pos), "talker_step_layers")
        return res, out

    def dec_x(self):
        out = np.empty(self.H, np.float32)
        lib().qwen_hip_talker_get_dec_x(self.h, _p(out))
        return out

    def upload_kv(self, kv_k, kv_v, n):
        check(lib().qwen_hip_talker_upload_kv(self.h, _p(kv_k), _p(kv_v), kv_k.shape[1], n), "upload_kv")

    def prefill(self, embeds, bf16_layers=None):
        """Device prefill of embeds f32[seq][H] (qwen_talker_prefill); fills KV rows
        [0, seq) and dec_x.  A state built from bf16 descriptors (also when quantized on
        the device) passes its own descriptor layers as the bf16 weights."""
        e = np.ascontiguousarray(embeds, np.float32)
        if bf16_layers is None and self.desc.prec == BF16:
            bf16_layers = self.desc.layers
        lp = None if bf16_layers is None else C.cast(bf16_layers, C.c_void_p)
        check(lib().qwen_hip_talker_prefill(self.h, lp, _p(e), e.shape[0]), "talker_prefill")
        self._pf_keep = e
        return self.dec_x()

    def download_kv(self, n):
        k = np.zeros((self.nl, self.kv_max, self.kvd), np.uint16)
        v = np.zeros_like(k)
        check(lib().qwen_hip_talker_download_kv(self.h, _p(k), _p(v), self.kv_max, n), "download_kv")
        return k, v

    def greedy(self, codec_head, codec_emb, embed, pos, frame0, n_steps):
        toks = np.empty(n_steps, np.int32)
        hid = np.empty(self.H, np.float32)
        self._heads = (codec_head, codec_emb)
        check(lib().qwen_hip_talker_greedy(self.h, _p(codec_head), _p(codec_emb), codec_head.shape[0],
                                           _p(np.ascontiguousarray(embed, np.float32)), pos, frame0, n_steps,
                                           _p(toks), _p(hid)), "talker_greedy")
        return toks, hid

    def sample(self, codec_head, codec_emb, embed, pos, frame0, n_steps, temp, top_k, top_p, rep, prev=(), seed=12345,
               greedy_warmup=0, text_len=0):
        """Device frame loop with sampling; returns (tokens generated (ends at the first EOS),
        last normed hidden, new seed)."""
        toks = np.full(n_steps, -1, np.int32)
        hid = np.empty(self.H, np.float32)
        pv = np.ascontiguousarray(prev, np.int32)
        sd = np.array([seed], np.uint32)
        sp = SampleParams(temperature=temp, top_k=top_k, top_p=top_p, rep_penalty=rep, greedy_warmup=greedy_warmup,
                          text_len=text_len)
        self._heads = (codec_head, codec_emb)
        n = lib().qwen_hip_talker_sample(self.h, _p(codec_head), _p(codec_emb), codec_head.shape[0],
                                         _p(np.ascontiguousarray(embed, np.float32)), pos, frame0, n_steps,
                                         C.byref(sp), _p(pv) if pv.size else None, pv.size, _p(sd), _p(toks), _p(hid))
        if n < 0:
            raise RuntimeError(f"talker_sample failed: {last_error()}")
        return toks[:n], hid, int(sd[0])

    def dequant(self, layer, which, r0, n, cols):
        out = np.empty((n, cols), np.float32)
        check(lib().qwen_hip_talker_dequant(self.h, layer, which, r0, n, _p(out)), "dequant")
        return out

    def free(self):
        if self.h:
            lib().qwen_hip_talker_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def generate(talker, cp, codec_head, codec_emb, tts_pad, hidden0, pos, frame0, n_frames, temp=0.0, top_k=0,
             top_p=1.0, rep=1.0, prev=(), seed=12345, greedy_warmup=0, text_len=0):
    """The device frame loop (qwen_hip_generate): returns (codes [n][16] of the frames
    generated, the codes row of the EOS frame or None, last normed hidden, new seed)."""
    codes = np.full((n_frames, 16), -1, np.int32)
    hid = np.empty(talker.H, np.float32)
    pv = np.ascontiguousarray(prev, np.int32)
    sd = np.array([seed], np.uint32)
    sp = SampleParams(temperature=temp, top_k=top_k, top_p=top_p, rep_penalty=rep, greedy_warmup=greedy_warmup,
                      text_len=text_len)
    talker._heads = (codec_head, codec_emb)
    n = lib().qwen_hip_generate(talker.h, cp.h, _p(codec_head), _p(codec_emb), codec_head.shape[0],
                                _p(np.ascontiguousarray(tts_pad, np.float32)),
                                _p(np.ascontiguousarray(hidden0, np.float32)), pos, frame0, n_frames, C.byref(sp),
                                _p(pv) if pv.size else None, pv.size, _p(sd), _p(codes), _p(hid))
    if n < 0:
        raise RuntimeError(f"generate failed: {last_error()}")
    return codes[:n], (codes[n] if n < n_frames else None), hid, int(sd[0])


class SpeechDecoder:
    """The device speech decoder (qwen_hip_sd_*): codes [n][16] -> audio [1920 n]."""

    def __init__(self, h):
        if not h:
            raise RuntimeError(f"speech decoder init failed: {last_error()}")
        self.h = h

    @classmethod
    def from_file(cls, path):
        return cls(lib().qwen_hip_sd_load_file(str(path).encode()))

    @classmethod
    def from_tensors(cls, tensors):
        """Through qwen_hip_sd_init with a getter over a {name: f32 array} dict."""
        keep = {}

        def get(_user, name, n):
            a = tensors.get(name.decode())
            if a is None or a.size != n:
                return None
            keep["cur"] = np.ascontiguousarray(a, np.float32)
            return keep["cur"].ctypes.data

        cb = SD_GET_FN(get)
        return cls(lib().qwen_hip_sd_init(cb, None))

    def decode(self, codes):
        codes = np.ascontiguousarray(codes, np.int32)
        n = codes.shape[0]
        out = np.empty(n * SD_SAMPLES_PER_FRAME, np.float32)
        ns = lib().qwen_hip_sd_decode(self.h, codes.ctypes.data, n, out.ctypes.data, out.size)
        if ns < 0:
            raise RuntimeError(f"sd_decode failed: {last_error()}")
        return out[:ns]

    def latent(self, codes):
        codes = np.ascontiguousarray(codes, np.int32)
        out = np.empty((codes.shape[0], 1024), np.float32)
        check(lib().qwen_hip_sd_latent(self.h, codes.ctypes.data, codes.shape[0], out.ctypes.data), "sd_latent")
        return out

    def free(self):
        if self.h:
            lib().qwen_hip_sd_free(self.h)
            self.h = None


class SpeechDecoderStream:
    """Streaming decode over a SpeechDecoder (qwen_hip_sd_stream_*): each call returns the
    new frames' 1920 samples each."""

    def __init__(self, dec):
        self.h = lib().qwen_hip_sd_stream_new(dec.h)
        if not self.h:
            raise RuntimeError(f"sd stream init failed: {last_error()}")

    def decode(self, codes):
        codes = np.ascontiguousarray(codes, np.int32)
        out = np.empty(codes.shape[0] * SD_SAMPLES_PER_FRAME, np.float32)
        ns = lib().qwen_hip_sd_stream_decode(self.h, codes.ctypes.data, codes.shape[0], out.ctypes.data, out.size)
        if ns < 0:
            raise RuntimeError(f"sd_stream_decode failed: {last_error()}")
        return out[:ns]

    def reset(self):
        check(lib().qwen_hip_sd_stream_reset(self.h), "sd_stream_reset")

    def free(self):
        if self.h:
            lib().qwen_hip_sd_stream_free(self.h)
            self.h = None


class TalkerBatch:
    """B streams over a Talker's resident weights (qwen_hip_talker_batch_*)."""

    def __init__(self, talker, B):
        self.t, self.B = talker, B
        self.h = lib().qwen_hip_talker_batch_init(talker.h, B)
        if not self.h:
            raise RuntimeError("qwen_hip_talker_batch_init failed: " + last_error())

    def step(self, embeds, pos):
        e = np.ascontiguousarray(embeds, np.float32).reshape(self.B, self.t.H)
        p = np.ascontiguousarray(pos, np.int32)
        out = np.empty((self.B, self.t.H), np.float32)
        check(lib().qwen_hip_talker_batch_step(self.h, _p(e), _p(p), _p(out)), "talker_batch_step")
        return out

    def step_layers(self, embeds, pos):
        """One ungraphed batched step; returns (residuals [n_layers][B][H], hidden [B][H])."""
        e = np.ascontiguousarray(embeds, np.float32).reshape(self.B, self.t.H)
        p = np.ascontiguousarray(pos, np.int32)
        res = np.empty((self.t.nl, self.B, self.t.H), np.float32)
        out = np.empty((self.B, self.t.H), np.float32)
        check(lib().qwen_hip_talker_batch_step_layers(self.h, _p(e), _p(p), _p(res), _p(out)), "talker_batch_step_layers")
        return res, out

    def fold_pieces(self, on):
        """int8: activation pieces inside the projection launches (True) or apart; returns the mode in effect."""
        r = lib().qwen_hip_batch_fold_pieces(self.h, int(bool(on)))
        if r < 0:
            raise RuntimeError("qwen_hip_batch_fold_pieces failed: " + last_error())
        return bool(r)

    def upload_slot(self, b, kv_k, kv_v, n):
        """kv_k/kv_v: [B][n_layers][src_kv_max][kv_dim] bf16 (the batch engine layout)."""
        check(lib().qwen_hip_talker_batch_upload_slot(self.h, b, _p(kv_k), _p(kv_v), kv_k.shape[2], n), "upload_slot")

    def download_slot(self, b, n):
        k = np.zeros((self.B, self.t.nl, self.t.kv_max, self.t.kvd), np.uint16)
        v = np.zeros_like(k)
        check(lib().qwen_hip_talker_batch_download_slot(self.h, b, _p(k), _p(v), self.t.kv_max, n), "download_slot")
        return k[b], v[b]

    def free(self):
        if self.h:
            lib().qwen_hip_talker_batch_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class CodePredictor:
    def __init__(self, desc: CpDesc, keep):
        self.desc, self.keep = desc, keep
        self.h = lib().qwen_hip_cp_init(C.byref(desc))
        if not self.h:
            raise RuntimeError("qwen_hip_cp_init failed: " + last_error())
        self.H = desc.cp.hidden

    def frame(self, talker_hidden, code0):
        out = (C.c_int * 15)()
        check(lib().qwen_hip_cp_frame(self.h, _p(np.ascontiguousarray(talker_hidden, np.float32)), code0, out),
              "cp_frame")
        return np.array(list(out), np.int32)

    def step(self, x, pos):
        x = np.array(x, np.float32, copy=True)
        check(lib().qwen_hip_cp_step(self.h, _p(x), pos), "cp_step")
        return x

    def download_kv(self, n):
        """Positions [0, n) of the CP cache as host bf16 [cp_layers][n][kv_dim]."""
        L, kvd = self.desc.cp.n_layers, self.desc.cp.n_kv_heads * self.desc.cp.head_dim
        k = np.zeros((L, n, kvd), np.uint16)
        v = np.zeros_like(k)
        check(lib().qwen_hip_cp_download_kv(self.h, _p(k), _p(v), n, n), "cp_download_kv")
        return k, v

    def fused(self, on):
        """Frames on the role-specialised kernel (True) or the per-kernel graph; returns the mode in effect."""
        r = lib().qwen_hip_cp_fused(self.h, int(bool(on)))
        if r < 0:
            raise RuntimeError("qwen_hip_cp_fused failed: " + last_error())
        return bool(r)

    def set_prefill2(self, on):
        """Frames start with the two-position pass (int8 CP weights only)."""
        check(lib().qwen_hip_cp_set_prefill2(self.h, int(on)), "cp_set_prefill2")

    def prefill2(self, x0, x1):
        """Positions 0 and 1 as one two-column pass; returns the two residuals."""
        x0 = np.array(x0, np.float32, copy=True)
        x1 = np.array(x1, np.float32, copy=True)
        check(lib().qwen_hip_cp_prefill2(self.h, _p(x0), _p(x1)), "cp_prefill2")
        return x0, x1

    def batch_step(self, x, pos):
        """One pass for B streams (own CP KVs) over this CP's weights; x [B][H]."""
        x = np.array(x, np.float32, copy=True)
        B = x.shape[0]
        if getattr(self, "_bh", None) is None or self._bB != B:
            if getattr(self, "_bh", None):
                lib().qwen_hip_cp_batch_free(self._bh)
            self._bh = lib().qwen_hip_cp_batch_init(self.h, B)
            self._bB = B
            if not self._bh:
                raise RuntimeError("qwen_hip_cp_batch_init failed: " + last_error())
        check(lib().qwen_hip_cp_batch_step(self._bh, _p(x), _p(np.ascontiguousarray(pos, np.int32))), "cp_batch_step")
        return x

    def free(self):
        if getattr(self, "_bh", None):
            lib().qwen_hip_cp_batch_free(self._bh)
            self._bh = None
        if self.h:
            lib().qwen_hip_cp_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def cp_from_tensors(t, shape, prec=BF16, cp_kv_max=64):
    """A CodePredictor (bf16 weights, optionally quantized on the device to ``prec``) over
    synth tensors {reference name: bf16 array}: CP layers, cp_norm, the 15 lm heads and
    codec embeddings, the Talker codec embedding, and (when the Talker and CP hidden sizes
    differ, as in the 1.7B model) the small_to_mtp_projection in bf16 with its bias."""
    from .synth import bf16_to_f32, rope_tables
    s = shape
    keep = []
    layers = layers_from_tensors(t, s, cp=True)
    arr = (Layer * len(layers))()
    for l, ly in enumerate(layers):
        for nm in ["q", "k", "v", "o", "gate_up", "down"]:
            w, _ = ly[nm]
            keep.append(w)
            getattr(arr[l], nm).w = w.ctypes.data
            getattr(arr[l], nm).scale = None
        for nm in ["input_norm", "post_attn_norm", "q_norm", "k_norm"]:
            a = np.ascontiguousarray(ly[nm], np.float32)
            keep.append(a)
            setattr(arr[l], nm, a.ctypes.data)
    cos, sin = rope_tables(s.cp_head_dim, s.rope_theta, cp_kv_max)
    fn = np.ascontiguousarray(bf16_to_f32(t["talker.code_predictor.model.norm.weight"]))
    keep += [arr, cos, sin, fn]
    d = CpDesc()
    d.cp = TalkerDesc(hidden=s.cp_hidden, inter=s.cp_inter, n_heads=s.cp_heads, n_kv_heads=s.cp_kv_heads,
                      head_dim=s.cp_head_dim, n_layers=len(layers), kv_max=cp_kv_max, eps=s.eps, prec=BF16,
                      quantize_to=-1 if prec == BF16 else prec, layers=arr, final_norm=fn.ctypes.data,
                      rope_cos=cos.ctypes.data, rope_sin=sin.ctypes.data, rope_len=cp_kv_max)
    d.codebook = s.codebook
    d.lm_prec = BF16
    for g in range(15):
        lm = np.ascontiguousarray(t[f"talker.code_predictor.lm_head.{g}.weight"])
        ce = np.ascontiguousarray(t[f"talker.code_predictor.model.codec_embedding.{g}.weight"])
        keep += [lm, ce]
        d.lm_head[g].w = lm.ctypes.data
        d.lm_head[g].scale = None
        d.cp_codec_emb[g] = ce.ctypes.data
    te = np.ascontiguousarray(t["talker.model.codec_embedding.weight"])
    keep.append(te)
    d.talker_codec_emb = te.ctypes.data
    d.codec_vocab = s.codec_vocab
    d.talker_hidden = s.hidden
    d.emb_dim = s.hidden
    d.mtp.w = None
    if s.hidden != s.cp_hidden:
        mw = np.ascontiguousarray(t["talker.code_predictor.small_to_mtp_projection.weight"])
        mb = np.ascontiguousarray(bf16_to_f32(t["talker.code_predictor.small_to_mtp_projection.bias"]))
        keep += [mw, mb]
        d.mtp_prec = BF16
        d.mtp.w = mw.ctypes.data
        d.mtp.scale = None
        d.mtp_bias = mb.ctypes.data
    return CodePredictor(d, keep)


def layers_from_ref(ref, prec_code, cp=False):
    """Layer dicts over the reference-loaded (and reference-quantized) weights."""
    s = ref.shape
    nl = s.cp_layers if cp else s.layers
    kind = {BF16: "bf16", INT8: "int8", Q4_0: "q4"}[prec_code]
    out = []
    for l in range(nl):
        d = {}
        for nm in ["q", "k", "v", "o", "gate_up", "down"]:
            m = ref.layer_mat(l, nm, cp=cp)
            d[nm] = (m[kind], m["scale"] if prec_code == INT8 else None)
        d["input_norm"] = ref.layer_norm(l, "input", cp=cp)
        d["post_attn_norm"] = ref.layer_norm(l, "post", cp=cp)
        d["q_norm"] = ref.layer_norm(l, "q", cp=cp)
        d["k_norm"] = ref.layer_norm(l, "k", cp=cp)
        out.append(d)
    return out


def layers_from_tensors(t, shape, cp=False):
    """Layer dicts (bf16) straight from synth tensors {name: uint16 array}; gate|up
    interleaved the way the reference loader does (qwen_tts_talker.c:378-388)."""
    from .synth import interleave_gate_up, bf16_to_f32
    s = shape
    nl = s.cp_layers if cp else s.layers
    pre = "talker.code_predictor.model.layers." if cp else "talker.model.layers."
    out = []
    for l in range(nl):
        p = f"{pre}{l}."
        gu = interleave_gate_up(t[p + "mlp.gate_proj.weight"], t[p + "mlp.up_proj.weight"])
        out.append({
            "q": (t[p + "self_attn.q_proj.weight"], None), "k": (t[p + "self_attn.k_proj.weight"], None),
            "v": (t[p + "self_attn.v_proj.weight"], None), "o": (t[p + "self_attn.o_proj.weight"], None),
            "gate_up": (gu, None), "down": (t[p + "mlp.down_proj.weight"], None),
            "input_norm": bf16_to_f32(t[p + "input_layernorm.weight"]),
            "post_attn_norm": bf16_to_f32(t[p + "post_attention_layernorm.weight"]),
            "q_norm": bf16_to_f32(t[p + "self_attn.q_norm.weight"]),
            "k_norm": bf16_to_f32(t[p + "self_attn.k_norm.weight"]),
        })
    return out
