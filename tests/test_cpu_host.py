"""Host-side checks that need no GPU: the C-ABI library loads and exports every symbol
include/qwen_tts_hip.h declares, the ctypes mirrors have the C layouts, the synthetic
weight generator is deterministic and rounds like the reference's bf16 export, the
product path fails loudly without a GPU (no CPU fallback), and bench.py refuses
multi-GPU runs."""
import ctypes as C
import os
import re
import subprocess
import sys
import tempfile

import numpy as np
import pytest

from conftest import HIP_LIB, ROOT

HEADER = os.path.join(ROOT, "include", "qwen_tts_hip.h")
need_lib = pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libqwen_tts_hip.so not built")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(qwen_hip_\w+)\s*\(", src)))


def test_exports_list_matches_header():
    from qwen3_tts_amd import hip
    assert sorted(hip.EXPORTS) == header_functions()


@need_lib
def test_library_loads_and_exports_every_declared_symbol():
    lib = C.CDLL(HIP_LIB)
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", HIP_LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (qwen_hip_\w+)", out))
    assert set(header_functions()) <= exported


@need_lib
def test_no_gpu_means_a_loud_failure_not_a_fallback():
    """Without a GPU (this container) the library reports unavailability and init
    returns NULL with an error message; nothing computes on the CPU instead."""
    from qwen3_tts_amd import hip, synth
    L = hip.lib()
    if L.qwen_hip_available():
        pytest.skip("a GPU is visible")
    s = synth.SHAPES["tiny"]
    t = synth.generate(s, 1, 0.0, threads=4, only=lambda n: n.startswith("talker.model."))
    layers = hip.layers_from_tensors(t, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, 64)
    with pytest.raises(RuntimeError):
        hip.Talker(s, layers, synth.bf16_to_f32(t["talker.model.norm.weight"]), cos, sin, hip.BF16, 64)


def test_missing_library_raises(monkeypatch):
    from qwen3_tts_amd import hip
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setattr(hip, "LIB_PATH", "/nonexistent/libqwen_tts_hip.so")
    with pytest.raises(RuntimeError):
        hip.lib()


def test_ctypes_structs_match_c_layout():
    """Compile a probe against the header and compare sizeof/offsetof with hip.py."""
    from qwen3_tts_amd import hip
    structs = {"qwen_hip_mat_t": hip.Mat, "qwen_hip_layer_t": hip.Layer,
               "qwen_hip_talker_desc_t": hip.TalkerDesc, "qwen_hip_cp_desc_t": hip.CpDesc,
               "qwen_hip_sample_params_t": hip.SampleParams}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "qwen_tts_hip.h"', 'int main(void){']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, "probe.c")
        open(src, "w").write("\n".join(lines))
        exe = os.path.join(td, "probe")
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
                        "-D__HIP_PLATFORM_AMD__", src, "-o", exe], check=True, capture_output=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for ln in out:
        if ln:
            a, b, c = ln.split()
            got[(a, b)] = int(c)
    for cname, py in structs.items():
        assert got[(cname, "size")] == C.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, (cname, f)


def test_synth_is_deterministic_and_seed_sensitive():
    from qwen3_tts_amd import synth
    s = synth.SHAPES["tiny"]
    only = lambda n: n.startswith("talker.model.layers.0.")  # noqa: E731
    a = synth.generate(s, 42, 0.1, threads=2, only=only)
    b = synth.generate(s, 42, 0.1, threads=4, only=only)
    c = synth.generate(s, 43, 0.1, threads=2, only=only)
    assert a.keys() == b.keys() and len(a) > 0
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    k = "talker.model.layers.0.self_attn.q_proj.weight"
    assert not np.array_equal(a[k], c[k])
    w = synth.bf16_to_f32(a[k]).astype(np.float64)
    assert abs(w.std() - 0.02) < 0.002 and abs(w.mean()) < 0.002


def test_bf16_round_to_nearest_even():
    """f32 -> bf16 as the reference's weight export stores it: nearest, ties to even."""
    from qwen3_tts_amd import synth
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, 5000).astype(np.float32)
    # add exact ties: low 16 bits 0x8000
    t = (rng.integers(0, 2**31, 200, dtype=np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, t.view(np.float32)[np.isfinite(t.view(np.float32))]])
    b = synth.f32_to_bf16_rne(x)
    lo = (x.view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((x.view(np.uint32) & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    got = synth.bf16_to_f32(b).astype(np.float64)
    xd = x.astype(np.float64)
    near = np.where(np.abs(xd - lo) < np.abs(hi - xd), lo, hi)
    tie = np.abs(xd - lo) == np.abs(hi - xd)
    even = np.where(((x.view(np.uint32) >> 16) & 1) == 0, lo, hi)
    assert np.array_equal(got, np.where(tie, even, near))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout


REF_ROOT = "/root/reference"


@pytest.mark.skipif(not os.path.isdir(REF_ROOT), reason="reference sources not present")
def test_glue_compiles_against_reference_header():
    """The reference-side glue (qwen3-tts_amd/glue) is real C against the reference's own
    qwen_tts.h: it compiles warning-free with the reference's flags."""
    glue = os.path.join(ROOT, "qwen3-tts_amd", "glue")
    r = subprocess.run(["gcc", "-fsyntax-only", "-O3", "-mavx2", "-mfma", "-ffast-math", "-Wall", "-Wextra",
                        "-Wno-unused-parameter", "-Werror", f"-I{REF_ROOT}", f"-I{REF_ROOT}/vendor",
                        f"-I{REF_ROOT}/third_party/ingot/include", "-I", os.path.join(ROOT, "include"), "-I", glue,
                        os.path.join(glue, "qwen_tts_hip_glue.c")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_glue_calls_only_declared_entry_points():
    """Every library function the glue calls is declared in include/qwen_tts_hip.h."""
    src = open(os.path.join(ROOT, "qwen3-tts_amd", "glue", "qwen_tts_hip_glue.c")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    called = set(re.findall(r"\b(qwen_hip_(?!glue_)\w+)\s*\(", src))
    assert called and called <= set(header_functions()), called - set(header_functions())


def _load_desc(shape, kv_max=64):
    from qwen3_tts_amd import hip, synth
    cos, sin = synth.rope_tables(shape.head_dim, shape.rope_theta, kv_max)
    return hip.TalkerDesc(hidden=shape.hidden, inter=shape.inter, n_heads=shape.heads, n_kv_heads=shape.kv_heads,
                          head_dim=shape.head_dim, n_layers=shape.layers, kv_max=kv_max, eps=shape.eps, prec=0,
                          quantize_to=-1, layers=None, final_norm=None, rope_cos=cos.ctypes.data,
                          rope_sin=sin.ctypes.data, rope_len=kv_max), (cos, sin)


@need_lib
def test_load_file_validates_before_touching_the_gpu(tmp_path):
    """qwen_hip_talker_load_file parses the safetensors header and checks every tensor the
    step needs (name, dtype, shape, extent) before any GPU call: a valid model gets as far
    as 'no HIP device' here; a missing file, a broken header, a missing tensor or a
    dimension mismatch are reported by name."""
    import ctypes as C
    import json
    import struct
    from qwen3_tts_amd import hip, synth
    L = hip.lib()
    if L.qwen_hip_available():
        pytest.skip("a GPU is visible")
    s = synth.SHAPES["tiny"]
    good = tmp_path / "good"
    synth.write_model_dir(str(good), s, 7, 0.0, threads=4)
    desc, keep = _load_desc(s)
    assert not L.qwen_hip_talker_load_file(str(good).encode(), C.byref(desc))
    assert "no HIP device" in hip.last_error()
    assert not L.qwen_hip_talker_load_file(str(tmp_path / "nope").encode(), C.byref(desc))
    assert "cannot open" in hip.last_error()
    # a header that is not JSON
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", 5) + b"{oops" + b"\0" * 16)
    assert not L.qwen_hip_talker_load_file(str(bad).encode(), C.byref(desc))
    assert "malformed" in hip.last_error()
    # a tensor missing: rewrite the header without the last layer's v_proj
    raw = (good / "model.safetensors").read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    name = f"talker.model.layers.{s.layers - 1}.self_attn.v_proj.weight"
    del hdr[name]
    h2 = json.dumps(hdr).encode()
    miss = tmp_path / "miss.safetensors"
    miss.write_bytes(struct.pack("<Q", len(h2)) + h2 + raw[8 + n:])
    assert not L.qwen_hip_talker_load_file(str(miss).encode(), C.byref(desc))
    assert "missing tensor " + name in hip.last_error()
    # dimensions that do not match the file
    desc2, keep2 = _load_desc(synth.ModelShape(hidden=512, layers=2, heads=4, kv_heads=2, inter=512))
    assert not L.qwen_hip_talker_load_file(str(good).encode(), C.byref(desc2))
    assert "expected BF16" in hip.last_error()
