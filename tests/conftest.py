"""Shared fixtures.  GPU tests are marked ``gpu``; everything else runs on the CPU."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_pkg():
    """Import the hyphenated package directory qwen3-tts_amd as ``qwen3_tts_amd``."""
    if "qwen3_tts_amd" in sys.modules:
        return sys.modules["qwen3_tts_amd"]
    pdir = os.path.join(ROOT, "qwen3-tts_amd")
    spec = importlib.util.spec_from_file_location("qwen3_tts_amd", os.path.join(pdir, "__init__.py"),
                                                  submodule_search_locations=[pdir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qwen3_tts_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


load_pkg()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long-running parity case")


REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libqwen_ref.so")
ORACLE_LIB = os.path.join(ROOT, "oracle", "liboracle.so")
HIP_LIB = os.path.join(ROOT, "qwen3-tts_amd", "libqwen_tts_hip.so")

need_ref = pytest.mark.skipif(not os.path.exists(REF_LIB), reason="oracle/_ref not built (no reference sources)")
need_oracle = pytest.mark.skipif(not os.path.exists(ORACLE_LIB), reason="oracle/liboracle.so not built")

_MODEL_CACHE = {}


def model_dir(name, seed=0x5EED0001, gain_jitter=0.1):
    """Write (once per session) a synthetic model directory; returns (dir, shape, tensors)."""
    from qwen3_tts_amd import synth
    key = (name, seed, gain_jitter)
    if key not in _MODEL_CACHE:
        base = os.environ.get("QWEN_TEST_MODELS", "/tmp/qwen3tts_test_models")
        d = os.path.join(base, f"{name}_{seed:x}_{gain_jitter}")
        shape = synth.SHAPES[name]
        t = synth.generate(shape, seed, gain_jitter, threads=8)
        if not os.path.exists(os.path.join(d, "model.safetensors")):
            synth.write_model_dir(d, shape, seed, gain_jitter, tensors=t)
        _MODEL_CACHE[key] = (d, shape, t)
    return _MODEL_CACHE[key]


_SD_CACHE = {}


def sd_model(seed=0x5EED0D0C):
    """Write (once per session) the synthetic speech-decoder file; returns (path, tensors)."""
    from qwen3_tts_amd import synth_sd
    if seed not in _SD_CACHE:
        base = os.environ.get("QWEN_TEST_MODELS", "/tmp/qwen3tts_test_models")
        t = synth_sd.generate_sd(seed)
        _SD_CACHE[seed] = (synth_sd.write_sd(os.path.join(base, f"sd_{seed:x}"), seed, tensors=t), t)
    return _SD_CACHE[seed]


def sd_codes(n, seed):
    """Seeded codes [n][16] in [0, 2048), with one code out of range (-1 or 2048) in every
    third frame (the reference skips those lookups, sd.c:607-623)."""
    rng = np.random.default_rng(seed)
    c = rng.integers(0, 2048, (n, 16)).astype(np.int32)
    for f in range(0, n, 3):
        c[f, int(rng.integers(0, 16))] = -1 if f % 2 else 2048
    return c


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    if not os.path.exists(ORACLE_LIB):
        pytest.skip("oracle not built")
    return Oracle()


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def sample_cases(n_cases, seed, rule=False):
    """Seeded arguments for qwen_tts_sample (vocab 1..4096, temperatures including greedy,
    top-k, top-p, repetition penalty with repeated history tokens); ties at the maximum
    only where top-p is off (the one place tie order decides the result)."""
    rng = np.random.default_rng(seed)
    for c in range(n_cases):
        V = 3072 if (rule or c % 3) else int(rng.integers(1, 4097))
        lg = (rng.standard_normal(V) * [0.5, 2.0, 5.0][c % 3]).astype(np.float32)
        temp = [0.0, 0.3, 0.9, 1.0, 1.5][c % 5]
        top_k = [0, 1, 50, 200, V][(c // 5) % 5]
        top_p = [1.0, 0.9, 0.5, 0.99, 1e-6][(c // 3) % 5]
        rep = [1.0, 1.05, 1.3][(c // 7) % 3]
        if top_p == 1.0 and c % 4 == 0:
            lg[rng.integers(0, V, 12)] = lg.max()
        prev = rng.integers(0, V, int(rng.integers(0, 40))).astype(np.int32)
        sd = int(rng.integers(0, 2 ** 32))
        extra = (int(rng.integers(0, 6)), float([0.0, 0.0, 3.5][c % 3])) if rule else None
        yield dict(logits=lg, temp=temp, top_k=top_k, top_p=top_p, rep=rep, prev=prev, seed=sd, rule=extra)


def draw_margin(dist, seed_after):
    """Distance of the draw r (from the advanced LCG state) to the nearest boundary of the
    cumulative distribution: two correct samplers whose sums round differently may only
    disagree when this is tiny."""
    r = float((seed_after >> 16) & 0x7FFF) / 32768.0
    cum = np.cumsum(dist.astype(np.float64))
    return float(np.min(np.abs(cum - r)))
