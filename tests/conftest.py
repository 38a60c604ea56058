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


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    if not os.path.exists(ORACLE_LIB):
        pytest.skip("oracle not built")
    return Oracle()


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
