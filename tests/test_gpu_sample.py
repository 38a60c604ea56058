"""GPU parity of the device sampler (qwen_tts_sample, qwen_tts_sampling.c:160-202, and the
codec-head rule of qwen_tts.c:1652-1679 in front of it) against the oracle's restatement,
which is pinned to the compiled reference's qwen_tts_sample.  The LCG state must always
agree; greedy tokens must agree exactly; sampled tokens must agree unless the draw lies
within rounding of a cumulative boundary (the device sums in a tree order)."""
import numpy as np
import pytest

from conftest import draw_margin, sample_cases

pytestmark = pytest.mark.gpu

from qwen3_tts_amd import hip  # noqa: E402


def _dev(case):
    L = hip.lib()
    lg = np.ascontiguousarray(case["logits"], np.float32)
    pv = np.ascontiguousarray(case["prev"], np.int32)
    sd = np.array([case["seed"]], np.uint32)
    pp = pv.ctypes.data if pv.size else None
    if case["rule"] is None:
        t = L.qwen_hip_op_sample(lg.ctypes.data, lg.size, case["temp"], case["top_k"], case["top_p"], case["rep"],
                                 pp, pv.size, sd.ctypes.data)
    else:
        fr, boost = case["rule"]
        t = L.qwen_hip_op_codec_sample(lg.ctypes.data, lg.size, fr, boost, case["temp"], case["top_k"],
                                       case["top_p"], case["rep"], pp, pv.size, sd.ctypes.data)
    assert t >= 0, hip.last_error()
    return t, int(sd[0])


@pytest.mark.parametrize("rule", [False, True])
def test_sample_matches_oracle(oracle, rule):
    print(f"[case] device sampling rule={rule}", flush=True)
    n = diff = 0
    for case in sample_cases(400, 17 + rule, rule=rule):
        t, s = _dev(case)
        t_o, s_o, dist = oracle.sample(case["logits"], case["temp"], case["top_k"], case["top_p"], case["rep"],
                                       case["prev"], case["seed"], rule=case["rule"])
        n += 1
        assert s == s_o
        if case["temp"] < 1e-6:
            assert t == t_o
        elif t != t_o:
            diff += 1
            assert draw_margin(dist, s) < 1e-5, (case["temp"], case["top_k"], case["top_p"], t, t_o)
    assert diff <= n // 100, diff


def test_sample_argument_errors():
    L = hip.lib()
    lg = np.zeros(5000, np.float32)
    sd = np.array([1], np.uint32)
    assert L.qwen_hip_op_sample(lg.ctypes.data, 5000, 1.0, 0, 1.0, 1.0, None, 0, sd.ctypes.data) == -1
    assert L.qwen_hip_op_sample(lg.ctypes.data, 0, 1.0, 0, 1.0, 1.0, None, 0, sd.ctypes.data) == -1
    assert L.qwen_hip_op_sample(lg.ctypes.data, 16, 1.0, 0, 1.0, 1.0, None, 3, sd.ctypes.data) == -1
    assert int(sd[0]) == 1
    assert L.qwen_hip_op_sample(lg.ctypes.data, 16, 1.0, 0, 1.0, 1.0, None, 0, sd.ctypes.data) >= 0
