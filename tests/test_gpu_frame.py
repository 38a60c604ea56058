"""The whole frame loop on the device (qwen_hip_generate) against the reference's own frame
loop (qwen_tts.c:1649-1778): codec head + rule + sampling for code0, qwen_cp_predict for
the 15 CP codes, the next input codec_embedding[code0] + sum_g cp_codec_emb[g][code_g] +
tts_pad (restated here in the reference's f32 add order, lookup_codec_embed
qwen_tts.c:919-924 and qwen_bf16_accum_f32 qwen_tts_kernels.c:3900-3925), then
qwen_talker_step.  The loop starts after a reference prefill: the device gets the
prefill's KV through upload_kv and last_hidden = rms_norm(dec_x, talker_norm)
(qwen_tts.c:1521-1522), as the reference's own GPU hand-off does."""
import numpy as np
import pytest

from conftest import draw_margin, model_dir, need_ref, rel_l2

pytestmark = [pytest.mark.gpu, need_ref]

from qwen3_tts_amd import hip, synth  # noqa: E402


def _setup(name, prec, n_prefill=12, kv_max=128):
    from oracle.oracle import RefModel
    from test_gpu_parity import _gpu_cp
    d, s, _ = model_dir(name)
    ref = RefModel(d, s, prec=prec, threads=8)
    pc = hip.PREC[prec]
    layers = hip.layers_from_ref(ref, pc)
    cos, sin = ref.rope()
    g = hip.Talker(s, layers, ref.final_norm(), cos, sin, pc, kv_max)
    cp = _gpu_cp(ref, s, pc)
    emb = ref.codec_emb()
    rng = np.random.default_rng(31)
    E = synth.bf16_to_f32(emb[rng.integers(0, 2048, n_prefill)]).astype(np.float32)
    ref.kv_len = 0
    dx = ref.prefill(E)
    kr, vr = ref.kv()
    g.upload_kv(np.ascontiguousarray(kr[:, :n_prefill]), np.ascontiguousarray(vr[:, :n_prefill]), n_prefill)
    h0 = np.empty(s.hidden, np.float32)
    R = RefModel.load_lib()
    fn = ref.final_norm()
    R.ref_rms_norm(h0.ctypes.data, dx.ctypes.data, fn.ctypes.data, 1, s.hidden, np.float32(s.eps))
    pad = (rng.standard_normal(s.hidden) * 0.02).astype(np.float32)      # the text side's tts_pad embedding
    return ref, s, g, cp, h0, pad, n_prefill


def _next_input(ref, emb, codes, pad):
    e = synth.bf16_to_f32(emb[codes[0]]).astype(np.float32)
    for gi in range(15):
        e = (e + synth.bf16_to_f32(ref.cp_codec_emb(gi)[codes[gi + 1]])).astype(np.float32)
    return (e + pad).astype(np.float32)


def _f64_rows(bf16=None, i8=None, scale=None, rows=0, cols=0):
    if i8 is not None:
        return i8.reshape(rows, cols).astype(np.float64) * scale.astype(np.float64)[:, None]
    return synth.bf16_to_f32(bf16.reshape(rows, cols)).astype(np.float64)


def _code_margin(ref, s, cp, h, frame, want, got, k):
    """|logit(want[k]) - logit(got[k])| where the two frames first part at code k, on the
    reference's trajectory (hidden h entering the frame, its codes `want`): code 0 from the
    reference's own codec-head logits; a CP code from the logits of the CP pass that
    chooses it, on the device's pass (qwen_hip_cp_step, teacher-forced with the reference's
    codes; mtp projection and lm head in float64 on the host).  A parting by f32 rounding
    is a near-tie: the gap is a rounding-sized number."""
    if k == 0:
        _, lg = ref.codec_greedy(h, frame)
        return abs(float(lg[want[0]]) - float(lg[got[0]]))
    R = ref.lib
    mtp = None
    if s.hidden != s.cp_hidden:
        m = ref.cp_mtp()
        w = _f64_rows(i8=m["int8"], scale=m["scale"], rows=s.cp_hidden, cols=s.hidden) \
            if R.ref_cp_mtp(ref.h, 1) else _f64_rows(bf16=m["bf16"], rows=s.cp_hidden, cols=s.hidden)
        mtp = (w, m["bias"].astype(np.float64) if m["bias"] is not None else 0.0)

    def proj(v):
        if mtp is None:
            return v.astype(np.float32)
        return (mtp[0] @ v.astype(np.float64) + mtp[1]).astype(np.float32)

    emb = ref.codec_emb()
    cn = ref.cp_norm().astype(np.float64)
    x = proj(h)
    for p in range(k + 1):
        if p == 1:
            x = proj(synth.bf16_to_f32(emb[want[0]]))
        elif p >= 2:
            x = proj(synth.bf16_to_f32(ref.cp_codec_emb(p - 2)[want[p - 1]]))
        x = cp.step(x, p)
    xd = x.astype(np.float64)
    xn = xd / np.sqrt((xd * xd).mean() + s.eps) * cn
    lm = ref.cp_lm_head(k - 1)
    W = _f64_rows(i8=lm["int8"], scale=lm["scale"], rows=s.codebook, cols=s.cp_hidden) \
        if R.ref_cp_lm_head(ref.h, k - 1, 1) else _f64_rows(bf16=lm["bf16"], rows=s.codebook, cols=s.cp_hidden)
    lg = W @ xn
    return abs(float(lg[want[k]]) - float(lg[got[k]]))


@pytest.mark.parametrize("name,prec", [("mini", "bf16"), ("mini", "int8"), ("mini17", "int8"), ("0.6B", "bf16"),
                                       ("1.7B", "int8")])
def test_generate_greedy_matches_reference(name, prec):
    """Greedy decoding: every frame's code0 and 15 CP codes identical to the reference's,
    and the final hidden state within the north-star bars.  16 frames at the full shapes."""
    print(f"[case] generate greedy {name} {prec}", flush=True)
    ref, s, g, cp, h0, pad, P = _setup(name, prec)
    n = 10 if name.startswith("mini") else 16
    head = np.ascontiguousarray(ref.codec_head())
    embc = np.ascontiguousarray(ref.codec_emb())
    codes, eos_row, h_dev, _ = hip.generate(g, cp, head, embc, pad, h0, P, 0, n)
    want, hs, h = [], [h0], h0
    for f in range(n):
        code0, _ = ref.codec_greedy(h, f)
        if code0 == 2150:
            break
        row = [code0] + [int(c) for c in ref.cp_predict(h, code0)]
        want.append(row)
        h = ref.step(_next_input(ref, embc, row, pad))
        hs.append(h)
    got = [[int(c) for c in r] for r in codes]
    first = next((i for i in range(min(len(got), len(want))) if got[i] != want[i]), None)
    if first is None:
        assert len(got) == len(want)
        if len(want) == n:
            assert eos_row is None
            assert np.abs(h_dev - h).max() <= 2e-2 and rel_l2(h_dev, h) <= 1e-3, rel_l2(h_dev, h)
        print(f"[result] generate greedy {name} {prec}: {len(got)} frames x 16 codes identical", flush=True)
    else:
        # The trajectories part at frame `first`.  Re-run the device loop up to that frame
        # (it rewrites the same KV rows with the same values) to get the hidden state it
        # entered the frame with: it must be within the north-star bars of the reference's,
        # and the reference's own codec head + qwen_cp_predict evaluated on the device's
        # hidden state must give the device's 16 codes -- then every component agrees on
        # equal inputs and the parting is an argmax near-tie crossed by f32 rounding.
        _, _, h_in, _ = hip.generate(g, cp, head, embc, pad, h0, P, 0, first)
        if first == 0:
            h_in = h0
        r = rel_l2(h_in, hs[first])
        assert np.abs(h_in - hs[first]).max() <= 2e-2 and r <= 1e-3, (first, r)
        code0, _ = ref.codec_greedy(h_in, first)
        on_dev = [code0] + [int(c) for c in ref.cp_predict(h_in, code0)]
        assert on_dev == got[first], (first, on_dev, got[first], want[first])
        # and the first parting code was a near-tie on the reference's own trajectory
        k = next(i for i in range(16) if got[first][i] != want[first][i])
        gap = _code_margin(ref, s, cp, hs[first], first, want[first], got[first], k)
        assert gap <= 5e-3, (first, k, gap)
        print(f"[result] generate greedy {name} {prec}: frames 0..{first - 1} identical; frame {first} parts "
              f"({sum(a != b for a, b in zip(got[first], want[first]))} of 16 codes, first at code {k}, logit gap "
              f"{gap:.1e}) on hidden states {r:.1e} apart, and equals the reference's frame on the device's hidden "
              f"state", flush=True)
    cp.free()
    g.free()


@pytest.mark.parametrize("text_len,top_p", [(0, 1.0), (1, 0.9)])
def test_generate_sampled_matches_reference(oracle, text_len, top_p):
    """The reference's default sampling (temperature 0.9, top-k 50, repetition penalty 1.05
    over the code0 history), with the EOS boost for text_len (2 x 3 x text_len frames in,
    0.5 per frame): frames identical to the reference loop with the oracle sampler (pinned
    to the reference's qwen_tts_sample) until a draw lands within rounding of a cumulative
    boundary (the trajectories part there); at least the first 4 frames must agree, and
    where nothing parted the EOS frame, the frame count and the LCG state agree."""
    print(f"[case] generate sampled text_len={text_len} top_p={top_p}", flush=True)
    ref, s, g, cp, h0, pad, P = _setup("mini", "int8")
    n = 24
    head = np.ascontiguousarray(ref.codec_head())
    embc = np.ascontiguousarray(ref.codec_emb())
    prev0 = [7, 7, 300]
    codes, eos_row, _, seed_dev = hip.generate(g, cp, head, embc, pad, h0, P, 0, n, temp=0.9, top_k=50, top_p=top_p,
                                               rep=1.05, prev=prev0, seed=2024, text_len=text_len)
    seed, prev, h, same, parted, ref_n, ref_eos = 2024, list(prev0), h0, 0, False, 0, False
    start = 6 * text_len
    for f in range(n):
        _, lg = ref.codec_greedy(h, f)
        boost = float(min(np.float32(0.5) * np.float32(f - start), np.float32(10.0))) if text_len and f > start else 0.0
        code0, seed, dist = oracle.sample(lg, 0.9, 50, top_p, 1.05, prev, seed, rule=(f, boost))
        if code0 == 2150:
            ref_eos = True
            if not (len(codes) == f and eos_row is not None):      # EOS on the reference side only
                assert dist is not None and draw_margin(dist, seed) < 1e-4, (f, "EOS on one side only")
                parted = True
            break
        if f >= len(codes) or int(codes[f][0]) != code0:
            assert dist is not None and draw_margin(dist, seed) < 1e-4, (f, code0)
            parted = True
            break
        row = [code0] + [int(c) for c in ref.cp_predict(h, code0)]
        assert [int(c) for c in codes[f]] == row, f
        same += 1
        ref_n += 1
        prev.append(code0)
        h = ref.step(_next_input(ref, embc, row, pad))
    print(f"[result] generate sampled text_len={text_len}: {same} frames identical, device {len(codes)} frames"
          f"{' + EOS' if eos_row is not None else ''}, reference {ref_n}{' + EOS' if ref_eos else ''}", flush=True)
    assert same >= min(4, ref_n)
    if not parted:
        assert len(codes) == ref_n and (eos_row is not None) == ref_eos and seed_dev == seed
    if text_len:
        assert ref_eos or parted, "the EOS boost should end the utterance within the run"
    cp.free()
    g.free()


def test_generate_rejects_bad_arguments():
    ref, s, g, cp, h0, pad, P = _setup("mini", "bf16")
    head = np.ascontiguousarray(ref.codec_head())
    embc = np.ascontiguousarray(ref.codec_emb())
    with pytest.raises(RuntimeError):
        hip.generate(g, cp, head, embc, pad, h0, P, -1, 4)                 # frame0 < 0
    with pytest.raises(RuntimeError):
        hip.generate(g, cp, head, embc, pad, h0, 8190, 0, 40)              # past the largest cache (8192)
    codes, _, _, _ = hip.generate(g, cp, head, embc, pad, h0, P, 0, 2)     # the states stay usable
    assert len(codes) == 2
    cp.free()
    g.free()
