"""The speech decoder's float64 oracle (oracle/sd_oracle.py) pinned against the reference's
own compiled one-shot decode (qwen_speech_decoder_decode, qwen_tts_speech_decoder.c:579-1290,
built by oracle/Makefile without BLAS, so it sums in its naive loop order in f32)."""
import numpy as np

from conftest import need_ref, rel_l2, sd_codes, sd_model


@need_ref
def test_sd_oracle_matches_compiled_reference():
    """Three frames, including out-of-range codes: the f64 restatement and the reference's
    f32 decode agree to the reference's own f32 rounding (measured 6e-6)."""
    from oracle import sd_oracle
    from oracle.oracle import RefSpeechDecoder
    path, t = sd_model()
    codes = sd_codes(3, 11)
    ref = RefSpeechDecoder(path, threads=8).decode(codes)
    st = {}
    orc = sd_oracle.decode(t, codes, st)
    assert ref.shape == orc.shape == (3 * 1920,)
    assert np.abs(ref - orc).max() <= 1e-4 and rel_l2(ref, orc) <= 1e-4, (np.abs(ref - orc).max(), rel_l2(ref, orc))
    assert st["latent"].shape == (3, 1024) and st["convnext"].shape == (12, 1024)
