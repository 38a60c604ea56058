"""MI355X (gfx950) Talker / Code-Predictor decode-step library for Qwen3-TTS.

The product is the C-ABI shared library ``libqwen_tts_hip.so`` in this directory, built
from ``csrc/`` (declared in ``include/qwen_tts_hip.h``); ``glue/`` holds the reference-side
C glue.  The Python modules here are thin helpers around it:
``hip`` (ctypes binding of the C-ABI), ``build`` (compiles the library with hipcc)
and ``synth`` (seeded random-init weights in the reference layout).
"""
