"""Host side of the hk decode engine for MI355X.

Mirrors the reference's ``npu_llm/runtime`` package so callers that put this
directory's parent on ``sys.path`` and import ``runtime.generate`` /
``runtime.qwen_engine`` / ``runtime.engine`` keep working:

- ``runtime.hip``          ctypes binding of ``libhk.so`` (C ABI in include/hk.h)
- ``runtime.qwen_engine``  ``QwenDecoderEngine``: every layer + head per step
- ``runtime.engine``       ``DecoderEngine``: layers + final norm (SmolLM form)
- ``runtime.generate``     ``NPUDecoder``: the step API used by servers and chat
- ``runtime.synthetic``    seeded random-init models of the benchmark shapes
- ``runtime.bf16``         host-side bfloat16 bit conversions
"""
