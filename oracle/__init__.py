"""CPU oracle for the whole-model decode step.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the package under
``hawkpoint-npu-llm_amd/``) imports this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, and only as the checker or as the timed CPU baseline, never as the thing
measured or shipped.

The oracle is a NumPy restatement of the reference's NumPy BF16 CPU runtime
(``npu_llm/runtime/cpu_backend.py``) and of the host arithmetic around it in
``npu_llm/runtime/generate.py`` and ``npu_llm/tools/convert_smollm2.py``.
The reference module imports ``ml_dtypes``, which this image lacks, so the
BF16 cast is restated with integer arithmetic in :mod:`oracle.bf16`.

Modules
-------
bf16         float32 <-> bfloat16 round-to-nearest-even on uint16 bit patterns.
cpu_backend  ``CPUDecoderStage`` (per-layer decode arithmetic), the step loop of
             ``NPUDecoder.decode_token`` with ``npu_layers=0`` and its argmax.
quant        the per-output-row int8 quantiser and the W8 projection formula.
moe          the routed-expert block (router, top-k, experts, combine).
experts      the GGML MUL_MAT_ID and Colibri expert-group offload contracts
             (upload formats, W8 requantisation, 2048-column tiles, SwiGLU).

Pinning status of each function is recorded in its docstring and checked by
``tests/test_oracle_*.py``.
"""
