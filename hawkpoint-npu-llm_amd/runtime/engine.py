"""``DecoderEngine``: the reference's SmolLM engine interface on the hk engine.

``npu_llm/runtime/engine.py:29-91`` runs every decoder layer plus the final
RMSNorm for one token and returns the normalised hidden state (bf16); the
LM head then runs on the host.  Here the same call runs the layers on the GPU
and returns the final-RMSNorm output; ``QwenDecoderEngine`` is the variant
that also runs the LM head and argmax on the device.
"""

import numpy as np

from runtime.qwen_engine import QwenDecoderEngine, supports

__all__ = ["DecoderEngine", "supports"]


class DecoderEngine:
    def __init__(self, model, rope_inv_freq=None, *, context_length=64, device=0):
        meta = model.metadata
        if rope_inv_freq is not None:
            half = int(meta["head_dim"]) // 2
            theta = float(meta.get("rope_theta", 10000.0))
            own = 1.0 / (theta ** (np.arange(half, dtype=np.float32) / np.float32(half)))
            if not np.array_equal(np.asarray(rope_inv_freq, np.float32), own):
                raise ValueError("rope_inv_freq does not match the model's rope_theta")
        self._engine = QwenDecoderEngine(model, context_length=context_length, device=device)
        self.layers = self._engine.layers

    def reset(self):
        """Forget every cached position (a new sequence starts at 0)."""
        self._engine.reset()

    def step(self, embedding, position):
        """Run every layer for one token; return the final-RMSNorm output as
        bf16 bits [H].  Attention reads slots 0..position."""
        self._engine.step(embedding, position, logits=False)
        return self._engine.final_hidden()

    def close(self):
        if self._engine is not None:
            self._engine.close()
            self._engine = None
