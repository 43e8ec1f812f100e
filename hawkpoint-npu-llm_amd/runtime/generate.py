"""``NPUDecoder``: the reference's decode-step API, backed by the hk engine.

Callers written against ``npu_llm/runtime/generate.py`` (the OpenAI server's
worker, the terminal chat, the token gates) construct ``NPUDecoder(model_dir,
npu_layers=...)`` and call ``decode_token``, ``warmup``,
``reset_prefix_cache`` and ``close``.  Those keep their signatures, return
values and errors (generate.py:41-47, 709-973, 1258-1316):

- ``decode_token(token_id, position, *, diagnostics=False, select=None,
  compute_logits=True)`` -> ``(next_token, elapsed_seconds[, diag])``, or
  ``(None, elapsed)`` with ``compute_logits=False``; ``ValueError`` when
  ``position`` is outside the context;
- the prefix bookkeeping (``_cached_prefix``, ``_reusable_prefix``,
  ``_decode_step``) and ``HAWKPOINT_PREFIX_CACHE=0``;
- ``close()`` is idempotent.

Differences: every layer runs on the GPU (``npu_layers`` may be ``None`` or
the layer count; a CPU/NPU split has no GPU meaning and raises ValueError);
``context_length`` may be any size up to 65536 instead of exactly 64.  Greedy
steps without ``select``/``diagnostics`` take the argmax on the device and
copy only the token id back.
"""

import os
import time
from collections import OrderedDict

import numpy as np

from runtime.qwen_engine import QwenDecoderEngine

__all__ = ["NPUDecoder"]


def _load_model(model):
    if isinstance(model, (str, os.PathLike)):
        from runtime.model import XDNA1Model

        return XDNA1Model(model)
    return model


class NPUDecoder:
    def __init__(self, model_dir, context_length=64, npu_layers=None, *, w8=None, device=0):
        if not 0 < int(context_length) <= 65536:
            raise ValueError("context_length must be between 1 and 65536")
        self._closed = False
        self.model = _load_model(model_dir)
        meta = self.model.metadata
        self.model_family = meta.get("model_family", "llama")
        self.context_length = int(context_length)
        self.hidden_size = meta["hidden_size"]
        self.intermediate_size = meta["intermediate_size"]
        self.q_heads = meta["attention_heads"]
        self.kv_heads = meta["kv_heads"]
        self.head_dim = meta["head_dim"]
        self.q_per_kv = self.q_heads // self.kv_heads
        self.layers = meta["layers"]
        self.rms_norm_eps = float(meta.get("rms_norm_eps", 1e-5))
        self.npu_layers = self.layers if npu_layers is None else int(npu_layers)
        if not 0 <= self.npu_layers <= self.layers:
            raise ValueError(f"npu_layers must be between 0 and {self.layers}")
        if self.npu_layers != self.layers:
            raise ValueError("the GPU engine runs every layer; npu_layers must be None or the layer count")
        if w8 is None:
            w8 = os.environ.get("HAWKPOINT_DECODER_W8") == "1"
        self._cached_prefix = []
        self._prefix_cache_enabled = os.environ.get("HAWKPOINT_PREFIX_CACHE", "1") != "0"
        self._profile_enabled = os.environ.get("HAWKPOINT_PROFILE") == "1"
        self._phase_totals = {}
        self._engine = QwenDecoderEngine(self.model, context_length=self.context_length, w8=bool(w8),
                                         device=device)
        self.tokenizer = None
        self._qwen_embedding_cache = OrderedDict()

    # -- step ------------------------------------------------------------------
    def _record_phase(self, name, start):
        if self._profile_enabled:
            self._phase_totals[name] = self._phase_totals.get(name, 0.0) + time.perf_counter() - start

    @staticmethod
    def _decode_result(logits, start, diagnostics, select=None):
        """argmax or ``select`` plus optional top-5 diagnostics (generate.py:709-730)."""
        logits_f32 = np.asarray(logits, dtype=np.float32)
        next_token = int(np.argmax(logits_f32)) if select is None else int(select(logits_f32))
        elapsed = time.perf_counter() - start
        if not diagnostics:
            return next_token, elapsed
        top = np.argpartition(logits_f32, -5)[-5:]
        top = top[np.argsort(logits_f32[top])[::-1]]
        return next_token, elapsed, {
            "top_token_ids": [int(i) for i in top],
            "top_logits": [float(logits_f32[i]) for i in top],
            "top_logit_margin": float(logits_f32[top[0]] - logits_f32[top[1]]),
        }

    def decode_token(self, token_id, position, *, diagnostics=False, select=None, compute_logits=True):
        """Run one decode step and return ``(next_token, elapsed_seconds)``
        (see the module docstring for the full contract)."""
        if not 0 <= position < self.context_length:
            raise ValueError(f"position outside the {self.context_length}-token context")
        del self._cached_prefix[position:]
        start = time.perf_counter()
        if self._engine is None:
            raise RuntimeError("decoder is closed")
        if not compute_logits:
            self._engine.step_token(token_id, position, logits=False)
            self._record_phase("gpu_engine", start)
            return None, time.perf_counter() - start
        if select is None and not diagnostics:
            token, _ = self._engine.step_token(token_id, position, logits=True, want_logits_array=False)
            self._record_phase("gpu_engine", start)
            return token, time.perf_counter() - start
        _, logits = self._engine.step_token(token_id, position, logits=True)
        self._record_phase("gpu_engine", start)
        return self._decode_result(logits, start, diagnostics, select)

    def logits(self, token_id, position):
        """float32 logits of one step (for gates that compare logits)."""
        if not 0 <= position < self.context_length:
            raise ValueError(f"position outside the {self.context_length}-token context")
        del self._cached_prefix[position:]
        _, logits = self._engine.step_token(token_id, position, logits=True)
        return logits

    def warmup(self):
        """Capture the step graphs, then forget the warm-up position."""
        eos = 0
        if self.tokenizer is not None and getattr(self.tokenizer, "eos_id", None) is not None:
            eos = int(self.tokenizer.eos_id)
        self.decode_token(eos, 0, compute_logits=False)
        self.decode_token(eos, 0)
        self._engine.reset()
        self._cached_prefix.clear()

    def reset_prefix_cache(self):
        self._cached_prefix.clear()

    def _reusable_prefix(self, prompt_ids):
        """Leading prompt positions reusable from the cache; the final prompt
        position is always recomputed (generate.py:952-965)."""
        if not self._prefix_cache_enabled:
            return 0
        shared = 0
        for cached, token in zip(self._cached_prefix, prompt_ids):
            if cached != token:
                break
            shared += 1
        return min(shared, len(prompt_ids) - 1)

    def _decode_step(self, token_id, position, **kwargs):
        del self._cached_prefix[position:]
        result = self.decode_token(token_id, position, **kwargs)
        if len(self._cached_prefix) == position:
            self._cached_prefix.append(int(token_id))
        return result

    def generate_ids(self, prompt_ids, max_new_tokens):
        """Greedy generation from token ids with prefix reuse: batched prefill
        of the uncached prompt tail (logits only at the last prompt position),
        then the engine's device-driven greedy loop.  Returns ``(token_ids, stats)`` with the
        reference's TTFT / decode-rate definitions (generate.py:1110-1188)."""
        if not prompt_ids:
            raise ValueError("prompt must not be empty")
        if len(prompt_ids) + max_new_tokens - 1 > self.context_length:
            raise ValueError("prompt plus generated tokens exceed the context")
        reused = self._reusable_prefix(prompt_ids)
        t0 = time.perf_counter()
        # the un-cached prompt tail in one batched pass (logits at its end only)
        del self._cached_prefix[reused:]
        first, _ = self._engine.prefill(prompt_ids[reused:], start=reused, logits=True,
                                        want_logits_array=False)
        self._cached_prefix = [int(t) for t in prompt_ids]
        ttft = time.perf_counter() - t0
        tokens = [first]
        t1 = time.perf_counter()
        if max_new_tokens > 1:
            tokens += self._engine.generate(first, len(prompt_ids), max_new_tokens - 1)
            self._cached_prefix = list(prompt_ids) + tokens[:-1]
        decode_seconds = time.perf_counter() - t1
        steps = max_new_tokens - 1
        return tokens, {
            "prompt_tokens": len(prompt_ids),
            "cached_prompt_tokens": reused,
            "ttft_seconds": ttft,
            "decode_steps": steps,
            "decode_seconds": decode_seconds,
            "decode_tokens_per_second": steps / max(1e-9, decode_seconds),
        }

    def close(self):
        """Release the engine and its device memory; idempotent."""
        if getattr(self, "_closed", False):
            return
        self._closed = True
        self._cached_prefix = []
        engine = getattr(self, "_engine", None)
        if engine is not None:
            engine.close()
        self._engine = None
