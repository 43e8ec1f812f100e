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

Generation (generate.py:1000-1260): ``generate_messages(messages,
max_new_tokens=16, sampling=None, *, stop=None, logprobs=None)``,
``generate_text`` and ``generate`` yield ``(text, None)`` chunks and a final
``("", stats)`` (triples with ``logprobs``), with the reference's sampling
(``runtime.sampling``), stop sequences and log probabilities
(``runtime.stopping``), UTF-8-safe streaming (``runtime.tokenizer``), prefix
reuse and statistics.  The uncached prompt tail runs as one batched prefill
on the GPU (logits only at its last position), where the reference steps it
position by position; a decoder without an engine (a test double) takes the
reference's per-position path.

Differences: every layer runs on the GPU (``npu_layers`` may be ``None`` or
the layer count; a CPU/NPU split has no GPU meaning and raises ValueError);
``context_length`` may be any size up to 65536 instead of exactly 64.  Greedy
steps without ``select``/``diagnostics`` take the argmax on the device and
copy only the token id back.
"""

import os
import resource
import time
from collections import OrderedDict
from pathlib import Path

import numpy as np

from runtime.qwen_engine import QwenDecoderEngine
from runtime.sampling import GREEDY, Sampler, SamplingParams
from runtime.stopping import StopMatcher, log_softmax, normalize_logprobs, normalize_stop
from runtime.tokenizer import StreamDetokenizer

__all__ = ["NPUDecoder", "default_system_prompt"]

QWEN2_SYSTEM = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant."
SMOLLM_SYSTEM = "You are a helpful AI assistant named SmolLM."


def default_system_prompt(model_family):
    """System turn the chat template adds when the messages carry none: Qwen's
    own for ``model_family == "qwen2"``, SmolLM's otherwise
    (npu_llm/runtime/generate.py:47-51)."""
    return QWEN2_SYSTEM if model_family == "qwen2" else SMOLLM_SYSTEM


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
        if isinstance(model_dir, (str, os.PathLike)) and (Path(model_dir) / "tokenizer.json").exists():
            from runtime.tokenizer import SmolLMTokenizer

            self.tokenizer = SmolLMTokenizer(model_dir, default_system=default_system_prompt(self.model_family))
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

    # -- generation (generate.py:1000-1260) -----------------------------------
    def _logprob_entry(self, logits, token_id, top_logprobs):
        """One emitted token in the OpenAI ``logprobs`` format, from the raw
        distribution (before penalties, temperature and filtering)."""
        lp = log_softmax(logits)

        def entry(i):
            i = int(i)
            return {"token": self.tokenizer.decode([i]), "logprob": float(lp[i]),
                    "bytes": list(self.tokenizer.token_bytes(i))}

        out = entry(token_id)
        top = []
        if top_logprobs:
            k = min(top_logprobs, lp.shape[0])
            best = np.argpartition(lp, -k)[-k:]
            top = [entry(i) for i in best[np.argsort(lp[best])[::-1]]]
        out["top_logprobs"] = top
        return out

    def _request(self, max_new_tokens, sampling, stop, logprobs):
        if not 0 < max_new_tokens < self.context_length:
            raise ValueError(f"max_new_tokens must be between 1 and {self.context_length - 1}")
        if sampling is None:
            params = GREEDY
        elif isinstance(sampling, SamplingParams):
            params = sampling
        else:
            params = SamplingParams.from_dict(sampling)
        stop_matcher = StopMatcher(normalize_stop(stop))
        top_logprobs = normalize_logprobs(logprobs)
        sampler = Sampler(params, vocab_size=self.model.metadata["vocab_size"])
        if getattr(self, "_profile_enabled", False):
            self._phase_totals = {}
        return sampler, stop_matcher, top_logprobs

    def generate_messages(self, messages, max_new_tokens=16, sampling=None, *, stop=None, logprobs=None):
        """Chat completion for OpenAI-style messages; the prompt is fitted into
        ``context_length - max_new_tokens`` tokens at turn boundaries."""
        sampler, stop_matcher, top_logprobs = self._request(max_new_tokens, sampling, stop, logprobs)
        prompt_ids, truncation = self.tokenizer.encode_chat_window(messages, self.context_length - max_new_tokens)
        yield from self._generate_tokens_core(prompt_ids, truncation, max_new_tokens, sampler, stop_matcher,
                                              top_logprobs)

    def generate_text(self, prompt, max_new_tokens=16, sampling=None, *, stop=None, logprobs=None):
        """Completion of a raw prompt (no ChatML turns)."""
        sampler, stop_matcher, top_logprobs = self._request(max_new_tokens, sampling, stop, logprobs)
        prompt_ids, truncated = self.tokenizer.encode_prompt_window(prompt, self.context_length - max_new_tokens)
        yield from self._generate_tokens_core(prompt_ids, {"truncated_prompt": truncated}, max_new_tokens,
                                              sampler, stop_matcher, top_logprobs)

    def generate(self, prompt, max_new_tokens=32, sampling=None, *, stop=None, logprobs=None):
        """A single user message (the reference's backward-compatible entry)."""
        yield from self.generate_messages([{"role": "user", "content": prompt}], max_new_tokens=max_new_tokens,
                                          sampling=sampling, stop=stop, logprobs=logprobs)

    def _prefill_tail(self, prompt_ids, reused, select):
        """Positions ``reused..`` of the prompt; returns ``(next_token,
        seconds per position)``.  The selector runs once, at the last
        position, since only that position's token is used."""
        last = len(prompt_ids) - 1
        if getattr(self, "_engine", None) is None:
            timings, token = [], None
            for i in range(reused, len(prompt_ids)):
                token, elapsed = self._decode_step(prompt_ids[i], i, select=select if i == last else None,
                                                   compute_logits=i == last)
                timings.append(elapsed)
            return token, timings
        del self._cached_prefix[reused:]
        start = time.perf_counter()
        token, logits = self._engine.prefill(prompt_ids[reused:], start=reused, logits=True,
                                             want_logits_array=select is not None)
        if select is not None:
            token = int(select(np.asarray(logits, dtype=np.float32)))
        self._record_phase("gpu_engine", start)
        self._cached_prefix = [int(t) for t in prompt_ids]
        elapsed = time.perf_counter() - start
        n = len(prompt_ids) - reused
        return token, [elapsed / n] * n

    def _generate_tokens_core(self, prompt_ids, truncation, max_new_tokens, sampler, stop_matcher, top_logprobs):
        """The decode loop of generate.py:1050-1200 (see the module docstring)."""
        history = list(prompt_ids)  # penalties see the prompt too
        # log-probability entries wait, keyed by the byte offset where their
        # token starts in the generated text, until that text is emitted;
        # entries of text a stop sequence discards are never reported
        pending = []
        chosen_entry = None
        bytes_generated = 0
        bytes_emitted = 0

        def choose(logits):
            nonlocal chosen_entry
            token = int(np.argmax(logits)) if sampler.greedy else sampler.select(logits, history)
            if top_logprobs is not None:
                chosen_entry = self._logprob_entry(logits, token, top_logprobs)
            return token

        select = None if (sampler.greedy and top_logprobs is None) else choose

        def take_entries(text, final=False):
            nonlocal bytes_emitted
            bytes_emitted += len(text.encode("utf-8"))
            if final and stop_matcher.matched is None:
                n = len(pending)
            else:
                n = 0
                while n < len(pending) and pending[n][0] < bytes_emitted:
                    n += 1
            out = [e for _, e in pending[:n]]
            del pending[:n]
            return out

        def chunk(text, entries):
            return (text, None) if top_logprobs is None else (text, None, entries)

        reused = self._reusable_prefix(prompt_ids)
        next_token, timings = self._prefill_tail(prompt_ids, reused, select)
        prefill_steps = len(timings)
        position = len(prompt_ids)
        detok = StreamDetokenizer(self.tokenizer)
        generated = []
        finish_reason = "length"
        text = ""
        while len(generated) < max_new_tokens:
            entry, chosen_entry = chosen_entry, None
            if next_token == self.tokenizer.eos_id:  # not part of the content, nor its log probability
                finish_reason = "stop"
                break
            generated.append(next_token)
            history.append(next_token)
            if entry is not None:
                pending.append((bytes_generated, entry))
                bytes_generated += len(self.tokenizer.token_bytes(next_token))
            text = stop_matcher.feed(detok.push(next_token))
            if stop_matcher.matched is not None:
                finish_reason = "stop"
                break
            if text:
                yield chunk(text, take_entries(text))
            if len(generated) >= max_new_tokens:  # no step for a token that would be discarded
                break
            next_token, elapsed = self._decode_step(next_token, position, select=select)
            timings.append(elapsed)
            position += 1
        if stop_matcher.matched is None:
            text = stop_matcher.feed(detok.flush())
            if stop_matcher.matched is not None:
                finish_reason = "stop"
            text += stop_matcher.flush()
        entries = take_entries(text, final=True) if top_logprobs is not None else []
        if text or entries:
            yield chunk(text, entries)
        prefill_seconds = sum(timings[:prefill_steps])
        decode_seconds = sum(timings[prefill_steps:])
        decode_steps = len(timings) - prefill_steps
        stats = {
            "prompt_tokens": len(prompt_ids),
            "cached_prompt_tokens": reused,
            "prompt_truncation": truncation,
            "generated_tokens": len(generated),
            "generated_token_ids": generated,
            "npu_layers": self.npu_layers,
            "cpu_layers": self.layers - self.npu_layers,
            "finish_reason": finish_reason,
            "stop_sequence": stop_matcher.matched,
            "ttft_seconds": prefill_seconds,
            "prefill_tokens_per_second": prefill_steps / max(1e-9, prefill_seconds),
            "decode_steps": decode_steps,
            "decode_seconds": decode_seconds,
            "decode_tokens_per_second": decode_steps / max(1e-9, decode_seconds),
            "peak_ram_mib": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1024,
            "sampling": sampler.stats(),
        }
        if getattr(self, "_profile_enabled", False):
            stats["phase_ms"] = {k: round(v * 1000.0, 3) for k, v in self._phase_totals.items()}
        yield ("", stats) if top_logprobs is None else ("", stats, [])

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
