"""NumPy restatement of the reference's BF16 CPU decode step (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, smoke() and bench's CPU baseline.

Follows ``npu_llm/runtime/cpu_backend.py`` operation by operation:

===============================  =========================================
reference (file:line)            here
===============================  =========================================
cpu_backend.py:7-8   ``_bf16``   ``oracle.bf16.round_f32`` / ``to_bits``
cpu_backend.py:26-32 inv-freq    ``CPUDecoderStage.__init__``
cpu_backend.py:37-50 KV caches   ``CPUDecoderStage.__init__`` (uint16 bits)
cpu_backend.py:64-69 ``project``  ``CPUDecoderStage.project``
cpu_backend.py:71-76 ``norm``     ``CPUDecoderStage.norm``
cpu_backend.py:78-93 ``_rotate``  ``CPUDecoderStage.rotate``
cpu_backend.py:95-129 attention  ``CPUDecoderStage.attention``
cpu_backend.py:131-171 ``layer``  ``CPUDecoderStage.layer``
cpu_backend.py:173-181 logits    ``CPUDecoderStage.logits``
generate.py:215-223, 832 embed   ``OracleDecoder.decode_token``
generate.py:709-730 argmax       ``decode_result``
generate.py:830-846 CPU step     ``OracleDecoder.decode_token``
generate.py:1110-1158 loop       ``OracleDecoder.generate_greedy``
generate.py:1110-1125 prefill    ``OracleDecoder.prefill`` (rows at once)
validate_engine_npu.py:58-64     ``OracleDecoder.teacher_forced`` (rows at once)
===============================  =========================================

BF16 tensors are carried as uint16 bit patterns because ``ml_dtypes`` is not
available; every place the reference holds a ``bfloat16`` array this module
holds its bits and widens them exactly with :func:`oracle.bf16.from_bits`.
All arithmetic is float32 NumPy, with the same rounding points as the
reference.  Python-float constants (eps, clip bounds, the attention scale)
combine with float32 arrays as float32, as under NumPy 2's promotion rules.

W8 mode (``w8=True``) replaces the four layer projections with the reference's
int8 device formula ``bf16((sum_k f32(q) * f32(x)) * scale[row])``
(``kernels/project_w8bf16.cc:14-38``, ``kernels/decoder_layer_bf16.cc:64-98``);
the LM head stays BF16.

Model interface expected from ``model``: ``metadata`` (the package's
metadata dict), ``tensors`` (name -> spec), ``raw_f32(name)`` (float32 copy of
a raw tensor), ``bf16_projection(name)`` (uint16 bits, shape [M, K]) and, for
W8, ``quantized(name)`` with ``.weight`` (int8 [M, K]) and ``.scale``
(float32 [M]).

Pinning: see ``tests/test_oracle_cpu_backend.py`` -- the attention is checked
against the reference test's per-head loop (``tests/test_cpu_backend.py:17-52``),
projections against float64 brute force with a forward error bound, norm /
RoPE / SwiGLU / residual against closed forms, and argmax against its
first-maximum invariant.  The exact NumPy reduction orders of BLAS ``sgemv``,
``np.mean`` and ``np.einsum`` are those of this image's NumPy, not the
reference's pinned 2.5.4: parity with the reference at that level is unpinned
and absorbed by the rel-L2 <= 1e-2 / near-tie tolerance.
"""

import time

import numpy as np

from oracle.bf16 import from_bits, round_f32, to_bits
from oracle.quant import project_w8

__all__ = ["CPUDecoderStage", "OracleDecoder", "decode_result", "rope_inv_frequency"]


def rope_inv_frequency(theta, head_dim):
    """``1 / theta ** (arange(half) / half)`` in float32 (cpu_backend.py:26-32)."""
    half = head_dim // 2
    return 1.0 / (float(theta) ** (np.arange(half, dtype=np.float32) / np.float32(half)))


class CPUDecoderStage:
    """Decoder layers ``first_layer..layers-1`` and their BF16 KV caches."""

    def __init__(self, model, first_layer, context_length, *, w8=False):
        meta = model.metadata
        self.model = model
        self.metadata = meta
        self.first_layer = first_layer
        self.context_length = context_length
        self.w8 = bool(w8)
        self.hidden_size = meta["hidden_size"]
        self.intermediate_size = meta["intermediate_size"]
        self.q_heads = meta["attention_heads"]
        self.kv_heads = meta["kv_heads"]
        self.head_dim = meta["head_dim"]
        self.q_per_kv = self.q_heads // self.kv_heads
        self.rope_theta = float(meta.get("rope_theta", 10000.0))
        self._rope_inv_frequency = rope_inv_frequency(self.rope_theta, self.head_dim)
        self.epsilon = float(meta.get("rms_norm_eps", 1e-5))
        self._weights = {}
        self._quant = {}
        self._raw = {}
        self._lm_head_f32 = None
        shape = (self.kv_heads, context_length, self.head_dim)
        layers = range(first_layer, meta["layers"])
        self.key_cache = {layer: np.zeros(shape, dtype=np.uint16) for layer in layers}
        self.value_cache = {layer: np.zeros(shape, dtype=np.uint16) for layer in layers}

    # -- tensors -----------------------------------------------------------
    def raw(self, name):
        if name not in self._raw:
            self._raw[name] = np.asarray(self.model.raw_f32(name), dtype=np.float32)
        return self._raw[name]

    def weight(self, name):
        """BF16 projection bits; widened to float32 on every use, as the
        reference widens its memmap on every ``project`` call."""
        if name not in self._weights:
            self._weights[name] = self.model.bf16_projection(name)
        return self._weights[name]

    # -- ops ---------------------------------------------------------------
    def project(self, name, activation):
        """``bf16(W_f32 @ f32(bf16(x)))`` or, in W8 mode for layer weights,
        ``bf16((f32(q) @ f32(bf16(x))) * scale)``."""
        if self.w8 and name != "lm_head":
            q = self.quantized(name)
            return project_w8(q.weight, q.scale, activation)
        return round_f32(from_bits(self.weight(name)) @ round_f32(activation))

    def quantized(self, name):
        if name not in self._quant:
            self._quant[name] = self.model.quantized(name)
        return self._quant[name]

    def project_rows(self, name, rows):
        """``project`` applied to every row of ``rows`` [n, K] at once: one
        matrix product instead of n matrix-vector products, so only the
        float32 summation order differs from calling ``project`` per row."""
        x = round_f32(rows)
        if self.w8 and name != "lm_head":
            q = self.quantized(name)
            acc = x @ np.asarray(q.weight, dtype=np.float32).T
            return round_f32(acc * np.asarray(q.scale, dtype=np.float32))
        return round_f32(x @ from_bits(self.weight(name)).T)

    def norm(self, activation, gamma_name):
        """``bf16((v * inv) * gamma)`` with ``inv = 1/sqrt(mean(v*v) + eps)``."""
        value = round_f32(activation)
        inverse_rms = 1.0 / np.sqrt(np.mean(value * value, dtype=np.float32) + self.epsilon)
        return round_f32(value * inverse_rms * self.raw(gamma_name))

    def norm_rows(self, rows, gamma_name):
        """``norm`` of every row of ``rows`` [n, H]."""
        value = round_f32(rows)
        mean = np.mean(value * value, axis=-1, dtype=np.float32, keepdims=True)
        inverse_rms = 1.0 / np.sqrt(mean + self.epsilon)
        return round_f32(value * inverse_rms * self.raw(gamma_name))

    def rope_tables(self, position):
        angle = np.float32(position) * self._rope_inv_frequency
        return np.cos(angle), np.sin(angle)

    def rotate(self, heads, position):
        """Split-half rotation ``[x1 c - x2 s, x2 c + x1 s]``, then bf16."""
        heads = np.asarray(heads, dtype=np.float32)
        half = self.head_dim // 2
        cosine, sine = self.rope_tables(position)
        first, second = heads[..., :half], heads[..., half:]
        rotated = np.concatenate(
            [first * cosine - second * sine, second * cosine + first * sine], axis=-1
        )
        return round_f32(rotated)

    def attention(self, qkv, layer, position):
        """RoPE, KV append at slot ``position``, GQA softmax attention, bf16."""
        d = self.head_dim
        nq = self.q_heads * d
        nkv = self.kv_heads * d
        qkv = np.asarray(qkv, dtype=np.float32)
        query = self.rotate(qkv[:nq].reshape(self.q_heads, d), position)
        key = self.rotate(qkv[nq:nq + nkv].reshape(self.kv_heads, d), position)
        value = qkv[nq + nkv:].reshape(self.kv_heads, d)
        self.key_cache[layer][:, position] = to_bits(key)
        self.value_cache[layer][:, position] = to_bits(value)
        keys = from_bits(self.key_cache[layer][:, : position + 1])
        values = from_bits(self.value_cache[layer][:, : position + 1])
        grouped = query.reshape(self.kv_heads, self.q_per_kv, d)
        scores = np.einsum("kqd,ksd->kqs", grouped, keys, optimize=True) * d**-0.5
        scores -= np.max(scores, axis=-1, keepdims=True)
        probabilities = np.exp(scores)
        probabilities /= np.sum(probabilities, axis=-1, keepdims=True)
        out = np.einsum("kqs,ksd->kqd", probabilities, values, optimize=True)
        return round_f32(out.reshape(-1))

    # prompts of at least this many rows score their attention with batched
    # BLAS matrix products instead of ``attention``'s einsum (minutes instead
    # of hours for 4096-token prompts at full depth); only the float32
    # summation order differs
    BLAS_ROWS = 256

    def attention_rows(self, qkv_rows, layer, start, block=256):
        """``attention`` for rows at positions start..start+n-1 at once: every
        row's RoPE and KV append first, then each row attends to slots
        0..its position (causal), as n calls of ``attention`` in order would.
        Rows are scored in blocks of ``block`` to bound the score matrix.
        Below ``BLAS_ROWS`` rows the products are ``attention``'s own einsum
        contractions, which sum each output in the order the per-position
        calls do (the two agree bit for bit); from ``BLAS_ROWS`` rows they are
        batched matrix products."""
        d = self.head_dim
        nq = self.q_heads * d
        nkv = self.kv_heads * d
        qkv_rows = np.asarray(qkv_rows, dtype=np.float32)
        n = qkv_rows.shape[0]
        positions = np.arange(start, start + n)
        half = d // 2
        angle = positions.astype(np.float32)[:, None] * self._rope_inv_frequency[None, :]
        cosine, sine = np.cos(angle)[:, None, :], np.sin(angle)[:, None, :]

        def rotate_rows(heads):
            first, second = heads[..., :half], heads[..., half:]
            return round_f32(np.concatenate(
                [first * cosine - second * sine, second * cosine + first * sine], axis=-1))

        query = rotate_rows(qkv_rows[:, :nq].reshape(n, self.q_heads, d))
        key = rotate_rows(qkv_rows[:, nq:nq + nkv].reshape(n, self.kv_heads, d))
        value = qkv_rows[:, nq + nkv:].reshape(n, self.kv_heads, d)
        self.key_cache[layer][:, start:start + n] = to_bits(key).transpose(1, 0, 2)
        self.value_cache[layer][:, start:start + n] = to_bits(value).transpose(1, 0, 2)
        end = start + n
        keys = from_bits(self.key_cache[layer][:, :end])      # [kvh, end, d]
        values = from_bits(self.value_cache[layer][:, :end])
        out = np.empty((n, self.q_heads, d), dtype=np.float32)
        grouped = query.reshape(n, self.kv_heads, self.q_per_kv, d)
        slots = np.arange(end)
        blas = n >= self.BLAS_ROWS
        keys_t = np.ascontiguousarray(keys.transpose(0, 2, 1)) if blas else None  # [kvh, d, end]
        for r0 in range(0, n, block):
            r1 = min(n, r0 + block)
            rows = r1 - r0
            q = grouped[r0:r1].transpose(1, 0, 2, 3)          # [kvh, rows, qpk, d]
            if blas:  # [kvh, rows * qpk, d] @ [kvh, d, end]
                q = np.ascontiguousarray(q).reshape(self.kv_heads, -1, d)
                scores = (np.matmul(q, keys_t) * d**-0.5).reshape(self.kv_heads, rows, self.q_per_kv, end)
            else:
                scores = np.einsum("krqd,ksd->krqs", q, keys, optimize=True) * d**-0.5
            future = slots[None, :] > positions[r0:r1, None]  # [rows, end]
            scores += np.where(future, -np.inf, 0.0).astype(np.float32)[None, :, None, :]
            scores -= np.max(scores, axis=-1, keepdims=True)
            probabilities = np.exp(scores)
            probabilities /= np.sum(probabilities, axis=-1, keepdims=True)
            if blas:
                o = np.matmul(probabilities.reshape(self.kv_heads, -1, end), values).reshape(
                    self.kv_heads, rows, self.q_per_kv, d)
            else:
                o = np.einsum("krqs,ksd->krqd", probabilities, values, optimize=True)
            out[r0:r1] = o.transpose(1, 0, 2, 3).reshape(rows, self.q_heads, d)
        return round_f32(out.reshape(n, -1))

    def layer_rows(self, hidden_rows, layer, start):
        """``layer`` for rows at positions start..start+n-1 at once."""
        p = f"layer{layer:02d}"
        hidden_rows = np.asarray(hidden_rows, dtype=np.float32)
        normalized = self.norm_rows(hidden_rows, f"{p}.input_norm")
        bias_name = f"{p}.qkv_bias"
        bias = self.raw(bias_name) if bias_name in self.model.tensors else 0.0
        qkv = round_f32(self.project_rows(f"{p}.qkv", normalized) + bias)
        attended = self.attention_rows(qkv, layer, start)
        after_attention = round_f32(self.project_rows(f"{p}.o_proj", attended) + hidden_rows)
        post = self.norm_rows(after_attention, f"{p}.post_attn_norm")
        gate_up = self.project_rows(f"{p}.gate_up", post)
        gate, up = np.split(gate_up, 2, axis=-1)
        activation = round_f32((gate / (1.0 + np.exp(-np.clip(gate, -80.0, 80.0)))) * up)
        return round_f32(self.project_rows(f"{p}.down_proj", activation) + after_attention)

    def layer(self, hidden, layer, position):
        p = f"layer{layer:02d}"
        normalized = self.norm(hidden, f"{p}.input_norm")
        bias_name = f"{p}.qkv_bias"
        bias = self.raw(bias_name) if bias_name in self.model.tensors else 0.0
        qkv = round_f32(self.project(f"{p}.qkv", normalized) + bias)
        attended = self.attention(qkv, layer, position)
        after_attention = round_f32(
            self.project(f"{p}.o_proj", attended) + np.asarray(hidden, np.float32)
        )
        post = self.norm(after_attention, f"{p}.post_attn_norm")
        gate_up = self.project(f"{p}.gate_up", post)
        gate, up = np.split(gate_up, 2)
        activation = round_f32((gate / (1.0 + np.exp(-np.clip(gate, -80.0, 80.0)))) * up)
        return round_f32(self.project(f"{p}.down_proj", activation) + after_attention)

    def logits(self, hidden):
        """FP32 logits ``W_lm_f32 @ f32(bf16(norm(h)))`` -- not rounded."""
        normalized = self.norm(hidden, "final_norm")
        if self._lm_head_f32 is None:
            self._lm_head_f32 = from_bits(self.weight("lm_head"))
        return self._lm_head_f32 @ round_f32(normalized)

    def logits_rows(self, hidden_rows):
        """``logits`` of every row of ``hidden_rows`` [n, H] as one product;
        returns [n, vocab]."""
        normalized = self.norm_rows(hidden_rows, "final_norm")
        if self._lm_head_f32 is None:
            self._lm_head_f32 = from_bits(self.weight("lm_head"))
        return (self._lm_head_f32 @ normalized.T).T

    def reset(self):
        for cache in self.key_cache.values():
            cache.fill(0)
        for cache in self.value_cache.values():
            cache.fill(0)


def decode_result(logits, diagnostics=False):
    """``np.argmax`` (first maximum wins) plus optional top-5 diagnostics
    (generate.py:709-730)."""
    logits = np.asarray(logits, dtype=np.float32)
    token = int(np.argmax(logits))
    if not diagnostics:
        return token
    top = np.argpartition(logits, -5)[-5:]
    top = top[np.argsort(logits[top])[::-1]]
    return token, {
        "top_token_ids": [int(i) for i in top],
        "top_logits": [float(logits[i]) for i in top],
        "top_logit_margin": float(logits[top[0]] - logits[top[1]]),
    }


class OracleDecoder:
    """The reference's CPU path (``NPUDecoder`` with ``npu_layers=0``).

    ``decode_token`` follows generate.py:830-846: ``bf16(E_f32[token])``,
    every layer on the CPU, then logits and argmax only when requested.
    """

    def __init__(self, model, context_length, *, w8=False):
        self.model = model
        self.layers = model.metadata["layers"]
        self.context_length = context_length
        self.stage = CPUDecoderStage(model, 0, context_length, w8=w8)
        self._embedding = model.raw_f32("token_embedding").reshape(
            model.metadata["vocab_size"], model.metadata["hidden_size"]
        )

    def hidden_after_layers(self, token_id, position):
        hidden = round_f32(self._embedding[token_id])
        for layer in range(self.layers):
            hidden = self.stage.layer(hidden, layer, position)
        return hidden

    def decode_token(self, token_id, position, compute_logits=True):
        """Return ``(next_token or None, logits or None)``."""
        if not 0 <= position < self.context_length:
            raise ValueError("position outside the context")
        hidden = self.hidden_after_layers(token_id, position)
        if not compute_logits:
            return None, None
        logits = self.stage.logits(hidden)
        return decode_result(logits), logits

    def prefill(self, prompt_ids, start=0, compute_logits=True, progress=None):
        """Every prompt token at slots start..start+n-1 with logits at the last
        one, like ``decode_token`` position by position (generate.py:1110-1125)
        but with each layer applied to all rows at once (matrix products and
        causal attention); only float32 summation orders differ.  Returns
        ``(next_token, logits)`` or ``(None, None)``.  ``progress(layer)``, if
        given, is called after each layer (long prompts take minutes)."""
        ids = [int(t) for t in prompt_ids]
        if not ids:
            raise ValueError("prefill needs at least one token")
        if start < 0 or start + len(ids) > self.context_length:
            raise ValueError("position outside the context")
        hidden = round_f32(self._embedding[np.asarray(ids)])
        for layer in range(self.layers):
            hidden = self.stage.layer_rows(hidden, layer, start)
            if progress is not None:
                progress(layer)
        if not compute_logits:
            return None, None
        logits = self.stage.logits(hidden[-1])
        return decode_result(logits), logits

    def teacher_forced(self, token_ids, start=0):
        """Logits at every position of ``token_ids`` fed from slot ``start``,
        as the reference's gate collects them by decoding the tokens one by
        one (npu_llm/tests/validate_engine_npu.py:58-64); here every row of
        ``prefill`` goes through the final norm and the LM head.  Returns an
        ``(n, vocab)`` float32 array."""
        ids = [int(t) for t in token_ids]
        if not ids:
            raise ValueError("teacher forcing needs at least one token")
        if start < 0 or start + len(ids) > self.context_length:
            raise ValueError("position outside the context")
        hidden = round_f32(self._embedding[np.asarray(ids)])
        for layer in range(self.layers):
            hidden = self.stage.layer_rows(hidden, layer, start)
        return np.ascontiguousarray(self.stage.logits_rows(hidden), dtype=np.float32)

    def generate_greedy(self, prompt_ids, new_tokens, *, keep_logits=True, timings=None):
        """Per-position prefill (logits at the last prompt position only),
        then greedy decode; returns ``(tokens, per-step logits)``.

        ``timings`` (a list) receives ``time.perf_counter`` durations of each
        step, prefill steps first, as generate.py:1110-1158 records them.
        """
        tokens, logits_seq = [], []
        last = len(prompt_ids) - 1
        nxt = None
        for i, tok in enumerate(prompt_ids):
            t0 = time.perf_counter()
            nxt, lg = self.decode_token(int(tok), i, compute_logits=(i == last))
            if timings is not None:
                timings.append(time.perf_counter() - t0)
        position = len(prompt_ids)
        if keep_logits:
            logits_seq.append(lg)
        tokens.append(nxt)
        while len(tokens) < new_tokens:
            t0 = time.perf_counter()
            nxt, lg = self.decode_token(tokens[-1], position)
            if timings is not None:
                timings.append(time.perf_counter() - t0)
            tokens.append(nxt)
            if keep_logits:
                logits_seq.append(lg)
            position += 1
        return tokens, logits_seq
