"""Host side of the hk decode engine: every decoder layer, the final RMSNorm,
the LM head and the argmax for one token per call, on one MI355X.

Keeps the reference engine's interface (``npu_llm/runtime/qwen_engine.py:37-102``):
``QwenDecoderEngine(model)``, ``step(embedding, position, logits=True)`` returning
float32 logits or None, ``reset()`` and ``close()``.  The work runs through
``libhk.so`` (include/hk.h); weights, the KV cache and the activations stay in
HBM, and the KV append happens on the device inside the step.

Differences from the NPU engine, all in the caller's favour:
- any layer count, head layout with 64-wide heads, and context length
  (the NPU engine is fixed to Qwen2.5-0.5B at 64 slots);
- ``step_token`` looks the embedding row up on the device;
- ``generate`` runs greedy decode steps back to back without host round trips.
"""

import ctypes

import numpy as np

from runtime import hip
from runtime.bf16 import to_bits

__all__ = ["QwenDecoderEngine", "rope_tables", "supports"]


def rope_tables(theta, head_dim, context):
    """cos/sin tables [context, head_dim/2] float32, computed per position with
    the reference's expression (npu_llm/runtime/cpu_backend.py:26-32, 81-83),
    so the device sees bit-identical angles."""
    half = head_dim // 2
    inv = 1.0 / (float(theta) ** (np.arange(half, dtype=np.float32) / np.float32(half)))
    cos = np.empty((context, half), dtype=np.float32)
    sin = np.empty((context, half), dtype=np.float32)
    for p in range(context):
        angle = np.float32(p) * inv
        cos[p] = np.cos(angle)
        sin[p] = np.sin(angle)
    return cos, sin


def supports(metadata):
    """Shapes the engine runs: 64-wide heads, grouped heads, aligned sizes."""
    try:
        return (
            int(metadata["head_dim"]) == 64
            and int(metadata["attention_heads"]) % int(metadata["kv_heads"]) == 0
            and int(metadata["attention_heads"]) // int(metadata["kv_heads"]) <= 16
            and int(metadata["hidden_size"]) % 16 == 0
            and int(metadata["intermediate_size"]) % 16 == 0
        )
    except (KeyError, TypeError, ValueError, ZeroDivisionError):
        return False


def _bits_of(model, name):
    """bf16 bit patterns (uint16) of a stored tensor."""
    raw = model.raw(name)
    if getattr(model, "is_bf16", None) is not None and model.is_bf16(name):
        return np.asarray(raw, dtype=np.uint16)
    return to_bits(np.asarray(raw, dtype=np.float32))


class QwenDecoderEngine:
    """All layers + final norm + LM head + argmax per call (see module doc)."""

    def __init__(self, model, *, context_length=4096, w8=False, device=0):
        meta = model.metadata
        if not supports(meta):
            raise ValueError("the hk engine needs 64-wide heads and 16-aligned sizes")
        hip.init(device)
        self._lib = hip.lib()
        self.layers = int(meta["layers"])
        self.hidden = int(meta["hidden_size"])
        self.vocab = int(meta["vocab_size"])
        self.kv_heads = int(meta["kv_heads"])
        self.context_length = int(context_length)
        self.w8 = bool(w8)
        self._buffers = []
        up = self._upload
        theta = float(meta.get("rope_theta", 10000.0))
        cos, sin = rope_tables(theta, int(meta["head_dim"]), self.context_length)
        has_bias = False
        layer_structs = (hip.LayerWeights * self.layers)()
        for layer in range(self.layers):
            p = f"layer{layer:02d}"
            lw = layer_structs[layer]
            for field, name in (
                ("qkv", "qkv"),
                ("o_proj", "o_proj"),
                ("gate_up", "gate_up"),
                ("down_proj", "down_proj"),
            ):
                full = f"{p}.{name}"
                if self.w8:
                    q = model.quantized(full)
                    setattr(lw, field, up(np.asarray(q.weight, dtype=np.int8)))
                    scale_field = {"qkv": "qkv_scale", "o_proj": "o_scale",
                                   "gate_up": "gate_up_scale", "down_proj": "down_scale"}[field]
                    setattr(lw, scale_field, up(np.asarray(q.scale, dtype=np.float32)))
                else:
                    setattr(lw, field, up(np.asarray(model.bf16_projection(full), dtype=np.uint16)))
            bias_name = f"{p}.qkv_bias"
            if bias_name in model.tensors:
                lw.qkv_bias = up(np.asarray(model.raw_f32(bias_name), dtype=np.float32))
                has_bias = True
            lw.input_norm = up(_bits_of(model, f"{p}.input_norm"))
            lw.post_attn_norm = up(_bits_of(model, f"{p}.post_attn_norm"))
        self._layer_structs = layer_structs
        emb = up(_bits_of(model, "token_embedding"))
        lm = model.bf16_projection("lm_head")
        emb_bits = model.raw("token_embedding") if hasattr(model, "raw") else None
        lm_ptr = emb if (emb_bits is not None and lm is emb_bits) else up(np.asarray(lm, np.uint16))
        weights = hip.ModelWeights(
            token_embedding=emb,
            lm_head=lm_ptr,
            final_norm=up(_bits_of(model, "final_norm")),
            rope_cos=up(cos),
            rope_sin=up(sin),
            layers=layer_structs,
        )
        flags = (hip.HK_MODEL_QKV_BIAS if has_bias else 0) | (hip.HK_MODEL_W8 if self.w8 else 0)
        desc = hip.ModelDesc(
            layers=self.layers,
            hidden=self.hidden,
            intermediate=int(meta["intermediate_size"]),
            q_heads=int(meta["attention_heads"]),
            kv_heads=int(meta["kv_heads"]),
            head_dim=int(meta["head_dim"]),
            vocab=self.vocab,
            max_context=self.context_length,
            rms_eps=float(np.float32(meta.get("rms_norm_eps", 1e-5))),
            flags=flags,
        )
        handle = ctypes.c_void_p()
        hip.check(
            self._lib.hk_engine_create(ctypes.byref(desc), ctypes.byref(weights), ctypes.byref(handle)),
            "hk_engine_create",
        )
        self._engine = handle.value
        self._logits = np.empty(self.vocab, dtype=np.float32)
        self._token = ctypes.c_int32()

    def _upload(self, array):
        buf = hip.DeviceBuffer.from_array(array)
        self._buffers.append(buf)
        return buf.ptr

    @property
    def stream(self):
        return self._lib.hk_engine_stream(self._engine)

    STEP_KINDS = {0: "kernels", 1: "persistent", 2: "xcd_split", 3: "xcd_split_long"}

    def step_kind(self, position):
        """How a decode step at `position` runs: "kernels" (one kernel per
        part, replayed as a hipGraph), "persistent" (one launch over all CUs),
        "xcd_split" (one launch, attention block on XCD 0, MLP on the other
        XCDs) or "xcd_split_long" (the same with the attention tasks on the
        MLP XCDs, for longer contexts)."""
        kind = ctypes.c_int32()
        hip.check(self._lib.hk_engine_step_kind(self._live(), int(position), ctypes.byref(kind)),
                  "hk_engine_step_kind")
        return self.STEP_KINDS[kind.value]

    def _live(self):
        if self._engine is None:
            raise RuntimeError("engine is closed")
        return self._engine

    def reset(self):
        hip.check(self._lib.hk_engine_reset(self._live()), "hk_engine_reset")

    def skip_epochs(self, count):
        """Test hook: advance the persistent step's epoch counter by ``count``
        (see hk_engine_skip_epochs)."""
        hip.check(self._lib.hk_engine_skip_epochs(self._live(), int(count)), "hk_engine_skip_epochs")

    def step(self, embedding, position, logits=True):
        """Run every layer for one token given its bf16 embedding row (uint16
        bits, [H]) and return its float32 logits (None with ``logits=False``).
        Attention reads slots 0..position; slot ``position`` is written."""
        row = np.ascontiguousarray(np.asarray(embedding, dtype=np.uint16))
        if row.shape != (self.hidden,):
            raise ValueError(f"embedding row must have {self.hidden} bf16 values")
        out = self._logits if logits else None
        hip.check(
            self._lib.hk_engine_step(
                self._live(), 0, int(position), 1 if logits else 0, row.ctypes.data,
                out.ctypes.data if out is not None else None, None,
            ),
            "hk_engine_step",
        )
        return np.array(out, copy=True) if logits else None

    def step_token(self, token_id, position, logits=True, want_logits_array=True):
        """Like ``step`` but the embedding row is looked up on the device.
        Returns ``(next_token, logits)``; ``(None, None)`` with ``logits=False``.
        ``want_logits_array=False`` skips copying the logits to the host."""
        if not logits:
            hip.check(
                self._lib.hk_engine_step(self._live(), int(token_id), int(position), 0, None, None, None),
                "hk_engine_step",
            )
            return None, None
        out = self._logits if want_logits_array else None
        hip.check(
            self._lib.hk_engine_step(
                self._live(), int(token_id), int(position), 1, None,
                out.ctypes.data if out is not None else None, ctypes.byref(self._token),
            ),
            "hk_engine_step",
        )
        return int(self._token.value), (np.array(out, copy=True) if out is not None else None)

    def prefill(self, token_ids, start=0, logits=True, want_logits_array=True):
        """All prompt tokens at slots start..start+n-1 in one batched pass
        (MFMA GEMMs, causal attention).  Returns ``(next_token, logits)`` for
        the last token, or ``(None, None)`` with ``logits=False``."""
        ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.int32))
        if ids.ndim != 1 or ids.size == 0:
            raise ValueError("prefill needs a non-empty 1-D list of token ids")
        out = self._logits if (logits and want_logits_array) else None
        hip.check(
            self._lib.hk_engine_prefill(
                self._live(), ids.ctypes.data, int(ids.size), int(start),
                out.ctypes.data if out is not None else None,
                ctypes.byref(self._token) if logits else None,
            ),
            "hk_engine_prefill",
        )
        if not logits:
            return None, None
        return int(self._token.value), (np.array(out, copy=True) if out is not None else None)

    def generate(self, token_id, position, n_steps):
        """Greedy decode: ``n_steps`` tokens starting from ``token_id`` at
        ``position`` (the token fed at step i is the argmax of step i-1)."""
        out = np.empty(int(n_steps), dtype=np.int32)
        hip.check(
            self._lib.hk_engine_generate(self._live(), int(token_id), int(position), int(n_steps), out.ctypes.data),
            "hk_engine_generate",
        )
        return [int(t) for t in out]

    def read_kv(self, layer, slot):
        """(k, v) bf16 bits [kv_heads, 64] stored at ``slot`` of ``layer``."""
        kvh = self.kv_heads
        k = np.empty((kvh, 64), dtype=np.uint16)
        v = np.empty((kvh, 64), dtype=np.uint16)
        hip.check(
            self._lib.hk_engine_read_kv(self._live(), int(layer), int(slot), k.ctypes.data, v.ctypes.data),
            "hk_engine_read_kv",
        )
        return k, v

    def final_hidden(self):
        """bf16 bits of RMSNorm(final_norm) applied to the last step's hidden state."""
        out = np.empty(self.hidden, dtype=np.uint16)
        hip.check(self._lib.hk_engine_final_hidden(self._live(), out.ctypes.data), "hk_engine_final_hidden")
        return out

    def close(self):
        if getattr(self, "_engine", None) is not None:
            self._lib.hk_engine_destroy(self._engine)
            self._engine = None
        for buf in getattr(self, "_buffers", []):
            buf.free()
        self._buffers = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
