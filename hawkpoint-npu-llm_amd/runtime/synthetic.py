"""Seeded random-init models in the reference's package layout.

A ``SyntheticModel`` exposes the accessor surface the engines read from an
on-disk package (``npu_llm/runtime/model.py:84-198``): ``metadata``,
``tensors``, ``raw``/``raw_f32``, ``bf16_projection`` and ``quantized``,
with the tensor names and concatenation orders the reference converter
writes (``npu_llm/tools/convert_smollm2.py:220-311``):

- ``token_embedding``             [V, H] bf16
- ``layerNN.qkv``                 [(Hq + 2 Hkv) D, H] rows q, k, v
- ``layerNN.qkv_bias``            [(Hq + 2 Hkv) D] float32 (zeros without bias)
- ``layerNN.o_proj``              [H, Hq D]
- ``layerNN.gate_up``             [2 I, H] rows gate then up
- ``layerNN.down_proj``           [H, I]
- ``layerNN.input_norm`` / ``layerNN.post_attn_norm`` / ``final_norm``  [H] bf16
- ``lm_head``                     tied: the embedding

Weights are N(0, 0.02) float32 samples rounded to bf16; RMSNorm gains are
1.0, or with ``norm_gains=g`` bf16 samples of U(0.5, 1.5) for the layer norms
and of g * U(0.5, 1.5) for the final norm, drawn from a generator of their
own (seed + 7919) so the weights stay those of the same seed; a final gain
of about 8 spreads the logits of these random weights like a trained
model's (standard deviation of a few units instead of about 0.5); the qkv
bias is N(0, 0.02) float32 when the shape has one.  W8 tensors
are the per-output-row int8 quantisation of the bf16 weights
(``convert_smollm2.py:81-86``), computed lazily.

Draw order from ``numpy.random.default_rng(seed)``: embedding, then per layer
qkv, qkv bias (bias shapes only), o_proj, gate_up, down_proj.
"""

import numpy as np

from runtime.bf16 import from_bits, to_bits

__all__ = ["SMOLLM2_135M", "QWEN25_05B", "SyntheticModel", "QuantizedWeights", "quantize_rows"]

SMOLLM2_135M = {
    "model_family": "llama",
    "hidden_size": 576,
    "intermediate_size": 1536,
    "attention_heads": 9,
    "kv_heads": 3,
    "head_dim": 64,
    "layers": 30,
    "vocab_size": 49152,
    "rope_theta": 100000.0,
    "rms_norm_eps": 1e-5,
    "qkv_bias": False,
}

QWEN25_05B = {
    "model_family": "qwen2",
    "hidden_size": 896,
    "intermediate_size": 4864,
    "attention_heads": 14,
    "kv_heads": 2,
    "head_dim": 64,
    "layers": 24,
    "vocab_size": 151936,
    "rope_theta": 1000000.0,
    "rms_norm_eps": 1e-6,
    "qkv_bias": True,
}

_ONE_BF16 = np.uint16(0x3F80)


def quantize_rows(weight_f32):
    """int8 per-output-row symmetric quantisation (convert_smollm2.py:81-86)."""
    w = np.asarray(weight_f32, dtype=np.float32)
    max_abs = np.max(np.abs(w), axis=1)
    scale = np.maximum(max_abs / 127.0, np.finfo(np.float32).tiny).astype(np.float32)
    q = np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale


class QuantizedWeights:
    """int8 weights [M, K] and float32 scales [M] (runtime/model.py:61-81)."""

    def __init__(self, weight, scale):
        self.weight = weight
        self.scale = scale
        self.shape = tuple(weight.shape)


class SyntheticModel:
    """Random-init model of a given shape; see the module docstring."""

    def __init__(self, shape, seed=0, *, layers=None, std=0.02, norm_gains=None):
        shape = dict(shape)
        if layers is not None:
            shape["layers"] = int(layers)
        self.shape = shape
        self.seed = int(seed)
        h = shape["hidden_size"]
        inter = shape["intermediate_size"]
        d = shape["head_dim"]
        nq, nkv = shape["attention_heads"], shape["kv_heads"]
        vocab = shape["vocab_size"]
        qkv_rows = (nq + 2 * nkv) * d
        self.metadata = {
            "model_family": shape["model_family"],
            "hidden_size": h,
            "intermediate_size": inter,
            "attention_heads": nq,
            "kv_heads": nkv,
            "head_dim": d,
            "layers": shape["layers"],
            "vocab_size": vocab,
            "rope_theta": float(shape["rope_theta"]),
            "rms_norm_eps": float(shape["rms_norm_eps"]),
            "activation_dtype": "bfloat16",
            "accumulator_dtype": "float32",
        }
        rng = np.random.default_rng(self.seed)
        sd = np.float32(std)

        def normal(*dims):
            return rng.standard_normal(dims, dtype=np.float32) * sd

        self._bits = {}
        self._f32 = {}
        self._quant = {}
        self.tensors = {}
        self._bits["token_embedding"] = to_bits(normal(vocab, h))
        self.tensors["token_embedding"] = {"shape": [vocab, h], "dtype": "bfloat16"}
        ones = np.full(h, _ONE_BF16, dtype=np.uint16)
        for layer in range(shape["layers"]):
            p = f"layer{layer:02d}"
            self._put_proj(f"{p}.qkv", normal(qkv_rows, h))
            bias = normal(qkv_rows) if shape["qkv_bias"] else np.zeros(qkv_rows, np.float32)
            self._f32[f"{p}.qkv_bias"] = bias
            self.tensors[f"{p}.qkv_bias"] = {"shape": [qkv_rows], "dtype": "float32"}
            self._put_proj(f"{p}.o_proj", normal(h, nq * d))
            self._put_proj(f"{p}.gate_up", normal(2 * inter, h))
            self._put_proj(f"{p}.down_proj", normal(h, inter))
            for g in ("input_norm", "post_attn_norm"):
                self._bits[f"{p}.{g}"] = ones
                self.tensors[f"{p}.{g}"] = {"shape": [h], "dtype": "bfloat16"}
        self._bits["final_norm"] = ones
        self.tensors["final_norm"] = {"shape": [h], "dtype": "bfloat16"}
        if norm_gains is not None:
            gain_rng = np.random.default_rng(self.seed + 7919)
            for layer in range(shape["layers"]):
                for g in ("input_norm", "post_attn_norm"):
                    self._bits[f"layer{layer:02d}.{g}"] = to_bits(gain_rng.uniform(0.5, 1.5, h).astype(np.float32))
            final = np.float32(norm_gains) * gain_rng.uniform(0.5, 1.5, h).astype(np.float32)
            self._bits["final_norm"] = to_bits(final)
        self._bits["lm_head"] = self._bits["token_embedding"]
        self.tensors["lm_head"] = {"shape": [vocab, h], "bf16_file": "tied"}

    def _put_proj(self, name, weight):
        self._bits[name] = to_bits(weight)
        self.tensors[name] = {"shape": list(weight.shape), "bf16_file": name}

    # -- accessors mirroring runtime/model.py ------------------------------
    def bf16_projection(self, name):
        """bf16 bits (uint16) of a projection, [M, K]."""
        return self._bits[name]

    def raw(self, name):
        """Stored tensor: uint16 bits for bf16 tensors, float32 otherwise."""
        if name in self._f32:
            return self._f32[name]
        return self._bits[name]

    def raw_f32(self, name):
        """Stored tensor widened to float32 (exact)."""
        if name in self._f32:
            return self._f32[name]
        return from_bits(self._bits[name])

    def is_bf16(self, name):
        return name in self._bits

    def quantized(self, name):
        if name not in self._quant:
            q, s = quantize_rows(from_bits(self._bits[name]))
            self._quant[name] = QuantizedWeights(q, s)
        return self._quant[name]
