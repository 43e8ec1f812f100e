"""Routed-expert (MoE) decode block on the GPU (C ABI: hk_moe_* in include/hk.h).

``MoEBlock.forward(x)`` runs the router, top-k, the routed and shared SwiGLU
experts and the weighted combine for a batch of tokens; ``experts(x, ids,
weights)`` runs only the experts for caller-supplied routing, the contract of
the reference's GGML ``MUL_MAT_ID`` offload
(``ollama-xdna/backend/ggml-xdna.cpp:1301-1441``, ``1681-1716``).

``synthetic_moe`` builds the benchmark block: hidden 2048, 64 routed experts
and 2 shared, SwiGLU intermediate 1408, top-6, bf16 N(0, 0.02) weights.
"""

import ctypes

import numpy as np

from runtime import hip
from runtime.bf16 import to_bits

__all__ = ["MoEBlock", "MoEDesc", "synthetic_moe", "MOE_2048_64X1408"]

MOE_2048_64X1408 = {"hidden": 2048, "intermediate": 1408, "experts": 64, "shared": 2, "top_k": 6}


class MoEDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("hidden", "intermediate", "experts", "shared", "top_k", "max_tokens")]


def synthetic_moe(shape=MOE_2048_64X1408, seed=0, std=0.02):
    """(router [E, H], gate_up [E+S, 2I, H], down [E+S, H, I]) bf16 bits."""
    rng = np.random.default_rng(seed)
    H, I, E, S = shape["hidden"], shape["intermediate"], shape["experts"], shape["shared"]
    sd = np.float32(std)
    router = to_bits(rng.standard_normal((E, H), dtype=np.float32) * sd)
    gate_up = np.empty((E + S, 2 * I, H), dtype=np.uint16)
    down = np.empty((E + S, H, I), dtype=np.uint16)
    for e in range(E + S):
        gate_up[e] = to_bits(rng.standard_normal((2 * I, H), dtype=np.float32) * sd)
        down[e] = to_bits(rng.standard_normal((H, I), dtype=np.float32) * sd)
    return router, gate_up, down


class MoEBlock:
    def __init__(self, router, gate_up, down, *, top_k=6, shared=2, max_tokens=16, device=0):
        hip.init(device)
        self._lib = hip.lib()
        router = np.ascontiguousarray(router, dtype=np.uint16)
        gate_up = np.ascontiguousarray(gate_up, dtype=np.uint16)
        down = np.ascontiguousarray(down, dtype=np.uint16)
        E, H = router.shape
        I = gate_up.shape[1] // 2
        if gate_up.shape != (E + shared, 2 * I, H) or down.shape != (E + shared, H, I):
            raise ValueError("expert weight shapes do not match the router and shared count")
        self.hidden, self.intermediate, self.n_experts = H, I, E
        self.shared, self.top_k, self.max_tokens = shared, top_k, max_tokens
        self._bufs = [hip.DeviceBuffer.from_array(a) for a in (router, gate_up, down)]
        desc = MoEDesc(hidden=H, intermediate=I, experts=E, shared=shared, top_k=top_k,
                       max_tokens=max_tokens)
        handle = ctypes.c_void_p()
        hip.check(self._lib.hk_moe_create(ctypes.byref(desc), self._bufs[0].ptr, self._bufs[1].ptr,
                                          self._bufs[2].ptr, ctypes.byref(handle)), "hk_moe_create")
        self._moe = handle.value
        self._x = hip.DeviceBuffer(2 * max_tokens * H)
        self._y = hip.DeviceBuffer(2 * max_tokens * H)
        self._ids = hip.DeviceBuffer(4 * max_tokens * top_k)
        self._w = hip.DeviceBuffer(4 * max_tokens * top_k)
        self._stream = None

    def _load_x(self, x_bits):
        x = np.ascontiguousarray(x_bits, dtype=np.uint16)
        if x.ndim != 2 or x.shape[1] != self.hidden or not 0 < x.shape[0] <= self.max_tokens:
            raise ValueError(f"x must be [1..{self.max_tokens}, {self.hidden}] bf16 bits")
        self._x.write(x)
        return x.shape[0]

    def forward(self, x_bits):
        """Returns (y bf16 bits [T, H], ids [T, k], weights [T, k])."""
        T = self._load_x(x_bits)
        hip.check(self._lib.hk_moe_forward(self._moe, self._x.ptr, T, self._y.ptr, self._ids.ptr,
                                           self._w.ptr, None), "hk_moe_forward")
        hip.check(self._lib.hk_stream_sync(None), "sync")
        k = self.top_k
        return (self._y.read(np.uint16, T * self.hidden).reshape(T, self.hidden),
                self._ids.read(np.int32, T * k).reshape(T, k),
                self._w.read(np.float32, T * k).reshape(T, k))

    def experts(self, x_bits, ids, weights):
        """Experts + combine for caller routing; returns y bf16 bits [T, H]."""
        T = self._load_x(x_bits)
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(T, self.top_k)
        weights = np.ascontiguousarray(weights, dtype=np.float32).reshape(T, self.top_k)
        self._ids.write(ids)
        self._w.write(weights)
        hip.check(self._lib.hk_moe_experts(self._moe, self._x.ptr, T, self._ids.ptr, self._w.ptr,
                                           self._y.ptr, None), "hk_moe_experts")
        hip.check(self._lib.hk_stream_sync(None), "sync")
        return self._y.read(np.uint16, T * self.hidden).reshape(T, self.hidden)

    def launch(self, tokens):
        """Enqueue one forward on the default stream for `tokens` rows already
        loaded (for timing)."""
        hip.check(self._lib.hk_moe_forward(self._moe, self._x.ptr, int(tokens), self._y.ptr, None,
                                           None, None), "hk_moe_forward")

    def close(self):
        if getattr(self, "_moe", None):
            self._lib.hk_moe_destroy(self._moe)
            self._moe = None
        for b in getattr(self, "_bufs", []):
            b.free()
        self._bufs = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
