"""ctypes binding of include/hk_experts.h: the GGML MUL_MAT_ID and Colibri
``coli_cuda_*`` expert-projection shims exported by libhk.so.

Both contracts take host arrays.  ``GgmlExperts`` wraps one MUL_MAT_ID weight
tensor (ollama-xdna/backend/ggml-xdna.cpp:1301-1441); ``ColiTensor`` and
``expert_group`` wrap Colibri's tensor upload and expert group
(colibri-xdna/backend/backend_xdna.cpp:273-358).  Colibri's functions report
failure as 0 (the caller falls back to its CPU path); here that becomes
``RuntimeError``, as there is no fallback behind this binding.
"""

import ctypes

import numpy as np

from runtime import hip

__all__ = ["EXPORTED", "GgmlExperts", "ggml_supported", "dense_supported", "quant_supported", "GGML_Q4_K",
           "GGML_Q6_K", "ColiTensor", "coli_init", "coli_shutdown", "coli_matmul", "expert_group", "expert_mlp"]

GGML_Q4_K = 12  # ggml_type values (include/hk_experts.h)
GGML_Q6_K = 14
BLOCK_BYTES = {GGML_Q4_K: 144, GGML_Q6_K: 210}

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

_SIGNATURES = {
    "hk_ggml_experts_supported": (ctypes.c_int, [_i64, _i64, _i64, _i64, _i64]),
    "hk_ggml_experts_create": (ctypes.c_int, [_vp, _i64, _i64, _i64, ctypes.POINTER(_vp)]),
    "hk_ggml_mul_mat_id": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64, _vp]),
    "hk_ggml_experts_destroy": (None, [_vp]),
    "hk_ggml_mul_mat_id_repeat": (ctypes.c_int, [_vp, _vp, _i64, ctypes.POINTER(ctypes.c_float)]),
    "hk_ggml_dense_supported": (ctypes.c_int, [_i64, _i64, _i64]),
    "hk_ggml_quant_supported": (ctypes.c_int, [ctypes.c_int, _i64]),
    "hk_ggml_dense_create": (ctypes.c_int, [_vp, _i64, _i64, ctypes.POINTER(_vp)]),
    "hk_ggml_quant_create": (ctypes.c_int, [ctypes.c_int, _vp, _i64, _i64, _i64, ctypes.POINTER(_vp)]),
    "hk_ggml_mul_mat": (ctypes.c_int, [_vp, _vp, _vp]),
    "coli_cuda_init": (ctypes.c_int, [_vp, ctypes.c_int]),
    "coli_cuda_shutdown": (None, []),
    "coli_cuda_available_device_count": (ctypes.c_int, []),
    "coli_cuda_device_count": (ctypes.c_int, []),
    "coli_cuda_device_at": (ctypes.c_int, [ctypes.c_int]),
    "coli_cuda_tensor_upload_g": (
        ctypes.c_int, [ctypes.POINTER(_vp), _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                       ctypes.c_int, ctypes.c_int]),
    "coli_cuda_tensor_upload": (
        ctypes.c_int, [ctypes.POINTER(_vp), _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "coli_cuda_tensor_free": (None, [_vp]),
    "coli_cuda_tensor_device": (ctypes.c_int, [_vp]),
    "coli_cuda_tensor_update": (ctypes.c_int, [_vp, _vp, _vp]),
    "coli_cuda_matmul": (
        ctypes.c_int, [ctypes.POINTER(_vp), _vp, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                       ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "coli_cuda_expert_group_pinned": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, ctypes.c_int]),
    "coli_cuda_expert_group": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp]),
    "coli_cuda_expert_mlp": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int]),
}

EXPORTED = tuple(_SIGNATURES)

_bound = None


def lib():
    global _bound
    if _bound is None:
        handle = hip.lib()
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _bound = handle
    return _bound


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- GGML ----

def ggml_supported(in_dim, out_dim, n_experts, n_ids, input_rows):
    return bool(lib().hk_ggml_experts_supported(in_dim, out_dim, n_experts, n_ids, input_rows))


def dense_supported(in_dim, out_dim, input_rows=1):
    return bool(lib().hk_ggml_dense_supported(in_dim, out_dim, input_rows))


def quant_supported(ggml_type, in_dim):
    return bool(lib().hk_ggml_quant_supported(ggml_type, in_dim))


class GgmlExperts:
    """One GGML weight tensor on the device.

    ``GgmlExperts(w)``: float32 [n_experts][out][in], requantised per row
    (MUL_MAT_ID).  ``GgmlExperts.dense(w)``: float32 [out][in], one scale per
    (row, 2048-column tile) (MUL_MAT).  ``GgmlExperts.quant(type, blocks,
    n_experts, out, in)``: Q4_K / Q6_K blocks as GGML holds them (both).
    """

    def __init__(self, weights=None, *, _handle=None, _shape=None):
        if _handle is not None:
            self.handle = _handle
            self.n_experts, self.out_dim, self.in_dim = _shape
            return
        w = _f32(weights)
        if w.ndim != 3:
            raise ValueError("weights must be [n_experts][out][in]")
        self.n_experts, self.out_dim, self.in_dim = w.shape
        handle = _vp()
        hip.check(lib().hk_ggml_experts_create(w.ctypes.data, *w.shape, ctypes.byref(handle)),
                  "hk_ggml_experts_create")
        self.handle = handle.value

    @classmethod
    def dense(cls, weights):
        w = _f32(weights)
        if w.ndim != 2:
            raise ValueError("weights must be [out][in]")
        handle = _vp()
        hip.check(lib().hk_ggml_dense_create(w.ctypes.data, w.shape[0], w.shape[1], ctypes.byref(handle)),
                  "hk_ggml_dense_create")
        return cls(_handle=handle.value, _shape=(1, w.shape[0], w.shape[1]))

    @classmethod
    def quant(cls, ggml_type, blocks, n_experts, out_dim, in_dim):
        b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
        need = n_experts * out_dim * (in_dim // 256) * BLOCK_BYTES.get(ggml_type, 0)
        if ggml_type in BLOCK_BYTES and in_dim % 256 == 0 and b.size != need:
            raise ValueError(f"expected {need} bytes of blocks, got {b.size}")
        handle = _vp()
        hip.check(lib().hk_ggml_quant_create(ggml_type, b.ctypes.data, n_experts, out_dim, in_dim,
                                             ctypes.byref(handle)), "hk_ggml_quant_create")
        return cls(_handle=handle.value, _shape=(n_experts, out_dim, in_dim))

    def mul_mat(self, x):
        x = _f32(x).reshape(-1)
        if x.size != self.in_dim:
            raise ValueError("input length must equal in_dim")
        out = np.empty(self.out_dim, dtype=np.float32)
        hip.check(lib().hk_ggml_mul_mat(self.handle, x.ctypes.data, out.ctypes.data), "hk_ggml_mul_mat")
        return out

    def mul_mat_id(self, inputs, ids):
        x = _f32(inputs).reshape(-1, self.in_dim)
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        out = np.empty((ids.size, self.out_dim), dtype=np.float32)
        hip.check(lib().hk_ggml_mul_mat_id(self.handle, x.ctypes.data, x.shape[0], ids.ctypes.data,
                                           ids.size, out.ctypes.data), "hk_ggml_mul_mat_id")
        return out

    def repeat_ms(self, ids):
        """Average kernel time (ms) of launches re-running the last call with
        the id rows of ``ids`` ([launches][n_ids])."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        ms = ctypes.c_float()
        hip.check(lib().hk_ggml_mul_mat_id_repeat(self.handle, ids.ctypes.data, ids.shape[0], ctypes.byref(ms)),
                  "hk_ggml_mul_mat_id_repeat")
        return float(ms.value)

    def close(self):
        if getattr(self, "handle", None):
            lib().hk_ggml_experts_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- Colibri ----

def coli_init(device=0):
    devices = (ctypes.c_int * 1)(device)
    if not lib().coli_cuda_init(devices, 1):
        raise RuntimeError("coli_cuda_init failed")


def coli_shutdown():
    lib().coli_cuda_shutdown()


def _pointer(a):
    return None if a is None else a.ctypes.data


def _weights_array(weights, fmt):
    dtype = {0: np.float32, 1: np.int8, 2: np.uint8, 4: np.uint8}.get(fmt, np.uint8)
    return np.ascontiguousarray(weights, dtype=dtype)


class ColiTensor:
    """A Colibri weight upload: ``fmt`` 0/1/2/4 as backend_xdna.cpp:122-136."""

    def __init__(self, weights, scales, fmt, input_size, output_size, group=0, device=0):
        self._w = _weights_array(weights, fmt)
        self._s = None if scales is None else _f32(scales)
        handle = _vp()
        ok = lib().coli_cuda_tensor_upload_g(ctypes.byref(handle), self._w.ctypes.data, _pointer(self._s),
                                             fmt, input_size, output_size, device, group)
        if not ok:
            raise RuntimeError("coli_cuda_tensor_upload_g failed")
        self.handle = handle.value
        self.input_size, self.output_size = input_size, output_size

    def update(self, weights, scales):
        w = np.ascontiguousarray(weights, dtype=self._w.dtype)
        s = None if scales is None else _f32(scales)
        if not lib().coli_cuda_tensor_update(self.handle, w.ctypes.data, _pointer(s)):
            raise RuntimeError("coli_cuda_tensor_update failed")

    def device(self):
        return lib().coli_cuda_tensor_device(self.handle)

    def close(self):
        if getattr(self, "handle", None):
            lib().coli_cuda_tensor_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def coli_matmul(weights, scales, fmt, x, input_size, output_size, group=0):
    """``coli_cuda_matmul`` with a fresh tensor (uploaded on first use, then freed)."""
    x = _f32(x)
    w = _weights_array(weights, fmt)
    s = None if scales is None else _f32(scales)
    out = np.zeros(output_size, dtype=np.float32)
    handle = _vp()
    ok = lib().coli_cuda_matmul(ctypes.byref(handle), out.ctypes.data, x.ctypes.data, w.ctypes.data,
                                _pointer(s), fmt, 1, input_size, output_size, 0, group)
    if handle.value:
        lib().coli_cuda_tensor_free(handle.value)
    if not ok:
        raise RuntimeError("coli_cuda_matmul failed")
    return out


def expert_group(gates, ups, downs, x, pinned=0):
    """``coli_cuda_expert_group_pinned`` over ColiTensor lists; x back to back."""
    n = len(gates)
    arr = lambda ts: (_vp * n)(*[t.handle for t in ts])
    rows = (ctypes.c_int * n)(*([1] * n))
    x = _f32(x)
    out = np.zeros(sum(d.output_size for d in downs), dtype=np.float32)
    ok = lib().coli_cuda_expert_group_pinned(arr(gates), arr(ups), arr(downs), rows, n, out.ctypes.data,
                                             x.ctypes.data, pinned)
    if not ok:
        raise RuntimeError("coli_cuda_expert_group_pinned failed")
    return out


def expert_mlp(gate, up, down, x):
    x = _f32(x)
    out = np.zeros(down.output_size, dtype=np.float32)
    if not lib().coli_cuda_expert_mlp(gate.handle, up.handle, down.handle, out.ctypes.data, x.ctypes.data, 1):
        raise RuntimeError("coli_cuda_expert_mlp failed")
    return out
