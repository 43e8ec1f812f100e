"""ctypes binding of libhk.so, the C ABI declared in include/hk.h.

Loading fails loudly: there is no CPU fallback.  ``HK_ERR_INVALID`` maps to
``ValueError`` (the reference raises ValueError for bad positions,
npu_llm/runtime/qwen_engine.py:84-85); every other failure maps to
``RuntimeError`` (the reference's hardware/runtime errors).
"""

import ctypes
import os
import threading
from pathlib import Path

__all__ = [
    "LIB_PATH",
    "lib",
    "check",
    "ModelDesc",
    "LayerWeights",
    "ModelWeights",
    "HK_MODEL_QKV_BIAS",
    "HK_MODEL_W8",
]

LIB_PATH = Path(os.environ.get("HK_LIB", Path(__file__).resolve().parent.parent / "lib" / "libhk.so"))

HK_OK = 0
HK_ERR_INVALID = 1
HK_ERR_HIP = 2
HK_ERR_UNSUPPORTED = 3
HK_MODEL_QKV_BIAS = 1
HK_MODEL_W8 = 2
PARTS = {"qkv": 0, "attention": 1, "o_proj": 2, "gate_up": 3, "down_proj": 4, "lm_head": 5}
PART_STEP = 6  # the whole decode step as the engine runs it

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("layers", _i32),
        ("hidden", _i32),
        ("intermediate", _i32),
        ("q_heads", _i32),
        ("kv_heads", _i32),
        ("head_dim", _i32),
        ("vocab", _i32),
        ("max_context", _i32),
        ("rms_eps", _f32),
        ("flags", ctypes.c_uint32),
    ]


class LayerWeights(ctypes.Structure):
    _fields_ = [
        ("qkv", _vp),
        ("qkv_scale", _vp),
        ("qkv_bias", _vp),
        ("o_proj", _vp),
        ("o_scale", _vp),
        ("gate_up", _vp),
        ("gate_up_scale", _vp),
        ("down_proj", _vp),
        ("down_scale", _vp),
        ("input_norm", _vp),
        ("post_attn_norm", _vp),
    ]


class ModelWeights(ctypes.Structure):
    _fields_ = [
        ("token_embedding", _vp),
        ("lm_head", _vp),
        ("final_norm", _vp),
        ("rope_cos", _vp),
        ("rope_sin", _vp),
        ("layers", ctypes.POINTER(LayerWeights)),
    ]


# name -> (restype, argtypes)
_SIGNATURES = {
    "hk_abi_version": (_i32, []),
    "hk_last_error": (ctypes.c_char_p, []),
    "hk_init": (ctypes.c_int, [_i32]),
    "hk_engine_create": (
        ctypes.c_int,
        [ctypes.POINTER(ModelDesc), ctypes.POINTER(ModelWeights), ctypes.POINTER(_vp)],
    ),
    "hk_engine_step": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "hk_engine_generate": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp]),
    "hk_engine_prefill": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "hk_engine_final_hidden": (ctypes.c_int, [_vp, _vp]),
    "hk_engine_read_kv": (ctypes.c_int, [_vp, _i32, _i32, _vp, _vp]),
    "hk_engine_launch_part": (ctypes.c_int, [_vp, _i32, _i32]),
    "hk_engine_launch_part_repeat": (ctypes.c_int, [_vp, _i32, _i32]),
    "hk_gemv_repeat": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp]),
    "hk_engine_reset": (ctypes.c_int, [_vp]),
    "hk_engine_skip_epochs": (ctypes.c_int, [_vp, ctypes.c_uint32]),
    "hk_engine_stream": (_vp, [_vp]),
    "hk_engine_step_kind": (ctypes.c_int, [_vp, _i32, ctypes.POINTER(_i32)]),
    "hk_engine_destroy": (None, [_vp]),
    "hk_gemv_bf16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "hk_gemv_w8": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "hk_gemm_bf16": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "hk_rmsnorm": (ctypes.c_int, [_vp, _vp, _f32, _vp, _i32, _vp]),
    "hk_swiglu": (ctypes.c_int, [_vp, _vp, _i32, _vp]),
    "hk_argmax_f32": (ctypes.c_int, [_vp, _i32, _vp, _vp]),
    "hk_attention_decode": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp],
    ),
    "hk_attention_decode_noalloc": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp],
    ),
    "hk_stream_sync": (ctypes.c_int, [_vp]),
    "hk_moe_create": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.POINTER(_vp)]),
    "hk_moe_forward": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "hk_moe_experts": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "hk_moe_destroy": (None, [_vp]),
    "hk_malloc": (ctypes.c_int, [ctypes.c_uint64, ctypes.POINTER(_vp)]),
    "hk_free": (ctypes.c_int, [_vp]),
    "hk_memcpy_h2d": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64]),
    "hk_memcpy_d2h": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64]),
    "hk_memcpy_d2d": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64]),
    "hk_memset": (ctypes.c_int, [_vp, _i32, ctypes.c_uint64]),
    "hk_stream_create": (ctypes.c_int, [ctypes.POINTER(_vp)]),
    "hk_stream_destroy": (ctypes.c_int, [_vp]),
    "hk_event_create": (ctypes.c_int, [ctypes.POINTER(_vp)]),
    "hk_event_destroy": (ctypes.c_int, [_vp]),
    "hk_event_record": (ctypes.c_int, [_vp, _vp]),
    "hk_event_elapsed_ms": (ctypes.c_int, [_vp, _vp, ctypes.POINTER(_f32)]),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None
_initialised = set()


def lib():
    """Load libhk.so once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.is_file():
                raise RuntimeError(
                    f"{LIB_PATH} not found: build it with "
                    "`python hawkpoint-npu-llm_amd/csrc/build.py` (no CPU fallback exists)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
        return _lib


def last_error():
    msg = lib().hk_last_error()
    return msg.decode() if msg else ""


def check(rc, what):
    if rc == HK_OK:
        return
    message = f"{what}: {last_error()}"
    if rc == HK_ERR_INVALID:
        raise ValueError(message)
    raise RuntimeError(message)


def init(device=0):
    """hk_init once per device (selects it and checks it is a gfx950)."""
    if device in _initialised:
        return
    check(lib().hk_init(int(device)), "hk_init")
    _initialised.add(device)


class DeviceBuffer:
    """A device allocation owned by Python (freed by ``free`` or on collection)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        ptr = _vp()
        check(lib().hk_malloc(self.nbytes, ctypes.byref(ptr)), "hk_malloc")
        self.ptr = ptr.value

    @classmethod
    def from_array(cls, array):
        import numpy as np

        array = np.ascontiguousarray(array)
        buf = cls(max(array.nbytes, 1))
        if array.nbytes:
            check(
                lib().hk_memcpy_h2d(buf.ptr, array.ctypes.data, array.nbytes), "hk_memcpy_h2d"
            )
        buf.dtype = array.dtype
        buf.shape = array.shape
        return buf

    def write(self, array, offset=0):
        import numpy as np

        array = np.ascontiguousarray(array)
        if offset < 0 or offset + array.nbytes > self.nbytes:
            raise ValueError("write outside the device buffer")
        check(lib().hk_memcpy_h2d(self.ptr + offset, array.ctypes.data, array.nbytes), "hk_memcpy_h2d")

    def read(self, dtype, count, offset=0):
        import numpy as np

        out = np.empty(count, dtype=dtype)
        if offset < 0 or offset + out.nbytes > self.nbytes:
            raise ValueError("read outside the device buffer")
        check(lib().hk_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "hk_memcpy_d2h")
        return out

    def zero(self):
        check(lib().hk_memset(self.ptr, 0, self.nbytes), "hk_memset")

    def free(self):
        if getattr(self, "ptr", None):
            try:
                lib().hk_free(self.ptr)
            finally:
                self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    """A HIP event for timing work on a stream."""

    def __init__(self):
        ev = _vp()
        check(lib().hk_event_create(ctypes.byref(ev)), "hk_event_create")
        self.handle = ev.value

    def record(self, stream):
        check(lib().hk_event_record(self.handle, stream), "hk_event_record")

    def elapsed_ms(self, end):
        ms = _f32()
        check(lib().hk_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)), "hk_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                lib().hk_event_destroy(self.handle)
        except Exception:
            pass
