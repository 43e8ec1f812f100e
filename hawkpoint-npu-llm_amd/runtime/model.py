"""Model packages in the reference's on-disk format.

Reads (``XDNA1Model``) and writes (``write_package``) the directory layout the
reference converter produces (``npu_llm/tools/convert_smollm2.py:89-119``,
``174-337``) and its loader checks (``npu_llm/runtime/model.py:12-198``):

- ``metadata.json``: shape fields, a ``tensors`` manifest, a ``files``
  manifest of ``{sha256, size}`` per file and ``metadata_sha256`` over the
  canonical JSON of everything else (sorted keys, compact separators);
- ``<name>.w8.bin`` int8 [M, K] + ``<name>.scale.f32.bin`` float32 [M] +
  ``<name>.bf16.bin`` for projections; ``<name>.<dtype>.bin`` for raw tensors.

Every manifest path must stay inside the package, every tensor file must be in
the integrity manifest and match its size and sha256, and tensor shapes must
be positive integers below 2**31 elements.  Problems raise ``RuntimeError``.

``ml_dtypes`` is not needed: bfloat16 tensors are returned as uint16 bit
patterns (``is_bf16(name)`` tells which), and ``raw_f32`` widens exactly.
"""

import hashlib
import json
import os
from pathlib import Path

import numpy as np

from runtime.bf16 import from_bits

__all__ = ["XDNA1Model", "QuantizedTensor", "write_package"]

_MAX_TENSOR_ELEMENTS = 1 << 31
_BF16 = "bfloat16"


def _safe_model_path(root, name):
    if not isinstance(name, str) or not name:
        raise RuntimeError("model manifest contains an invalid file path")
    candidate = Path(name)
    if candidate.is_absolute():
        raise RuntimeError(f"absolute model path is not allowed: {name}")
    root = Path(root).resolve()
    resolved = (root / candidate).resolve()
    try:
        resolved.relative_to(root)
    except ValueError as exc:
        raise RuntimeError(f"model path escapes package root: {name}") from exc
    return resolved


def _shape(shape, name):
    if not isinstance(shape, (list, tuple)) or not shape:
        raise RuntimeError(f"tensor {name} has an invalid shape")
    elements = 1
    dims = []
    for d in shape:
        if isinstance(d, bool) or not isinstance(d, int):
            raise RuntimeError(f"tensor {name} has a non-integer shape")
        if d <= 0:
            raise RuntimeError(f"tensor {name} has a non-positive shape")
        elements *= d
        if elements > _MAX_TENSOR_ELEMENTS:
            raise RuntimeError(f"tensor {name} is too large")
        dims.append(d)
    return tuple(dims), elements


def _np_dtype(name):
    return np.dtype(np.uint16) if name == _BF16 else np.dtype(name)


def _checked_memmap(root, name, *, dtype, shape, files):
    path = _safe_model_path(root, name)
    dtype = np.dtype(dtype)
    _, elements = _shape(list(shape), name)
    expected = elements * dtype.itemsize
    actual = path.stat().st_size
    if actual != expected:
        raise RuntimeError(f"tensor file size mismatch for {name}: expected {expected}, got {actual}")
    if files is not None and name not in files:
        raise RuntimeError(f"tensor file is missing from integrity manifest: {name}")
    return np.memmap(path, mode="r", dtype=dtype, shape=tuple(shape))


def _canonical_digest(manifest):
    canonical = dict(manifest)
    canonical.pop("metadata_sha256", None)
    return hashlib.sha256(json.dumps(canonical, separators=(",", ":"), sort_keys=True).encode()).hexdigest()


def _sha256(path):
    digest = hashlib.sha256()
    with open(path, "rb") as stream:
        for chunk in iter(lambda: stream.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


class QuantizedTensor:
    """int8 weights and per-row float32 scales (runtime/model.py:61-81)."""

    def __init__(self, root, spec, files=None):
        if not isinstance(spec, dict):
            raise RuntimeError("quantized tensor specification must be an object")
        self.shape, _ = _shape(spec.get("shape"), "quantized tensor")
        if len(self.shape) != 2:
            raise RuntimeError("quantized tensors must be rank two")
        self.weight = _checked_memmap(root, spec.get("weight"), dtype=np.int8, shape=self.shape, files=files)
        self.scale = _checked_memmap(root, spec.get("scale"), dtype=np.float32, shape=(self.shape[0],), files=files)


class XDNA1Model:
    """A verified model package (runtime/model.py:84-198)."""

    def __init__(self, model_dir):
        self.root = Path(model_dir).resolve()
        try:
            self.metadata = json.loads(_safe_model_path(self.root, "metadata.json").read_text())
        except (OSError, json.JSONDecodeError) as exc:
            raise RuntimeError("model package has invalid metadata.json") from exc
        if not isinstance(self.metadata, dict):
            raise RuntimeError("model metadata must be a JSON object")
        tensors = self.metadata.get("tensors")
        if not isinstance(tensors, dict):
            raise RuntimeError("model metadata has no tensor manifest")
        digest = self.metadata.get("metadata_sha256")
        if not isinstance(digest, str) or len(digest) != 64:
            raise RuntimeError("model package has no metadata_sha256; reconvert the model")
        if _canonical_digest(self.metadata) != digest:
            raise RuntimeError("model metadata checksum mismatch")
        self._verify_integrity()
        self.tensors = tensors

    def _verify_integrity(self):
        files = self.metadata.get("files")
        if not isinstance(files, dict) or not files:
            raise RuntimeError("model package has no integrity manifest; reconvert the model")
        for name, expected in files.items():
            path = _safe_model_path(self.root, name)
            if not isinstance(expected, dict):
                raise RuntimeError(f"invalid integrity entry: {name}")
            size, sha = expected.get("size"), expected.get("sha256")
            if (isinstance(size, bool) or not isinstance(size, int) or size < 0
                    or not isinstance(sha, str) or len(sha) != 64):
                raise RuntimeError(f"invalid integrity entry: {name}")
            if not path.is_file() or path.stat().st_size != size:
                raise RuntimeError(f"model package file is missing or truncated: {name}")
            if _sha256(path) != sha:
                raise RuntimeError(f"model package checksum mismatch: {name}")
        for tensor_name, spec in self.metadata["tensors"].items():
            if not isinstance(spec, dict):
                raise RuntimeError(f"invalid tensor specification: {tensor_name}")
            for field in ("file", "weight", "scale", "bf16_file"):
                fname = spec.get(field)
                if fname is not None and fname not in files:
                    raise RuntimeError(f"tensor file is missing from integrity manifest: {fname}")

    def quantized(self, name):
        return QuantizedTensor(self.root, self.tensors[name], self.metadata["files"])

    def bf16_projection(self, name):
        """bf16 bit patterns (uint16 memmap) of a projection."""
        spec = self.tensors[name]
        if "bf16_file" not in spec:
            raise RuntimeError(f"{name} has no BF16 weights; reconvert the model")
        shape, _ = _shape(spec.get("shape"), name)
        return _checked_memmap(self.root, spec["bf16_file"], dtype=np.uint16, shape=shape,
                               files=self.metadata["files"])

    def is_bf16(self, name):
        return self.tensors[name].get("dtype") == _BF16

    def raw(self, name):
        """Stored tensor; bfloat16 tensors come back as uint16 bits."""
        spec = self.tensors[name]
        shape, _ = _shape(spec.get("shape"), name)
        try:
            dtype = _np_dtype(spec["dtype"])
        except (KeyError, TypeError, ValueError) as exc:
            raise RuntimeError(f"tensor {name} has an invalid dtype") from exc
        return _checked_memmap(self.root, spec["file"], dtype=dtype, shape=shape, files=self.metadata["files"])

    def raw_f32(self, name):
        raw = self.raw(name)
        if self.is_bf16(name):
            return from_bits(raw)
        return np.asarray(raw, dtype=np.float32)


def write_package(model, out_dir, *, quantized=True, extra_files=None):
    """Write ``model`` (any object with the accessor surface above) as a
    package in the reference format.  Projections get bf16 files and, with
    ``quantized``, int8 + scale files.  ``extra_files`` maps file names to
    bytes (tokenizer.json and the like).  The directory is written in place
    and ``metadata.json`` last."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    manifest = {
        "format": "xdna1-qwen2-w8a16-v1" if model.metadata.get("model_family") == "qwen2"
        else "xdna1-smollm2-w8a16-v1",
        **{k: v for k, v in model.metadata.items() if k != "tensors"},
        "context_length": int(model.metadata.get("context_length", 64)),
        "tensors": {},
    }
    projections = {n for n, s in model.tensors.items() if "bf16_file" in s}
    for name in model.tensors:
        if name in projections:
            bits = np.asarray(model.bf16_projection(name), dtype=np.uint16)
            spec = {"shape": list(bits.shape), "layout": "row_major",
                    "bf16_file": f"{name}.bf16.bin", "bf16_dtype": _BF16}
            bits.tofile(out / spec["bf16_file"])
            if quantized:
                q = model.quantized(name)
                np.asarray(q.weight, np.int8).tofile(out / f"{name}.w8.bin")
                np.asarray(q.scale, np.float32).tofile(out / f"{name}.scale.f32.bin")
                spec.update({"weight": f"{name}.w8.bin", "scale": f"{name}.scale.f32.bin",
                             "weight_dtype": "int8", "scale_dtype": "float32",
                             "quantization": "symmetric_per_output_channel"})
            manifest["tensors"][name] = spec
        else:
            bf = getattr(model, "is_bf16", lambda n: False)(name)
            arr = np.asarray(model.raw(name))
            dtype = _BF16 if bf else arr.dtype.name
            fname = f"{name}.{dtype}.bin"
            arr.astype(np.uint16 if bf else arr.dtype).tofile(out / fname)
            manifest["tensors"][name] = {"file": fname, "shape": list(arr.shape), "dtype": dtype}
    for fname, data in (extra_files or {}).items():
        _safe_model_path(out, fname).write_bytes(data)
    manifest["files"] = {
        p.name: {"sha256": _sha256(p), "size": p.stat().st_size}
        for p in sorted(out.iterdir()) if p.is_file() and p.name != "metadata.json"
    }
    manifest["metadata_sha256"] = _canonical_digest(manifest)
    meta = out / "metadata.json"
    tmp = out / "metadata.json.tmp"
    tmp.write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    os.replace(tmp, meta)
    return out
