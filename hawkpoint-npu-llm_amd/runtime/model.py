"""Model packages in the reference's on-disk format.

Reads (``XDNA1Model``) and writes (``write_package``) the directory the
reference converter produces (``npu_llm/tools/convert_smollm2.py:89-119``,
``174-337``), with the checks its loader makes (``npu_llm/runtime/model.py``):

Format (written out here as this module's specification):
- ``metadata.json``: a JSON object with the shape fields, ``tensors`` (tensor
  name -> spec object), ``files`` (file name -> ``{"size": int, "sha256": hex}``
  for every other file of the package) and ``metadata_sha256``, the sha256 of
  the canonical JSON of everything else (sorted keys, ``,`` / ``:``
  separators, no whitespace);
- a projection spec names ``weight`` (int8 [M, K]), ``scale`` (float32 [M])
  and ``bf16_file`` (bfloat16 [M, K]) with its ``shape``; a raw tensor spec
  names ``file``, ``shape`` and ``dtype`` (a NumPy dtype name or
  ``bfloat16``).

Loading verifies, in this order, and raises ``RuntimeError`` with the
reference's messages: metadata readable and an object; a tensor manifest; the
metadata digest; a non-empty file manifest whose paths stay inside the
package, whose entries are well formed and whose files have the recorded
size and sha256; every tensor spec an object whose files are all in the file
manifest.  Tensors are memory-mapped read-only on access, after their shape
(positive integers, at most 2**31 elements) and file size are checked.

``ml_dtypes`` is not needed: bfloat16 tensors come back as uint16 bit
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
_FILE_FIELDS = ("file", "weight", "scale", "bf16_file")


def _inside(root, name):
    """Absolute path of manifest entry ``name``, which must be a relative path
    that stays inside the package directory ``root``."""
    if type(name) is not str or name == "":
        raise RuntimeError("model manifest contains an invalid file path")
    if os.path.isabs(name):
        raise RuntimeError(f"absolute model path is not allowed: {name}")
    base = Path(root).resolve()
    target = base.joinpath(name).resolve()
    if target != base and base not in target.parents:
        raise RuntimeError(f"model path escapes package root: {name}")
    return target


def _dims(shape, label):
    """(shape tuple, element count) of a manifest shape."""
    if not isinstance(shape, (list, tuple)) or len(shape) == 0:
        raise RuntimeError(f"tensor {label} has an invalid shape")
    count = 1
    for d in shape:
        if type(d) is bool or not isinstance(d, int):
            raise RuntimeError(f"tensor {label} has a non-integer shape")
        if d < 1:
            raise RuntimeError(f"tensor {label} has a non-positive shape")
        count *= d
        if count > _MAX_TENSOR_ELEMENTS:
            raise RuntimeError(f"tensor {label} is too large")
    return tuple(shape), count


def _storage_dtype(name):
    return np.dtype(np.uint16) if name == _BF16 else np.dtype(name)


def _mapped(root, name, dtype, shape, files):
    """Read-only memory map of tensor file ``name`` after its checks."""
    path = _inside(root, name)
    dtype = np.dtype(dtype)
    dims, count = _dims(list(shape), name)
    want, have = count * dtype.itemsize, path.stat().st_size
    if have != want:
        raise RuntimeError(f"tensor file size mismatch for {name}: expected {want}, got {have}")
    if files is not None and name not in files:
        raise RuntimeError(f"tensor file is missing from integrity manifest: {name}")
    return np.memmap(path, mode="r", dtype=dtype, shape=dims)


def _canonical_digest(manifest):
    """sha256 of the metadata without its own digest, in canonical JSON."""
    body = {k: v for k, v in manifest.items() if k != "metadata_sha256"}
    return hashlib.sha256(json.dumps(body, separators=(",", ":"), sort_keys=True).encode()).hexdigest()


def _sha256(path):
    digest = hashlib.sha256()
    block = bytearray(4 << 20)
    view = memoryview(block)
    with open(path, "rb", buffering=0) as stream:
        while True:
            n = stream.readinto(block)
            if not n:
                return digest.hexdigest()
            digest.update(view[:n])


def _well_formed_entry(entry):
    if not isinstance(entry, dict):
        return False
    size, sha = entry.get("size"), entry.get("sha256")
    return (type(size) is int and size >= 0 and type(sha) is str and len(sha) == 64)


def _read_metadata(root):
    try:
        metadata = json.loads(_inside(root, "metadata.json").read_text())
    except (OSError, json.JSONDecodeError) as exc:
        raise RuntimeError("model package has invalid metadata.json") from exc
    if not isinstance(metadata, dict):
        raise RuntimeError("model metadata must be a JSON object")
    if not isinstance(metadata.get("tensors"), dict):
        raise RuntimeError("model metadata has no tensor manifest")
    recorded = metadata.get("metadata_sha256")
    if type(recorded) is not str or len(recorded) != 64:
        raise RuntimeError("model package has no metadata_sha256; reconvert the model")
    if _canonical_digest(metadata) != recorded:
        raise RuntimeError("model metadata checksum mismatch")
    return metadata


def _verify_files(root, metadata):
    """Check every file of the manifest against its size and sha256, then
    that every tensor's files are covered by it; returns the manifest."""
    files = metadata.get("files")
    if not isinstance(files, dict) or len(files) == 0:
        raise RuntimeError("model package has no integrity manifest; reconvert the model")
    for name, entry in files.items():
        path = _inside(root, name)
        if not _well_formed_entry(entry):
            raise RuntimeError(f"invalid integrity entry: {name}")
        if not (path.is_file() and path.stat().st_size == entry["size"]):
            raise RuntimeError(f"model package file is missing or truncated: {name}")
        if _sha256(path) != entry["sha256"]:
            raise RuntimeError(f"model package checksum mismatch: {name}")
    for tensor, spec in metadata["tensors"].items():
        if not isinstance(spec, dict):
            raise RuntimeError(f"invalid tensor specification: {tensor}")
        uncovered = [spec[f] for f in _FILE_FIELDS if spec.get(f) is not None and spec[f] not in files]
        if uncovered:
            raise RuntimeError(f"tensor file is missing from integrity manifest: {uncovered[0]}")
    return files


class QuantizedTensor:
    """int8 weights [M, K] and their float32 per-row scales [M]
    (npu_llm/runtime/model.py:61-81)."""

    def __init__(self, root, spec, files=None):
        if not isinstance(spec, dict):
            raise RuntimeError("quantized tensor specification must be an object")
        self.shape, _ = _dims(spec.get("shape"), "quantized tensor")
        if len(self.shape) != 2:
            raise RuntimeError("quantized tensors must be rank two")
        self.weight = _mapped(root, spec.get("weight"), np.int8, self.shape, files)
        self.scale = _mapped(root, spec.get("scale"), np.float32, self.shape[:1], files)


class XDNA1Model:
    """A verified model package (npu_llm/runtime/model.py:84-198)."""

    def __init__(self, model_dir):
        self.root = Path(model_dir).resolve()
        self.metadata = _read_metadata(self.root)
        self._files = _verify_files(self.root, self.metadata)
        self.tensors = self.metadata["tensors"]

    def _spec(self, name):
        return self.tensors[name]

    def quantized(self, name):
        return QuantizedTensor(self.root, self._spec(name), self._files)

    def bf16_projection(self, name):
        """bf16 bit patterns (uint16 memmap) of a projection."""
        spec = self._spec(name)
        if "bf16_file" not in spec:
            raise RuntimeError(f"{name} has no BF16 weights; rerun convert_smollm2.py")
        shape, _ = _dims(spec.get("shape"), name)
        return _mapped(self.root, spec["bf16_file"], np.uint16, shape, self._files)

    def is_bf16(self, name):
        return self._spec(name).get("dtype") == _BF16

    def raw(self, name):
        """A stored tensor; bfloat16 tensors come back as uint16 bits."""
        spec = self._spec(name)
        shape, _ = _dims(spec.get("shape"), name)
        try:
            dtype = _storage_dtype(spec["dtype"])
        except (KeyError, TypeError, ValueError) as exc:
            raise RuntimeError(f"tensor {name} has an invalid dtype") from exc
        return _mapped(self.root, spec["file"], dtype, shape, self._files)

    def raw_f32(self, name):
        """A stored tensor widened exactly to float32."""
        data = self.raw(name)
        return from_bits(data) if self.is_bf16(name) else np.asarray(data, dtype=np.float32)

    def layer(self, index):
        """One decoder layer's projections (int8 + scales) and norm gains."""
        p = f"layer{index:02d}"
        out = {k: self.quantized(f"{p}.{k}") for k in ("qkv", "o_proj", "gate_up", "down_proj")}
        out.update({k: self.raw(f"{p}.{k}") for k in ("input_norm", "post_attn_norm")})
        return out


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
        _inside(out, fname).write_bytes(data)
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
