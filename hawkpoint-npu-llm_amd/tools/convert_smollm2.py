"""Convert a Hugging Face safetensors checkpoint (SmolLM2 / Qwen2) into a
model package the hk engine and the reference runtime load.

Contract of ``npu_llm/tools/convert_smollm2.py`` (callers:
``scripts/prepare_model.py:38-50`` and the command line): ``convert(model_dir,
out_dir, *, model_id=None, source_model=None, source_revision=None,
display_name=None)`` returns the manifest; ``quantize_per_output_channel``;
``_validate_architecture`` (``SMOLLM_ARCHITECTURE``, ``QWEN_ARCHITECTURE``,
``SUPPORTED_ARCHITECTURES``, ``EXPECTED_ARCHITECTURE``); ``_convert_into``.
The package (layout in ``runtime/model.py``):

- ``token_embedding``: bf16 when the checkpoint holds bf16, else float16
  (``convert_smollm2.py:218-224``); same rule for the three RMSNorm gains;
- per layer ``qkv`` = rows of q_proj, k_proj, v_proj (``:230-237``) and
  ``gate_up`` = rows of gate_proj, up_proj (``:251-257``), plus ``o_proj``
  and ``down_proj``, each as int8 + float32 row scale (the W8 quantiser,
  ``:81-86``) and as bf16; ``qkv_bias`` float32, zeros for a projection
  without a bias (``:238-250``);
- ``lm_head`` from ``lm_head.weight`` or, when tied, the embedding
  (``:309-311``);
- the tokenizer and config files copied; ``files`` and ``metadata_sha256``.

The package is built in a staging directory beside ``out_dir``, every file
is checked against its recorded size and sha256 and flushed to disk, and
only then does it replace ``out_dir`` (a failed conversion leaves the
previous package in place).

Design: safetensors files are read here directly (an 8-byte header length,
a JSON header of dtype / shape / byte range per tensor, then the data), as
read-only memory maps; bf16 tensors stay uint16 bit patterns, so neither
``ml_dtypes`` nor torch is needed.  ``any_shape=True`` accepts every shape
the GPU engine runs (64-wide heads, sizes multiple of 16) instead of only the
two shapes the reference's NPU graphs are built for.
"""

import argparse
import hashlib
import json
import os
import shutil
import sys
import tempfile
import uuid
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

from runtime.bf16 import from_bits, to_bits  # noqa: E402
from runtime.model import _canonical_digest, _sha256  # noqa: E402
from runtime.synthetic import quantize_rows  # noqa: E402

SMOLLM_ARCHITECTURE = {
    "hidden_size": 576,
    "intermediate_size": 1536,
    "num_attention_heads": 9,
    "num_key_value_heads": 3,
    "num_hidden_layers": 30,
    "vocab_size": 49152,
}
QWEN_ARCHITECTURE = {
    "hidden_size": 896,
    "intermediate_size": 4864,
    "num_attention_heads": 14,
    "num_key_value_heads": 2,
    "num_hidden_layers": 24,
    "vocab_size": 151936,
}
SUPPORTED_ARCHITECTURES = {"llama": SMOLLM_ARCHITECTURE, "qwen2": QWEN_ARCHITECTURE}
EXPECTED_ARCHITECTURE = SMOLLM_ARCHITECTURE
COPIED_FILES = ("tokenizer.json", "tokenizer_config.json", "special_tokens_map.json",
                "generation_config.json", "config.json")

# safetensors dtype -> (numpy storage dtype, is bf16 bits)
_ST_DTYPES = {
    "BF16": (np.uint16, True), "F16": (np.float16, False), "F32": (np.float32, False),
    "F64": (np.float64, False), "I8": (np.int8, False), "U8": (np.uint8, False),
    "I16": (np.int16, False), "I32": (np.int32, False), "I64": (np.int64, False),
    "BOOL": (np.bool_, False),
}


def quantize_per_output_channel(weight):
    """int8 rows with one float32 scale each: s = max(absmax / 127, tiny),
    q = clip(rint(w / s), -127, 127) (convert_smollm2.py:81-86)."""
    return quantize_rows(weight)


class SafetensorsFile:
    """Tensors of one .safetensors file, memory-mapped on access."""

    def __init__(self, path):
        self.path = Path(path)
        size = self.path.stat().st_size
        with open(self.path, "rb") as f:
            head = f.read(8)
            if len(head) != 8:
                raise ValueError(f"{self.path}: not a safetensors file")
            n = int.from_bytes(head, "little")
            if n <= 0 or 8 + n > size:
                raise ValueError(f"{self.path}: bad safetensors header length")
            header = json.loads(f.read(n))
        self._data = 8 + n
        self.entries = {}
        for name, spec in header.items():
            if name == "__metadata__":
                continue
            storage, bf16 = _ST_DTYPES[spec["dtype"]]
            shape = tuple(int(d) for d in spec["shape"])
            begin, end = (int(o) for o in spec["data_offsets"])
            if end - begin != int(np.prod(shape, dtype=np.int64)) * np.dtype(storage).itemsize or \
                    self._data + end > size or begin < 0:
                raise ValueError(f"{self.path}: tensor {name} has an inconsistent byte range")
            self.entries[name] = (storage, bf16, shape, begin)

    def tensor(self, name):
        """(array, is_bf16): bf16 tensors as uint16 bit patterns."""
        storage, bf16, shape, begin = self.entries[name]
        if 0 in shape:
            return np.zeros(shape, storage), bf16
        return np.memmap(self.path, mode="r", dtype=storage, offset=self._data + begin, shape=shape), bf16


def _source_path(model_dir, name):
    p = Path(name)
    if p.is_absolute():
        raise ValueError(f"source tensor path must be relative: {p}")
    target = (model_dir / p).resolve()
    if target != model_dir and model_dir not in target.parents:
        raise ValueError(f"source tensor path escapes model directory: {p}")
    if not target.is_file():
        raise FileNotFoundError(f"missing source tensor file: {target}")
    return target


class TensorReader:
    """Checkpoint tensors by name, over ``model.safetensors`` or the shards
    named by ``model.safetensors.index.json``."""

    def __init__(self, model_dir):
        model_dir = Path(model_dir).resolve()
        index = model_dir / "model.safetensors.index.json"
        if index.exists():
            shard_of = {k: _source_path(model_dir, v) for k, v in json.loads(index.read_text())["weight_map"].items()}
        elif (model_dir / "model.safetensors").exists():
            single = _source_path(model_dir, "model.safetensors")
            shard_of = {k: single for k in SafetensorsFile(single).entries}
        else:
            raise FileNotFoundError(f"no safetensors weights in {model_dir}")
        self._shard_of = shard_of
        self._open = {}
        self.files = shard_of

    def has(self, name):
        return name in self._shard_of

    def get(self, name):
        """(array, is_bf16) of a checkpoint tensor."""
        path = self._shard_of[name]
        if path not in self._open:
            self._open[path] = SafetensorsFile(path)
        return self._open[path].tensor(name)

    def f32(self, name):
        data, bf16 = self.get(name)
        return from_bits(data) if bf16 else np.asarray(data, dtype=np.float32)


def _validate_architecture(config, any_shape=False):
    """The package family for a HF ``config.json``; ValueError when the model
    is not one the package format and engine support."""
    family = config.get("model_type")
    expected = SUPPORTED_ARCHITECTURES.get(family)
    if expected is None:
        raise ValueError(f"unsupported model_type {family!r}; expected one of "
                         + ", ".join(sorted(SUPPORTED_ARCHITECTURES)))
    if not any_shape:
        wrong = [f"{k}={config.get(k)!r} (expected {v})" for k, v in expected.items() if config.get(k) != v]
        if wrong:
            raise ValueError("model is incompatible with the selected XDNA1 graph: " + ", ".join(wrong))
    head_dim = int(config["hidden_size"]) // int(config["num_attention_heads"])
    if head_dim != 64:
        raise ValueError(f"head_dim={head_dim} is unsupported; expected 64")
    if any_shape:
        heads, kv = int(config["num_attention_heads"]), int(config["num_key_value_heads"])
        if heads % kv or heads // kv > 16 or int(config["hidden_size"]) % 16 or \
                int(config["intermediate_size"]) % 16:
            raise ValueError("the engine needs q heads a multiple (at most 16x) of kv heads and "
                             "hidden/intermediate sizes that are multiples of 16")
    return family


class _PackageWriter:
    def __init__(self, out_dir, manifest):
        self.out = Path(out_dir)
        self.manifest = manifest

    def projection(self, name, weight_f32, bf16_bits=None):
        """int8 + scale + bf16 files of a projection [M, K]."""
        q, scale = quantize_per_output_channel(weight_f32)
        bits = to_bits(weight_f32) if bf16_bits is None else np.asarray(bf16_bits, np.uint16)
        files = {"weight": f"{name}.w8.bin", "scale": f"{name}.scale.f32.bin", "bf16_file": f"{name}.bf16.bin"}
        q.tofile(self.out / files["weight"])
        scale.tofile(self.out / files["scale"])
        bits.tofile(self.out / files["bf16_file"])
        self.manifest["tensors"][name] = {
            **files, "shape": list(q.shape), "layout": "row_major", "weight_dtype": "int8",
            "scale_dtype": "float32", "quantization": "symmetric_per_output_channel", "bf16_dtype": "bfloat16"}

    def raw(self, name, array, dtype_name):
        """A plain tensor file; ``bfloat16`` arrays are given as uint16 bits."""
        data = np.asarray(array, dtype=np.uint16 if dtype_name == "bfloat16" else dtype_name)
        fname = f"{name}.{dtype_name}.bin"
        data.tofile(self.out / fname)
        self.manifest["tensors"][name] = {"file": fname, "shape": list(data.shape), "dtype": dtype_name}

    def kept_precision(self, name, reader, source):
        """A gain or table stored as bf16 when the checkpoint has bf16, else
        float16 (the reference's rule)."""
        data, bf16 = reader.get(source)
        if bf16:
            self.raw(name, data, "bfloat16")
        else:
            self.raw(name, np.asarray(data, np.float32).astype(np.float16), "float16")
        return data, bf16


def _stacked(reader, names):
    """Rows of several projections, one after the other: float32 values and,
    when every source is bf16, the exact bf16 bits."""
    parts = [reader.get(n) for n in names]
    bits = np.concatenate([d for d, _ in parts], axis=0) if all(b for _, b in parts) else None
    values = np.concatenate([from_bits(d) if b else np.asarray(d, np.float32) for d, b in parts], axis=0)
    return values, bits


def _convert_into(model_dir, out_dir, *, model_id=None, source_model=None, source_revision=None,
                  display_name=None, any_shape=False):
    """Write the package into ``out_dir`` (existing directory) and return its manifest."""
    model_dir, out_dir = Path(model_dir), Path(out_dir)
    config = json.loads((model_dir / "config.json").read_text())
    family = _validate_architecture(config, any_shape=any_shape)
    out_dir.mkdir(parents=True, exist_ok=True)
    reader = TensorReader(model_dir)
    layers = int(config["num_hidden_layers"])
    manifest = {
        "format": "xdna1-qwen2-w8a16-v1" if family == "qwen2" else "xdna1-smollm2-w8a16-v1",
        "model_family": family,
        "hidden_size": int(config["hidden_size"]),
        "intermediate_size": int(config["intermediate_size"]),
        "attention_heads": int(config["num_attention_heads"]),
        "kv_heads": int(config["num_key_value_heads"]),
        "head_dim": int(config.get("head_dim", config["hidden_size"] // config["num_attention_heads"])),
        "layers": layers,
        "vocab_size": int(config["vocab_size"]),
        "rope_theta": float(config.get("rope_theta", 10000.0)),
        "rms_norm_eps": float(config.get("rms_norm_eps", 1e-5)),
        "context_length": 64,
        "activation_dtype": "bfloat16",
        "accumulator_dtype": "float32",
        "tensors": {},
    }
    for key, value in (("model_id", model_id), ("source_model", source_model),
                       ("source_revision", source_revision), ("display_name", display_name)):
        if value:
            manifest[key] = value
    w = _PackageWriter(out_dir, manifest)
    embed, embed_bf16 = w.kept_precision("token_embedding", reader, "model.embed_tokens.weight")
    for layer in range(layers):
        src, dst = f"model.layers.{layer}", f"layer{layer:02d}"
        attn, mlp = f"{src}.self_attn", f"{src}.mlp"
        w.projection(f"{dst}.qkv", *_stacked(reader, [f"{attn}.{p}_proj.weight" for p in "qkv"]))
        bias = [reader.f32(f"{attn}.{p}_proj.bias") if reader.has(f"{attn}.{p}_proj.bias")
                else np.zeros(reader.get(f"{attn}.{p}_proj.weight")[0].shape[0], np.float32) for p in "qkv"]
        w.raw(f"{dst}.qkv_bias", np.concatenate(bias), "float32")
        w.projection(f"{dst}.o_proj", *_stacked(reader, [f"{attn}.o_proj.weight"]))
        w.projection(f"{dst}.gate_up", *_stacked(reader, [f"{mlp}.gate_proj.weight", f"{mlp}.up_proj.weight"]))
        w.projection(f"{dst}.down_proj", *_stacked(reader, [f"{mlp}.down_proj.weight"]))
        w.kept_precision(f"{dst}.input_norm", reader, f"{src}.input_layernorm.weight")
        w.kept_precision(f"{dst}.post_attn_norm", reader, f"{src}.post_attention_layernorm.weight")
    w.kept_precision("final_norm", reader, "model.norm.weight")
    if reader.has("lm_head.weight"):
        w.projection("lm_head", *_stacked(reader, ["lm_head.weight"]))
    else:  # tied to the embedding
        w.projection("lm_head", from_bits(embed) if embed_bf16 else np.asarray(embed, np.float32),
                     embed if embed_bf16 else None)
    for name in COPIED_FILES:
        if (model_dir / name).exists():
            shutil.copyfile(model_dir / name, out_dir / name)
    manifest["files"] = {p.name: {"sha256": _sha256(p), "size": p.stat().st_size}
                         for p in sorted(out_dir.iterdir()) if p.is_file() and p.name != "metadata.json"}
    manifest["metadata_sha256"] = _canonical_digest(manifest)
    meta = out_dir / "metadata.json"
    meta.write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    with open(meta, "rb") as f:
        os.fsync(f.fileno())
    return manifest


def _sync_dir(path):
    fd = os.open(path, os.O_RDONLY | os.O_DIRECTORY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def convert(model_dir, out_dir, **metadata):
    """Build, verify and atomically publish a package at ``out_dir``."""
    model_dir, out_dir = Path(model_dir), Path(out_dir)
    out_dir.parent.mkdir(parents=True, exist_ok=True)
    staging = Path(tempfile.mkdtemp(prefix=f".{out_dir.name}.staging-", dir=out_dir.parent))
    previous = out_dir.with_name(f".{out_dir.name}.previous-{uuid.uuid4().hex}")
    try:
        manifest = _convert_into(model_dir, staging, **metadata)
        for name, entry in manifest["files"].items():
            path = staging / name
            if path.stat().st_size != entry["size"]:
                raise OSError(f"size verification failed for {name}")
            if _sha256(path) != entry["sha256"]:
                raise OSError(f"checksum verification failed for {name}")
            with open(path, "rb") as f:
                os.fsync(f.fileno())
        _sync_dir(staging)
        moved = False
        if out_dir.exists():
            os.replace(out_dir, previous)
            moved = True
        try:
            os.replace(staging, out_dir)
            _sync_dir(out_dir.parent)
        except BaseException:
            if moved:
                os.replace(previous, out_dir)
            raise
        if moved:
            shutil.rmtree(previous, ignore_errors=True)
        return manifest
    finally:
        if staging.exists():
            shutil.rmtree(staging, ignore_errors=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("model_dir", type=Path)
    ap.add_argument("output_dir", type=Path)
    ap.add_argument("--any-shape", action="store_true",
                    help="accept any shape the GPU engine runs, not only SmolLM2-135M / Qwen2.5-0.5B")
    args = ap.parse_args(argv)
    manifest = convert(args.model_dir, args.output_dir, any_shape=args.any_shape)
    print(f"Converted {manifest['layers']} layers, hidden={manifest['hidden_size']}, "
          f"vocab={manifest['vocab_size']}")


if __name__ == "__main__":
    main()
