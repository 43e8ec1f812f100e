"""The safetensors -> package converter (hawkpoint-npu-llm_amd/tools/
convert_smollm2.py), on checkpoints written here: the reference's own
converter tests (npu_llm/tests/test_converter.py: quantiser bound,
architecture validation, atomic publish), and a round trip from a seeded
model through Hugging Face tensor names back to the loader, bit for bit.
CPU only."""

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

from runtime.bf16 import from_bits
from runtime.model import XDNA1Model
from runtime.synthetic import SyntheticModel

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "hawkpoint-npu-llm_amd" / "tools"))
import convert_smollm2 as conv  # noqa: E402

# small, with the 64-wide heads the converter requires
TINY = {"model_family": "qwen2", "hidden_size": 128, "intermediate_size": 256, "attention_heads": 2,
        "kv_heads": 1, "head_dim": 64, "layers": 2, "vocab_size": 97, "rope_theta": 1e6,
        "rms_norm_eps": 1e-6, "qkv_bias": True}

_ST_NAMES = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int8): "I8"}


def write_safetensors(path, tensors):
    """A .safetensors file from ``{name: array}``; ``(bits, "BF16")`` pairs
    are stored as bf16.  Written by hand from the format's definition."""
    header, blobs, offset = {}, [], 0
    for name, value in tensors.items():
        if isinstance(value, tuple):
            arr, dtype = np.ascontiguousarray(value[0]), value[1]
        else:
            arr = np.ascontiguousarray(value)
            dtype = _ST_NAMES[arr.dtype]
        raw = arr.tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    Path(path).write_bytes(len(text).to_bytes(8, "little") + text + b"".join(blobs))


def hf_checkpoint(model, directory, *, shards=1, bf16=True, tied=True):
    """Write ``model`` under Hugging Face names (the reverse of the reference
    converter's concatenations) with a config.json."""
    m = model.metadata
    H, I, D = m["hidden_size"], m["intermediate_size"], m["head_dim"]
    nq, nkv = m["attention_heads"], m["kv_heads"]

    def proj(name):
        bits = np.asarray(model.bf16_projection(name), np.uint16)
        return (bits, "BF16") if bf16 else from_bits(bits)

    def rows(t, a, b):
        return (t[0][a:b], "BF16") if isinstance(t, tuple) else t[a:b]

    def gain(name):
        bits = np.asarray(model.raw(name), np.uint16)
        return (bits, "BF16") if bf16 else from_bits(bits)

    tensors = {"model.embed_tokens.weight": gain("token_embedding"), "model.norm.weight": gain("final_norm")}
    for layer in range(m["layers"]):
        p, s = f"layer{layer:02d}", f"model.layers.{layer}"
        qkv = proj(f"{p}.qkv")
        bias = model.raw_f32(f"{p}.qkv_bias")
        for name, a, b in (("q", 0, nq * D), ("k", nq * D, (nq + nkv) * D), ("v", (nq + nkv) * D, (nq + 2 * nkv) * D)):
            tensors[f"{s}.self_attn.{name}_proj.weight"] = rows(qkv, a, b)
            if model.shape.get("qkv_bias"):
                tensors[f"{s}.self_attn.{name}_proj.bias"] = bias[a:b].copy()
        tensors[f"{s}.self_attn.o_proj.weight"] = proj(f"{p}.o_proj")
        gu = proj(f"{p}.gate_up")
        tensors[f"{s}.mlp.gate_proj.weight"] = rows(gu, 0, I)
        tensors[f"{s}.mlp.up_proj.weight"] = rows(gu, I, 2 * I)
        tensors[f"{s}.mlp.down_proj.weight"] = proj(f"{p}.down_proj")
        tensors[f"{s}.input_layernorm.weight"] = gain(f"{p}.input_norm")
        tensors[f"{s}.post_attention_layernorm.weight"] = gain(f"{p}.post_attn_norm")
    if not tied:
        tensors["lm_head.weight"] = proj("lm_head")
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    names = list(tensors)
    if shards == 1:
        write_safetensors(directory / "model.safetensors", tensors)
    else:
        weight_map = {}
        for k in range(shards):
            part = names[k::shards]
            fname = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(directory / fname, {n: tensors[n] for n in part})
            weight_map.update({n: fname for n in part})
        (directory / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    config = {"model_type": m["model_family"], "hidden_size": H, "intermediate_size": I,
              "num_attention_heads": nq, "num_key_value_heads": nkv, "num_hidden_layers": m["layers"],
              "vocab_size": m["vocab_size"], "rope_theta": m["rope_theta"], "rms_norm_eps": m["rms_norm_eps"]}
    (directory / "config.json").write_text(json.dumps(config))
    (directory / "tokenizer.json").write_text("{}")
    return directory


def test_per_channel_quantization_bound_of_the_reference_test():
    rng = np.random.default_rng(7)
    weight = rng.normal(0, 0.2, (32, 64)).astype(np.float32)
    q, scale = conv.quantize_per_output_channel(weight)
    assert q.dtype == np.int8 and scale.dtype == np.float32
    assert np.all(np.abs(q.astype(np.float32) * scale[:, None] - weight).max(axis=1) <= scale / 2 + 1e-6)


def test_architecture_validation():
    valid = {**conv.EXPECTED_ARCHITECTURE, "model_type": "llama"}
    assert conv._validate_architecture(valid) == "llama"
    with pytest.raises(ValueError, match="hidden_size=960"):
        conv._validate_architecture({**valid, "hidden_size": 960})
    assert conv._validate_architecture({**conv.QWEN_ARCHITECTURE, "model_type": "qwen2"}) == "qwen2"
    with pytest.raises(ValueError, match="unsupported model_type 'gpt2'"):
        conv._validate_architecture({**valid, "model_type": "gpt2"})
    # any_shape: every engine shape with 64-wide heads
    other = {**valid, "hidden_size": 960, "num_attention_heads": 15, "num_key_value_heads": 5}
    assert conv._validate_architecture(other, any_shape=True) == "llama"
    with pytest.raises(ValueError, match="head_dim=32"):
        conv._validate_architecture({**other, "num_attention_heads": 30}, any_shape=True)


def test_atomic_publish_and_failed_conversion_preserves_previous(tmp_path, monkeypatch):
    source, output = tmp_path / "source", tmp_path / "output"
    source.mkdir()
    output.mkdir()
    (output / "old.bin").write_bytes(b"old")

    def successful(_source, staging, **_):
        data = b"complete-model"
        (staging / "weights.bin").write_bytes(data)
        return {"files": {"weights.bin": {"size": len(data), "sha256": hashlib.sha256(data).hexdigest()}}}

    monkeypatch.setattr(conv, "_convert_into", successful)
    conv.convert(source, output)
    assert not (output / "old.bin").exists() and (output / "weights.bin").read_bytes() == b"complete-model"

    def failing(_source, staging, **_):
        (staging / "partial.bin").write_bytes(b"partial")
        raise OSError("simulated disk-full failure")

    monkeypatch.setattr(conv, "_convert_into", failing)
    with pytest.raises(OSError):
        conv.convert(source, output)
    assert (output / "weights.bin").read_bytes() == b"complete-model" and not (output / "partial.bin").exists()

    def corrupt(_source, staging, **_):
        (staging / "weights.bin").write_bytes(b"xx")
        return {"files": {"weights.bin": {"size": 2, "sha256": "0" * 64}}}

    monkeypatch.setattr(conv, "_convert_into", corrupt)
    with pytest.raises(OSError, match="checksum verification failed"):
        conv.convert(source, output)
    assert (output / "weights.bin").read_bytes() == b"complete-model"
    assert sorted(p.name for p in tmp_path.iterdir()) == ["output", "source"]  # no staging left


@pytest.mark.parametrize("shards,bf16,tied", [(1, True, True), (3, True, False), (2, False, True)])
def test_round_trip_through_hugging_face_names(tmp_path, shards, bf16, tied):
    """Seeded model -> HF safetensors (single file or sharded, bf16 or float32,
    tied or separate head) -> package -> loader: the q/k/v and gate/up
    concatenations, the W8 quantisation, the head and the gains come back
    exactly."""
    model = SyntheticModel(TINY, seed=8, std=0.15)
    src = hf_checkpoint(model, tmp_path / "hf", shards=shards, bf16=bf16, tied=tied)
    manifest = conv.convert(src, tmp_path / "pkg", any_shape=True, model_id="tiny")
    assert manifest["model_id"] == "tiny" and manifest["model_family"] == "qwen2"
    pkg = XDNA1Model(tmp_path / "pkg")
    for key in ("hidden_size", "intermediate_size", "attention_heads", "kv_heads", "head_dim", "layers",
                "vocab_size", "rope_theta", "rms_norm_eps"):
        assert pkg.metadata[key] == model.metadata[key], key
    for name in model.tensors:
        if "bf16_file" in model.tensors[name]:
            np.testing.assert_array_equal(pkg.bf16_projection(name), model.bf16_projection(name), err_msg=name)
            q1, q2 = pkg.quantized(name), model.quantized(name)
            np.testing.assert_array_equal(q1.weight, q2.weight, err_msg=name)
            np.testing.assert_array_equal(q1.scale, q2.scale, err_msg=name)
        elif bf16 or not (name.endswith("norm") or name == "token_embedding"):
            np.testing.assert_array_equal(pkg.raw_f32(name), model.raw_f32(name), err_msg=name)
        else:  # a float32 checkpoint's gains and table are stored as float16
            assert not pkg.is_bf16(name) and pkg.raw(name).dtype == np.float16
            np.testing.assert_array_equal(pkg.raw_f32(name), model.raw_f32(name).astype(np.float16))
    assert (tmp_path / "pkg" / "tokenizer.json").read_text() == "{}"
    assert (tmp_path / "pkg" / "config.json").is_file()


def test_missing_bias_becomes_zeros_and_bad_sources_are_rejected(tmp_path):
    model = SyntheticModel({**TINY, "qkv_bias": False}, seed=9, std=0.15)
    src = hf_checkpoint(model, tmp_path / "hf")
    conv.convert(src, tmp_path / "pkg", any_shape=True)
    pkg = XDNA1Model(tmp_path / "pkg")
    assert np.all(pkg.raw_f32("layer00.qkv_bias") == 0)
    (src / "model.safetensors").unlink()
    with pytest.raises(FileNotFoundError, match="no safetensors weights"):
        conv.convert(src, tmp_path / "pkg2", any_shape=True)
    (src / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a": "../outside.safetensors"}}))
    with pytest.raises(ValueError, match="escapes model directory"):
        conv.convert(src, tmp_path / "pkg2", any_shape=True)
    assert not (tmp_path / "pkg2").exists()
