"""Package format round trip and integrity checks (CPU only), after the
reference's tests/test_model_integrity.py and layout round-trip tests."""

import json

import numpy as np
import pytest

from runtime.model import XDNA1Model, write_package
from runtime.synthetic import SyntheticModel

TINY = {
    "model_family": "qwen2", "hidden_size": 64, "intermediate_size": 128, "attention_heads": 4,
    "kv_heads": 2, "head_dim": 16, "layers": 2, "vocab_size": 97, "rope_theta": 1e6,
    "rms_norm_eps": 1e-6, "qkv_bias": True,
}


@pytest.fixture()
def package(tmp_path):
    model = SyntheticModel(TINY, seed=4)
    write_package(model, tmp_path / "pkg", extra_files={"tokenizer.json": b"{}"})
    return model, tmp_path / "pkg"


def test_round_trip_is_bit_exact(package):
    model, path = package
    loaded = XDNA1Model(path)
    for name in model.tensors:
        if "bf16_file" in model.tensors[name]:
            np.testing.assert_array_equal(loaded.bf16_projection(name), model.bf16_projection(name))
            q1, q2 = loaded.quantized(name), model.quantized(name)
            np.testing.assert_array_equal(q1.weight, q2.weight)
            np.testing.assert_array_equal(q1.scale, q2.scale)
        else:
            np.testing.assert_array_equal(loaded.raw(name), model.raw(name))
            np.testing.assert_array_equal(loaded.raw_f32(name), model.raw_f32(name))
    for key in ("hidden_size", "layers", "vocab_size", "rope_theta", "rms_norm_eps"):
        assert loaded.metadata[key] == model.metadata[key]


def test_tampered_file_is_rejected(package):
    _, path = package
    f = path / "layer00.o_proj.bf16.bin"
    data = bytearray(f.read_bytes())
    data[10] ^= 1
    f.write_bytes(bytes(data))
    with pytest.raises(RuntimeError, match="checksum mismatch"):
        XDNA1Model(path)


def test_tampered_metadata_is_rejected(package):
    _, path = package
    meta = json.loads((path / "metadata.json").read_text())
    meta["layers"] = 3
    (path / "metadata.json").write_text(json.dumps(meta))
    with pytest.raises(RuntimeError, match="metadata checksum"):
        XDNA1Model(path)


def test_path_traversal_is_rejected(package):
    from runtime.model import _canonical_digest

    _, path = package
    meta = json.loads((path / "metadata.json").read_text())
    meta["files"]["../escape.bin"] = {"sha256": "0" * 64, "size": 0}
    meta["metadata_sha256"] = _canonical_digest(meta)
    (path / "metadata.json").write_text(json.dumps(meta))
    with pytest.raises(RuntimeError, match="escapes package root"):
        XDNA1Model(path)


def test_truncated_file_is_rejected(package):
    _, path = package
    f = path / "final_norm.bfloat16.bin"
    f.write_bytes(f.read_bytes()[:-2])
    with pytest.raises(RuntimeError, match="missing or truncated"):
        XDNA1Model(path)
