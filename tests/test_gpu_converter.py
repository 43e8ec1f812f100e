"""A checkpoint converted by tools/convert_smollm2.py decodes on the GPU like
the oracle: a Qwen2.5-0.5B-width model (2 layers, 4096-token vocabulary)
written under Hugging Face names as bf16 safetensors, converted into a
package, loaded by XDNA1Model, then run through the engine (bf16 and W8
projections from the package) against the oracle on the same package."""

import sys
from pathlib import Path

import numpy as np
import pytest

from runtime.model import XDNA1Model
from runtime.synthetic import QWEN25_05B, SyntheticModel
from test_converter import hf_checkpoint
from test_gpu_engine import _check_decode

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "hawkpoint-npu-llm_amd" / "tools"))
import convert_smollm2 as conv  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def package(tmp_path_factory):
    root = tmp_path_factory.mktemp("converted")
    model = SyntheticModel({**QWEN25_05B, "vocab_size": 4096}, seed=41, layers=2)
    src = hf_checkpoint(model, root / "hf", shards=2)
    conv.convert(src, root / "pkg", any_shape=True)
    return XDNA1Model(root / "pkg")


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_converted_package_decodes_like_the_oracle(package, w8):
    rng = np.random.default_rng(42)
    prompt = [int(t) for t in rng.integers(0, 4096, 24)]
    _check_decode(package, prompt, 8, 64, w8=w8, label="converted-qwen-2L")
