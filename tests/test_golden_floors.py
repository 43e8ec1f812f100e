"""The summation-order fixtures under tests/golden are what their scripts
make: one cheap row of each is recomputed here from the oracle.

order_sensitivity.json holds the rel-L2 between the oracle and the oracle
with exactly rounded projections (the floor the full-depth parity bars are
scaled from); gate_order_floor.json holds the same comparison per position of
the six-prompt gate's sequences (the noise that explains an argmax miss).
"""

import json
import sys
import tempfile
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))


def test_order_sensitivity_four_layer_smollm_row_reproduces():
    from order_sensitivity import floor_for
    from runtime.synthetic import SMOLLM2_135M

    label = "smollm2-135m 4 layers, last prompt position"
    want = {row["label"]: row for row in json.loads((GOLDEN / "order_sensitivity.json").read_text())}[label]
    got = floor_for(SMOLLM2_135M, 4, want["prompt_tokens"], want["prompt_seed"], label)
    assert got["rel_l2"] > 1e-3  # the two sums do differ
    np.testing.assert_allclose(got["rel_l2"], want["rel_l2"], rtol=1e-6)


def test_gate_noise_fixture_reproduces_for_smollm_w8():
    from oracle.cpu_backend import OracleDecoder
    from order_sensitivity import ExactSumStage
    from runtime.synthetic import SMOLLM2_135M, SyntheticModel
    import test_gpu_gate as gate

    fixture = json.loads((GOLDEN / "gate_order_floor.json").read_text())["smollm-w8"]
    model = SyntheticModel(SMOLLM2_135M, seed=0, norm_gains=8.0)
    with tempfile.TemporaryDirectory() as tmp:
        sequences, _, logits = gate._sequences(model, OracleDecoder(model, gate.CONTEXT, w8=True), Path(tmp))
    assert fixture["sequences"] == [list(map(int, s)) for s in sequences]
    exact = OracleDecoder(model, gate.CONTEXT, w8=True)
    exact.stage.__class__ = ExactSumStage
    rows = exact.teacher_forced(sequences[0])
    n = len(sequences[0])
    noise = [float(np.std(logits[0][p] - rows[p])) for p in range(n)]
    np.testing.assert_allclose(noise, fixture["noise"][:n], atol=2e-6)
    gaps = [float(np.sort(logits[0][p])[-1] - np.sort(logits[0][p])[-2]) for p in range(n)]
    np.testing.assert_allclose(gaps, fixture["gap"][:n], atol=2e-5)
    # the noise is a real difference, a few percent of the logits' spread
    assert 0.01 < np.median(noise) / np.median([np.std(r) for r in logits[0]]) < 0.05
