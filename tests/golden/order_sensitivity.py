#!/usr/bin/env python3
"""Measure how far the oracle moves from itself when only the float32
summation order of its projections changes.

The oracle (a NumPy restatement of the reference's CPU runtime) is run twice
on the engine tests' inputs: once as is (BLAS sgemv sums) and once with every
projection summed exactly in float64 before the float32 -> bf16 rounding.
Both are faithful evaluations of the reference's arithmetic; their logits
differ only because bf16 rounding points flip where the two sums straddle a
rounding boundary, and the flips compound with depth.  The rel-L2 between them
is the floor below which no implementation with a different summation order
(such as the GPU's) can be held.  W8 models (int8 weights, float32 row scale)
are measured the same way, with the exact sum taken before the scale.  Output: order_sensitivity.json next to
this script.  Run time: about an hour on 8 cores (the two 4064-token rows take
~25 minutes each; the others a few minutes).
"""

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "hawkpoint-npu-llm_amd")]

import numpy as np  # noqa: E402

from oracle.bf16 import from_bits, round_f32  # noqa: E402
from oracle.cpu_backend import CPUDecoderStage, OracleDecoder  # noqa: E402
from runtime.synthetic import QWEN25_05B, SMOLLM2_135M, SyntheticModel  # noqa: E402


class ExactSumStage(CPUDecoderStage):
    """The oracle with exactly rounded (float64-accumulated) projections."""

    def project(self, name, activation):
        x = round_f32(activation).astype(np.float64)
        if self.w8 and name != "lm_head":  # W8: exact sum of q * x, then the row scale
            q = self.quantized(name)
            acc = (np.asarray(q.weight, np.float64) @ x).astype(np.float32)
            return round_f32(acc * np.asarray(q.scale, np.float32))
        return round_f32((from_bits(self.weight(name)).astype(np.float64) @ x).astype(np.float32))

    def project_rows(self, name, rows):
        x = round_f32(rows).astype(np.float64)
        if self.w8 and name != "lm_head":
            q = self.quantized(name)
            acc = (x @ np.asarray(q.weight, np.float64).T).astype(np.float32)
            return round_f32(acc * np.asarray(q.scale, np.float32))
        return round_f32((x @ from_bits(self.weight(name)).astype(np.float64).T).astype(np.float32))


def floor_for(shape, layers, prompt_len, seed, label, w8=False):
    model = SyntheticModel(shape, seed=0, layers=layers)
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, shape["vocab_size"], prompt_len)]
    a = OracleDecoder(model, prompt_len + 1, w8=w8)
    b = OracleDecoder(model, prompt_len + 1, w8=w8)
    b.stage.__class__ = ExactSumStage
    for pos, tok in enumerate(prompt):
        last = pos == prompt_len - 1
        _, la = a.decode_token(tok, pos, compute_logits=last)
        _, lb = b.decode_token(tok, pos, compute_logits=last)
    err = float(np.linalg.norm(la - lb) / np.linalg.norm(lb))
    print(f"{label}: rel-L2 {err:.4e}, argmax {int(np.argmax(la))} vs {int(np.argmax(lb))}", flush=True)
    return {"label": label, "layers": model.metadata["layers"], "prompt_tokens": prompt_len,
            "prompt_seed": seed, "w8": w8, "rel_l2": err}


def floor_long_for(shape, prompt_len, steps, seed, label, w8=False):
    """The context-4096 workload: the prompt in one batched prefill (every
    layer on all rows at once), then `steps` decode steps on the oracle's own
    greedy tokens; the largest rel-L2 over the logits of the last prompt
    position and of the decode steps."""
    model = SyntheticModel(shape, seed=0)
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, shape["vocab_size"], prompt_len)]
    a = OracleDecoder(model, prompt_len + steps + 1, w8=w8)
    b = OracleDecoder(model, prompt_len + steps + 1, w8=w8)
    b.stage.__class__ = ExactSumStage
    tok, la = a.prefill(prompt)
    _, lb = b.prefill(prompt)
    errs = [float(np.linalg.norm(la - lb) / np.linalg.norm(lb))]
    for i in range(steps):
        pos = prompt_len + i
        nxt, la = a.decode_token(tok, pos)
        _, lb = b.decode_token(tok, pos)
        errs.append(float(np.linalg.norm(la - lb) / np.linalg.norm(lb)))
        tok = nxt
    err = max(errs)
    print(f"{label}: rel-L2 max {err:.4e} over {[round(e, 5) for e in errs]}", flush=True)
    return {"label": label, "layers": model.metadata["layers"], "prompt_tokens": prompt_len,
            "prompt_seed": seed, "w8": w8, "decode_steps": steps, "rel_l2": err}


def main():
    rows = [
        floor_for(SMOLLM2_135M, None, 35, 11, "smollm2-135m full depth, last prompt position"),
        floor_for(QWEN25_05B, None, 40, 12, "qwen2.5-0.5b full depth, last prompt position"),
        floor_for(QWEN25_05B, 4, 40, 12, "qwen2.5-0.5b 4 layers, last prompt position"),
        floor_for(SMOLLM2_135M, 4, 35, 11, "smollm2-135m 4 layers, last prompt position"),
        floor_for(QWEN25_05B, None, 40, 13, "qwen2.5-0.5b W8 full depth, last prompt position", w8=True),
        floor_for(QWEN25_05B, 4, 40, 13, "qwen2.5-0.5b W8 4 layers, last prompt position", w8=True),
        floor_long_for(QWEN25_05B, 4064, 4, 31, "qwen2.5-0.5b full depth, 4064-token prefill + 4 steps"),
        floor_long_for(QWEN25_05B, 4064, 4, 31, "qwen2.5-0.5b W8 full depth, 4064-token prefill + 4 steps",
                       w8=True),
    ]
    (HERE / "order_sensitivity.json").write_text(json.dumps(rows, indent=2) + "\n")


if __name__ == "__main__":
    main()
