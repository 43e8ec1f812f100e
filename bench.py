#!/usr/bin/env python3
"""Batch-1 greedy decode benchmark on one MI355X.

Workload: the Qwen2.5-0.5B-shaped decoder (24 layers, hidden 896, 14/2 heads,
SwiGLU 4864, vocab 151936, tied bf16 LM head, qkv bias) with seeded random
N(0, 0.02) bf16 weights.  A 40-token random prompt is prefilled position by
position (the reference's prefill, npu_llm/runtime/generate.py:1110-1125,
timed as per_position_ms) and in one batched chunk (the TTFT); greedy
decode then runs in 31-step runs at positions 40..70, each continuing from
the batched prefill's KV cache, i.e. 32 tokens per run with the prefill's
token, the reference's "40-token prompt, 32 tokens" protocol.  One step = one decode token: every layer, the final norm,
the LM head and the argmax, with weights and KV resident in HBM.

value = timed steps / wall seconds between two stream synchronisations, the
median of --runs (default 5) timed runs of --steps steps each.
roofline: the decode-step kernel -- one persistent launch runs the whole step
(all 24 layers, the LM head and the argmax) -- timed with HIP events on the
engine's stream over a graph of back-to-back step launches; achieved = the
step's algorithmic bytes (988 MB of weights plus KV) / its duration, against
the MI355X's 8 TB/s HBM peak.  The per-kernel path (one GEMV or attention
kernel per part, used for int8 weights and other shapes) is timed too.
cpu_baseline: the oracle (NumPy BF16 CPU restatement of the reference's CPU
runtime) on a bounded sample of the same workload, with every host core and
with one BLAS thread.
smollm2_135m: the SmolLM2-135M-shaped decoder's decode tok/s and step-kernel
roofline (35-token prompt, 16 greedy tokens, 64-slot context).

Other workloads (each prints its own JSON line): --workload experts (the
GGML / Colibri expert shims), gemv (the isolated batch-1 GEMVs at the
Qwen2.5-0.5B projection shapes, bf16 and W8, for kernel traces), prefill
(batched prefill of 40- and 4064-token prompts, for kernel traces), moe
(the routed-expert block at 1..16 tokens, against the HBM roofline).
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "hawkpoint-npu-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "decode tok/s @batch1 + HBM GB/s (% peak), Qwen2.5-0.5B-shape bf16"
HBM_PEAK_GBS = 8000.0
BF16_PEAK = 2.5e15  # MI355X dense bf16 matrix peak, FLOP/s
PROMPT = 40
RUN = 31  # decode steps per run after the prefill token (positions 40..70)
REFERENCE_TOKS = 28.83  # XDNA1 Qwen2.5-0.5B engine decode (reference README.md:92)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def step_bytes(meta, position, bias=True):
    """Algorithmic HBM bytes of one decode step at `position`: every weight
    once (bf16), the qkv bias (when the model has one), norm gains, the
    embedding row, KV read for slots 0..position and the new slot written."""
    h, i = meta["hidden_size"], meta["intermediate_size"]
    nq, nkv, d = meta["attention_heads"], meta["kv_heads"], meta["head_dim"]
    qkv = (nq + 2 * nkv) * d
    per_layer = 2 * (qkv * h + h * nq * d + 2 * i * h + h * i) + (4 * qkv if bias else 0) + 2 * 2 * h
    head = 2 * meta["vocab_size"] * h + 2 * h
    kv_slot = meta["layers"] * 2 * nkv * d * 2
    return meta["layers"] * per_layer + head + 2 * h + kv_slot * (position + 1) + kv_slot


def w8_step_bytes(meta, position):
    """Algorithmic HBM bytes of one W8 decode step: int8 layer projections
    with a float32 scale per output row, the bf16 LM head, qkv bias, norm
    gains, the embedding row and the KV traffic of ``step_bytes``."""
    h, i = meta["hidden_size"], meta["intermediate_size"]
    nq, nkv, d = meta["attention_heads"], meta["kv_heads"], meta["head_dim"]
    qkv = (nq + 2 * nkv) * d
    rows = qkv + h + 2 * i + h
    per_layer = (qkv * h + h * nq * d + 2 * i * h + h * i) + 4 * rows + 4 * qkv + 2 * 2 * h
    head = 2 * meta["vocab_size"] * h + 2 * h
    kv_slot = meta["layers"] * 2 * nkv * d * 2
    return meta["layers"] * per_layer + head + 2 * h + kv_slot * (position + 1) + kv_slot


def layer_params(meta):
    """Projection weights that every token multiplies (all layers, no head)."""
    h, i = meta["hidden_size"], meta["intermediate_size"]
    nq, nkv, d = meta["attention_heads"], meta["kv_heads"], meta["head_dim"]
    return meta["layers"] * ((nq + 2 * nkv) * d * h + h * nq * d + 2 * i * h + h * i)


def part_bytes(meta, part):
    h, i = meta["hidden_size"], meta["intermediate_size"]
    nq, nkv, d = meta["attention_heads"], meta["kv_heads"], meta["head_dim"]
    qkv = (nq + 2 * nkv) * d
    return {
        "qkv": 2 * qkv * h + 2 * h + 2 * h + 4 * qkv + 2 * qkv,
        "o_proj": 2 * h * nq * d + 2 * nq * d + 2 * h + 2 * h,
        "gate_up": 2 * 2 * i * h + 2 * h + 2 * h + 2 * i,
        "down_proj": 2 * h * i + 2 * i + 2 * h + 2 * h,
        "lm_head": 2 * meta["vocab_size"] * h + 2 * h + 2 * h + 4 * meta["vocab_size"],
    }.get(part)


def _blas_info():
    from threadpoolctl import threadpool_info

    blas = [t for t in threadpool_info() if t.get("user_api") == "blas"]
    return {"library": blas[0].get("internal_api") if blas else None,
            "version": blas[0].get("version") if blas else None,
            "threads": blas[0].get("num_threads") if blas else None}


def cpu_baseline(model, prompt, steps_all, steps_one):
    """Oracle decode tok/s on the host cores: the prompt through the oracle's
    batched prefill (untimed), one untimed decode step (it widens the LM head
    to float32 once, as the reference caches it), then timed greedy steps,
    first with every BLAS thread, then with one.  Decode tok/s = steps /
    their seconds (the reference's definition, generate.py:1167-1188)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle.cpu_backend import OracleDecoder

    n = len(prompt)
    oracle = OracleDecoder(model, n + max(steps_all, steps_one) + 2)
    first, _ = oracle.prefill(prompt)
    tok, _ = oracle.decode_token(first, n)

    def timed_steps(count):
        t, total = tok, 0.0
        for k in range(count):
            t0 = time.perf_counter()
            t, _ = oracle.decode_token(t, n + 1 + k)
            total += time.perf_counter() - t0
        return count / total

    blas = _blas_info()
    all_cores = timed_steps(steps_all)
    with threadpool_limits(limits=1):
        one = timed_steps(steps_one)
    host = {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "blas": blas["library"], "blas_version": blas["version"],
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS"),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"), "numpy": np.__version__}
    return {
        "value": round(all_cores, 3),
        "unit": "tok/s",
        "cores": blas["threads"],
        "kind": "port",
        "sample": f"{n}-token prompt (oracle batched prefill, untimed) and one untimed step, then "
        f"{steps_all} timed greedy decode steps of the same model; NumPy float32 BLAS with "
        f"{blas['threads']} threads",
        "one_thread": {"value": round(one, 3), "unit": "tok/s", "cores": 1,
                       "sample": f"the same after the prompt, {steps_one} timed steps, one BLAS thread"},
        "host": host,
    }


COPY_BYTES = 256 << 20
GEMV_SHAPES = [  # (name, M, K): Qwen2.5-0.5B projections
    ("qkv", 1152, 896), ("o_proj", 896, 896), ("gate_up", 9728, 896), ("down_proj", 896, 4864),
    ("lm_head", 151936, 896)]
ROTATE_BYTES = 512 << 20


def gemv_microbench(launches=200):
    """Isolated batch-1 GEMVs at the Qwen2.5-0.5B projection shapes, bf16 and
    W8 (int8 + per-row scale) weights, float32 output.  Each shape rotates
    through enough distinct weight copies to exceed 512 MiB, so the 256 MB
    Infinity Cache cannot serve them; timed with HIP events around one graph
    replay of the launches (directly enqueued, each launch would cost the
    host about as long as the kernel runs).  Bytes per launch = weights
    (+ scales) + x + y."""
    import ctypes

    import numpy as np

    from runtime import hip
    from runtime.bf16 import to_bits
    from runtime.synthetic import quantize_rows

    lib = hip.lib()
    rng = np.random.default_rng(2)
    out = {}
    for name, m, k in GEMV_SHAPES:
        w = rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02)
        x = hip.DeviceBuffer.from_array(to_bits(rng.standard_normal(k, dtype=np.float32)))
        y = hip.DeviceBuffer(4 * m)
        for dtype in ("bf16", "w8"):
            if dtype == "bf16":
                data, scale = to_bits(w), None
            else:
                data, scale = quantize_rows(from_bf16(to_bits(w)))
            wbytes = data.nbytes
            copies = max(2, -(-ROTATE_BYTES // wbytes))
            # the copies sit 4 KiB-aligned in one allocation, so every shape
            # sees the same page mapping (separate allocations of a few
            # hundred KB each timed up to 2x apart from run to run)
            stride = -(-wbytes // 4096) * 4096
            first = hip.DeviceBuffer.from_array(data)
            pool = hip.DeviceBuffer(stride * copies)
            for i in range(copies):
                hip.check(lib.hk_memcpy_d2d(pool.ptr + i * stride, first.ptr, wbytes), "copy")
            bufs = [first, pool]
            ptrs = (ctypes.c_void_p * copies)(*[pool.ptr + i * stride for i in range(copies)])
            sbuf = hip.DeviceBuffer.from_array(scale) if scale is not None else None
            sptrs = (ctypes.c_void_p * copies)(*([sbuf.ptr] * copies)) if sbuf else None
            ev0, ev1 = hip.Event(), hip.Event()
            # two warm rotations: every copy's pages have been touched by a
            # launch before the timed ones
            hip.check(lib.hk_gemv_repeat(ptrs, sptrs, copies, x.ptr, y.ptr, m, k, 2 * copies, None), "warm")
            # the timed call replays the graph this untimed one captures
            hip.check(lib.hk_gemv_repeat(ptrs, sptrs, copies, x.ptr, y.ptr, m, k, launches, None), "capture")
            ev0.record(None)
            hip.check(lib.hk_gemv_repeat(ptrs, sptrs, copies, x.ptr, y.ptr, m, k, launches, None), "gemv")
            ev1.record(None)
            us = ev0.elapsed_ms(ev1) * 1e3 / launches
            nbytes = wbytes + (4 * m if scale is not None else 0) + 2 * k + 4 * m
            out[f"{name}_{dtype}"] = {"M": m, "K": k, "us": round(us, 3), "bytes": nbytes,
                                      "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                                      "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                      "rotated_copies": copies}
            for b in bufs:
                b.free()
    return out


def from_bf16(bits):
    from runtime.bf16 import from_bits

    return from_bits(bits)


def probe(engine, meta, launches, position):
    """Workload for the rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE): the
    decode-step kernel, launched one step at a time at the last decode
    position, and, as the calibration of the counters, device-to-device copies
    of a known size (256 MiB read + 256 MiB written per copy)."""
    from runtime import hip

    lib = hip.lib()
    for _ in range(launches):
        hip.check(lib.hk_engine_launch_part(engine._engine, hip.PART_STEP, 0), "launch")
    hip.check(lib.hk_stream_sync(engine.stream), "sync")
    src, dst = hip.DeviceBuffer(COPY_BYTES), hip.DeviceBuffer(COPY_BYTES)
    src.zero()
    for _ in range(4):
        hip.check(lib.hk_memcpy_d2d(dst.ptr, src.ptr, COPY_BYTES), "copy")
    print(json.dumps({"probe": "decode_step", "launches": launches, "position": position,
                      "bytes_per_launch": step_bytes(meta, position), "copy_bytes": COPY_BYTES}))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3100)
    ap.add_argument("--warmup", type=int, default=310)
    ap.add_argument("--runs", type=int, default=5, help="timed runs of --steps steps; value is the median")
    ap.add_argument("--kernel-launches", type=int, default=240)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-microbench", action="store_true")
    ap.add_argument("--no-parts", action="store_true",
                    help="skip the per-kernel path timing, which replays hipGraphs (for profiler runs)")
    ap.add_argument("--cpu-steps", type=int, default=16)
    ap.add_argument("--cpu-steps-one-thread", type=int, default=4)
    ap.add_argument("--no-smollm", action="store_true", help="skip the SmolLM2-135M decode line")
    ap.add_argument("--workload", choices=("decode", "experts", "gemv", "prefill", "phases", "moe"),
                    default="decode",
                    help="experts: the GGML MUL_MAT_ID / Colibri expert-group shims; gemv: the isolated "
                    "GEMVs; prefill: batched prefills of 40 and 4064 tokens; phases: the per-layer phase "
                    "table of the decode step from lib/libhk_phases.so; moe: the routed-expert block "
                    "(H 2048, 64 + 2 experts of I 1408, top-6) at 1..16 tokens (each prints its own JSON line)")
    ap.add_argument("--phases-model", choices=("qwen", "qwen-w8", "smollm"), default="qwen",
                    help="phases: the decoder whose step is stamped")
    ap.add_argument("--phases-long", action="store_true",
                    help="phases: a 4064-token prompt, decode at positions 4064..4094 (the long form)")
    ap.add_argument("--probe", action="store_true",
                    help="only the counter-calibration workload: decode-step launches, then "
                    "4 device copies of 256 MiB")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the engine runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "experts":
        experts_main(args)
        return
    if args.workload == "gemv":
        gemv_main(args)
        return
    if args.workload == "prefill":
        prefill_main(args)
        return
    if args.workload == "phases":
        phases_main(args)
        return
    if args.workload == "moe":
        moe_main(args)
        return

    import numpy as np

    from runtime import hip
    from runtime.qwen_engine import QwenDecoderEngine
    from runtime.synthetic import QWEN25_05B, SyntheticModel

    log("building the synthetic Qwen2.5-0.5B-shape model")
    model = SyntheticModel(QWEN25_05B, seed=0)
    meta = model.metadata
    rng = np.random.default_rng(12)
    prompt = [int(t) for t in rng.integers(0, meta["vocab_size"], PROMPT)]
    engine = QwenDecoderEngine(model, context_length=4096)
    lib = hip.lib()

    def prefill_per_position():
        for pos, tok in enumerate(prompt[:-1]):
            engine.step_token(tok, pos, logits=False)
        first, _ = engine.step_token(prompt[-1], PROMPT - 1, logits=True, want_logits_array=False)
        return first

    def timed(fn, reps=5, warm=0):
        # median wall time of `reps` calls after `warm` untimed ones
        for _ in range(warm):
            fn()
        times, out = [], None
        for _ in range(reps):
            t0 = time.perf_counter()
            out = fn()
            times.append(time.perf_counter() - t0)
        return out, sorted(times)[len(times) // 2]

    first = prefill_per_position()  # captures both graphs
    if args.probe:
        probe(engine, meta, args.kernel_launches, PROMPT - 1)
        return
    first_pp, ttft_pp = timed(prefill_per_position, 3)
    first, ttft = timed(lambda: engine.prefill(prompt, 0, want_logits_array=False)[0], 20, 2)
    if first != first_pp:
        log(f"note: batched and per-position prefill pick {first} / {first_pp} (near-tie)")
    prefill_flops = 2.0 * PROMPT * layer_params(meta)
    log(f"prefill {PROMPT} tokens: TTFT batched {ttft * 1e3:.2f} ms, per position "
        f"{ttft_pp * 1e3:.2f} ms, first token {first}")

    def decode(n):
        tokens = []
        while n > 0:
            k = min(RUN, n)
            tokens = engine.generate(first, PROMPT, k)
            n -= k
        return tokens

    decode(args.warmup)
    run_tok_s = []
    for _ in range(max(1, args.runs)):
        hip.check(lib.hk_stream_sync(engine.stream), "sync")
        t0 = time.perf_counter()
        decode(args.steps)
        hip.check(lib.hk_stream_sync(engine.stream), "sync")
        run_tok_s.append(args.steps / (time.perf_counter() - t0))
    tok_s = sorted(run_tok_s)[len(run_tok_s) // 2]
    ms_step = 1e3 / tok_s
    last_pos = PROMPT + min(args.steps, RUN) - 1  # the positions a run covers: PROMPT .. last_pos
    mean_pos = (PROMPT + last_pos) / 2.0
    step_gbs = step_bytes(meta, mean_pos) / (ms_step * 1e-3) / 1e9
    log(f"decode: {tok_s:.1f} tok/s (median of {len(run_tok_s)} runs: "
        f"{', '.join(f'{v:.0f}' for v in run_tok_s)}), {ms_step * 1e3:.1f} us/step, {step_gbs:.0f} GB/s whole step")

    stream = engine.stream
    end_pos = PROMPT + RUN  # ctrl position after the last timed run
    # the decode-step kernel: a graph of back-to-back step launches at the
    # last position (no token feedback), timed with HIP events on its stream
    n = args.kernel_launches
    # (a persistent step is repeated as direct launches, no graph)
    ev0, ev1 = hip.Event(), hip.Event()
    hip.check(lib.hk_engine_launch_part_repeat(engine._engine, hip.PART_STEP, n), "step repeat")
    ev0.record(stream)
    hip.check(lib.hk_engine_launch_part_repeat(engine._engine, hip.PART_STEP, n), "step repeat")
    ev1.record(stream)
    step_kernel_us = ev0.elapsed_ms(ev1) * 1e3 / n
    dom_bytes = step_bytes(meta, end_pos)
    achieved = dom_bytes / (step_kernel_us * 1e-6) / 1e9
    log(f"decode-step kernel: {step_kernel_us:.1f} us/launch, {achieved:.0f} GB/s")

    # the per-kernel path, part by part (graph of launches over all layers)
    parts = {}
    layers = meta["layers"]
    if not args.no_parts:
        for name, part in hip.PARTS.items():
            e0, e1 = hip.Event(), hip.Event()
            hip.check(lib.hk_engine_launch_part_repeat(engine._engine, part, n), "launch_part_repeat")
            e0.record(stream)
            hip.check(lib.hk_engine_launch_part_repeat(engine._engine, part, n), "launch_part_repeat")
            e1.record(stream)
            parts[name] = e0.elapsed_ms(e1) * 1e3 / n
        log("per-kernel path us/launch: " + ", ".join(f"{k} {v:.2f}" for k, v in parts.items()))

    # context 4096: a 4064-token prompt in one batched prefill, then 31 greedy
    # decode steps at positions 4064..4094
    long_n = 4064
    long_prompt = [int(t) for t in rng.integers(0, meta["vocab_size"], long_n)]
    # (median of three after one untimed prefill: successive prefills of this
    # length in one process measured 8.4, 8.1 and 7.9 ms on one box)
    tok_long, t_long = timed(lambda: engine.prefill(long_prompt, 0, want_logits_array=False)[0], 3, 1)
    attn_flops = 4.0 * meta["attention_heads"] * meta["head_dim"] * meta["layers"] * long_n * (long_n + 1) / 2
    long_flops = 2.0 * long_n * layer_params(meta) + attn_flops
    hip.check(lib.hk_stream_sync(engine.stream), "sync")
    t0 = time.perf_counter()
    engine.generate(tok_long, long_n, RUN)
    long_decode = RUN / (time.perf_counter() - t0)
    log(f"ctx 4096: prefill {long_n} tokens {t_long * 1e3:.1f} ms "
        f"({long_flops / t_long / 1e12:.1f} TFLOP/s), decode {long_decode:.1f} tok/s")
    # which step kernel ran at the timed positions (both share one contract)
    split = engine.step_kind(end_pos) == "xcd_split"
    engine.close()

    # the W8 decoder: int8 layer projections with per-row float32 scales and
    # the bf16 LM head; the same 40-token prompt in one batched prefill, then
    # 31 greedy steps (32 tokens), median of 5 runs
    log("building the W8 engine (per-row int8 quantisation of the same weights)")
    w8 = QwenDecoderEngine(model, context_length=4096, w8=True)
    w8_first, w8_ttft = timed(lambda: w8.prefill(prompt, 0, want_logits_array=False)[0], 20, 2)
    w8.generate(w8_first, PROMPT, RUN)  # captures the step graph
    w8_runs = []
    for _ in range(5):
        hip.check(lib.hk_stream_sync(w8.stream), "sync")
        t0 = time.perf_counter()
        w8.generate(w8_first, PROMPT, RUN)
        w8_runs.append(RUN / (time.perf_counter() - t0))
    w8_tok_s = sorted(w8_runs)[len(w8_runs) // 2]
    w8_kind = w8.step_kind(PROMPT)
    w8_kernel_us = None
    if True:  # the W8 step kernel alone, as for the bf16 one above
        ev0, ev1 = hip.Event(), hip.Event()
        hip.check(lib.hk_engine_launch_part_repeat(w8._engine, hip.PART_STEP, n), "W8 step repeat")
        ev0.record(w8.stream)
        hip.check(lib.hk_engine_launch_part_repeat(w8._engine, hip.PART_STEP, n), "W8 step repeat")
        ev1.record(w8.stream)
        w8_kernel_us = ev0.elapsed_ms(ev1) * 1e3 / n
    w8.close()
    w8_gbs = w8_step_bytes(meta, mean_pos) * w8_tok_s / 1e9
    log(f"W8 decode: {w8_tok_s:.1f} tok/s ({w8_kind} step), {w8_gbs:.0f} GB/s whole step, "
        f"TTFT {w8_ttft * 1e3:.2f} ms, step kernel {w8_kernel_us} us")
    if split:
        kernel_name = "decode_step_xa_kernel (attention block on XCD 0, MLP on XCDs 1-7)"
        tfile = ROOT / "profiles" / "traffic_decode_step_xcd_split_qwen05b.json"
    else:
        kernel_name = "decode_step_kernel"
        tfile = ROOT / "profiles" / "traffic_decode_step_qwen05b.json"
    traffic = None
    if tfile.is_file():
        # HBM bytes per launch from the committed rocprofv3 --pmc runs
        traffic = json.loads(tfile.read_text()).get("traffic_bytes_per_launch")

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "runs": [round(v, 2) for v in run_tok_s],
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tok_s / REFERENCE_TOKS, 2),
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-0.5B-shape decoder (24L, H896, 14q/2kv heads, I4864, V151936, "
            "tied head, qkv bias), seeded N(0,0.02) bf16 weights, batch 1, 40-token random prompt "
            f"prefilled in one batched chunk, greedy decode from position 40 in runs of up to {RUN} steps "
            f"continuing from that KV cache; value = median of {len(run_tok_s)} timed runs",
            "batch": 1,
            "prompt_tokens": PROMPT,
            "decode_positions": [PROMPT, last_pos],
            "kv_slots_allocated": 4096,
        },
        "ttft_ms": round(ttft * 1e3, 3),
        "prefill": {
            "tokens": PROMPT,
            "batched_ms": round(ttft * 1e3, 3),
            "per_position_ms": round(ttft_pp * 1e3, 3),
            "mfma_tflops": round(prefill_flops / ttft / 1e12, 3),
            "mfma_frac_of_bf16_dense": round(prefill_flops / ttft / BF16_PEAK, 5),
        },
        "long_context": {
            "prompt_tokens": long_n,
            "prefill_ms": round(t_long * 1e3, 2),
            "prefill_tflops": round(long_flops / t_long / 1e12, 2),
            "prefill_mfma_frac_of_bf16_dense": round(long_flops / t_long / BF16_PEAK, 4),
            "decode_tok_s": round(long_decode, 1),
            "decode_positions": [long_n, long_n + RUN - 1],
        },
        "w8_decode": {
            "workload": "the same decoder with W8 layer projections (int8, per-output-row float32 "
            "scale), bf16 activations, KV cache and LM head; 40-token prompt, 32 greedy tokens",
            "tok_s": round(w8_tok_s, 1),
            "step": w8_kind,
            "ttft_ms": round(w8_ttft * 1e3, 3),
            "step_bytes": int(w8_step_bytes(meta, mean_pos)),
            "step_hbm_gbs": round(w8_gbs, 1),
            "step_hbm_frac": round(w8_gbs / HBM_PEAK_GBS, 4),
            "step_kernel_us": None if w8_kernel_us is None else round(w8_kernel_us, 2),
            "step_kernel_gbs": None if w8_kernel_us is None else
            round(w8_step_bytes(meta, end_pos) / (w8_kernel_us * 1e-6) / 1e9, 1),
        },
        "step_hbm_gbs": round(step_gbs, 1),
        "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "step_bytes": int(step_bytes(meta, mean_pos)),
        "step_kernel_us": round(step_kernel_us, 2),
        "per_kernel_path_us": {k: round(v, 3) for k, v in parts.items()},
        "roofline": {
            "bound": "hbm",
            "kernel": f"{kernel_name}, one launch per token (bytes/launch {dom_bytes} at "
            f"position {end_pos})",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "baseline_source": "28.83 tok/s, XDNA1 NPU Qwen2.5-0.5B engine (reference README.md:92)",
    }
    if not args.no_microbench:
        log("GEMV microbench (512 MiB rotation)")
        result["gemv_microbench"] = gemv_microbench()
        log(" ".join(f"{k}:{v['gbs']:.0f}GB/s" for k, v in result["gemv_microbench"].items()))
    if not args.no_smollm:
        log("SmolLM2-135M shape")
        result["smollm2_135m"] = smollm_decode(args)
    if not args.no_cpu_baseline:
        log("timing the CPU oracle")
        result["cpu_baseline"] = cpu_baseline(model, prompt, args.cpu_steps, args.cpu_steps_one_thread)
    print(json.dumps(result), flush=True)


def smollm_decode(args, runs=5):
    """SmolLM2-135M-shaped decoder (30 layers, H576, 9/3 heads, I1536,
    V49152, tied head, no qkv bias), seeded N(0,0.02) bf16 weights: a
    35-token prompt in one batched prefill, then 15 greedy steps (16 tokens)
    at positions 35..49 in a 64-slot context, median of `runs` runs; and the
    step kernel alone (direct launches at position 50, HIP events)."""
    import numpy as np

    from runtime import hip
    from runtime.qwen_engine import QwenDecoderEngine
    from runtime.synthetic import SMOLLM2_135M, SyntheticModel

    lib = hip.lib()
    model = SyntheticModel(SMOLLM2_135M, seed=0)
    meta = model.metadata
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, meta["vocab_size"], 35)]
    engine = QwenDecoderEngine(model, context_length=64)
    try:
        first, _ = engine.prefill(prompt, want_logits_array=False)
        engine.generate(first, 35, 15)
        rates = []
        for _ in range(runs):
            hip.check(lib.hk_stream_sync(engine.stream), "sync")
            t0 = time.perf_counter()
            engine.generate(first, 35, 15)
            rates.append(15 / (time.perf_counter() - t0))
        n = args.kernel_launches
        ev0, ev1 = hip.Event(), hip.Event()
        hip.check(lib.hk_engine_launch_part_repeat(engine._engine, hip.PART_STEP, n), "step repeat")
        ev0.record(engine.stream)
        hip.check(lib.hk_engine_launch_part_repeat(engine._engine, hip.PART_STEP, n), "step repeat")
        ev1.record(engine.stream)
        us = ev0.elapsed_ms(ev1) * 1e3 / n
        kind = engine.step_kind(50)
    finally:
        engine.close()
    nbytes = step_bytes(meta, 50, bias=False)
    gbs = nbytes / (us * 1e-6) / 1e9
    tok_s = sorted(rates)[len(rates) // 2]
    log(f"SmolLM2-135M: {tok_s:.1f} tok/s ({kind} step), step kernel {us:.1f} us, {gbs:.0f} GB/s")
    return {"workload": "SmolLM2-135M-shape decoder, seeded N(0,0.02) bf16 weights, 35-token prompt "
            "(batched prefill), 16 greedy tokens (15 decode steps at positions 35..49), 64-slot context",
            "tok_s": round(tok_s, 1), "runs": [round(v, 1) for v in rates], "step": kind,
            "step_kernel_us": round(us, 2), "step_bytes": int(nbytes),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "note": "269 MB per step: the weights fit the 256 MB Infinity Cache almost whole"}}


def gemv_main(args):
    """Only the isolated GEMV microbench (for kernel traces of its launches)."""
    from runtime import hip

    hip.init(0)
    out = gemv_microbench()
    print(json.dumps({"workload": "gemv", "gemv_microbench": out}), flush=True)


def phases_main(args):
    """Per-layer phase table of the XCD-split decode step, from the clock
    stamps that lib/libhk_phases.so (persistent.hip built with
    -DHK_PHASE_STAMPS) writes at fixed points of each layer: a prompt
    prefilled in one batch, two untimed 31-step runs, then the stamps of one
    more run's last launch (position prompt + 30).  Each segment is the mean
    over layers 1..L-2 of one phase's span, from the last producer of its
    input (the maximum over workgroups) to the median or last consumer."""
    import ctypes

    import numpy as np

    lib_path = ROOT / "hawkpoint-npu-llm_amd" / "lib" / "libhk_phases.so"
    if not lib_path.is_file():
        raise SystemExit(f"{lib_path} not found: build it with `python hawkpoint-npu-llm_amd/csrc/build.py`")
    os.environ["HK_LIB"] = str(lib_path)
    from runtime import hip
    from runtime.qwen_engine import QwenDecoderEngine
    from runtime.synthetic import QWEN25_05B, SMOLLM2_135M, SyntheticModel

    shape = SMOLLM2_135M if args.phases_model == "smollm" else QWEN25_05B
    model = SyntheticModel(shape, seed=0)
    meta = model.metadata
    n = 4064 if args.phases_long else (35 if args.phases_model == "smollm" else PROMPT)
    rng = np.random.default_rng(12)
    prompt = [int(t) for t in rng.integers(0, meta["vocab_size"], n)]
    engine = QwenDecoderEngine(model, context_length=4096, w8=args.phases_model == "qwen-w8")
    lib = hip.lib()
    lib.hk_phase_stamps.restype = ctypes.c_int
    lib.hk_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    ph = np.zeros((256, 32, 16), dtype=np.uint64)
    at = np.zeros((256, 32, 8), dtype=np.uint64)
    try:
        first, _ = engine.prefill(prompt, want_logits_array=False)
        steps = min(RUN, 4095 - n)
        kind = engine.step_kind(n + steps - 1)
        engine.generate(first, n, steps)
        engine.generate(first, n, steps)
        hip.check(lib.hk_phase_stamps(None, None, 1), "clear stamps")
        engine.generate(first, n, steps)
        hip.check(lib.hk_phase_stamps(ph.ctypes.data, at.ctypes.data, 0), "read stamps")
    finally:
        engine.close()
    T = ph.astype(np.int64) * 10  # 100 MHz clock, ns
    A = at.astype(np.int64) * 10
    L = min(meta["layers"], 32)
    wg = np.arange(256)
    x0 = wg % 8 == 0

    def sel(layer, slot, mask=None):
        v = T[:, layer, slot]
        m = v > 0
        if mask is not None:
            m &= mask
        return v[m]

    def med(layer, slot, mask=None):
        v = sel(layer, slot, mask)
        return float(np.median(v)) if v.size else float("nan")

    def last(layer, slot, mask=None):
        v = sel(layer, slot, mask)
        return float(v.max()) if v.size else float("nan")

    segments = [
        ("h -> QKV input staged + RMSNorm (XCD 0)", lambda l: med(l, 0) - last(l - 1, 9)),
        ("QKV dot products + store", lambda l: last(l, 1, x0) - med(l, 0)),
        ("QKV store -> last attention task done", lambda l: last(l, 2) - last(l, 1, x0)),
        ("attention -> O input staged", lambda l: med(l, 3) - last(l, 2)),
        ("O dot products + publish", lambda l: last(l, 4, x0) - med(l, 3)),
        ("O -> h1 staged across XCDs + RMSNorm", lambda l: med(l, 5) - last(l, 4, x0)),
        ("gate/up + SwiGLU + down partial + barrier", lambda l: last(l, 6) - med(l, 5)),
        ("workgroup partial store", lambda l: last(l, 7) - last(l, 6)),
        ("per-XCD reduction (median)", lambda l: med(l, 8, ~x0) - last(l, 7)),
        ("per-XCD reduction (last)", lambda l: last(l, 8, ~x0) - last(l, 7)),
        ("XCD-0 reduction + residual (median)", lambda l: med(l, 9) - last(l, 8, ~x0)),
        ("XCD-0 reduction + residual (last)", lambda l: last(l, 9) - last(l, 8, ~x0)),
        ("layer", lambda l: med(l + 1, 0) - med(l, 0)),
    ]
    layers = range(1, L - 1)
    table = {}
    for name, fn in segments:
        vals = [fn(l) for l in layers]
        vals = [v for v in vals if np.isfinite(v)]
        table[name] = round(float(np.mean(vals)), 1) if vals else None
    attn_names = ["start", "q/k/v polled", "scores", "softmax", "merge barrier", "stored (one chunk)",
                  "stored (merged)", "partial published"]
    attn = {}
    for k, name in enumerate(attn_names):
        vals = []
        for l in layers:
            v = A[:, l, k]
            v = v[v > 0]
            q = last(l, 1, x0)
            if v.size and np.isfinite(q):
                vals.append(float(np.median(v)) - q)
        attn[name] = round(float(np.mean(vals)), 1) if vals else None
    out = {"workload": "phases", "model": args.phases_model, "prompt_tokens": n, "step_kind": kind,
           "positions": [n, n + steps - 1], "layers_averaged": [1, L - 2],
           "ns_per_layer": table, "attention_task_ns_after_last_qkv_store": attn}
    for name, v in table.items():
        log(f"{name:45s} {v if v is not None else '-':>8} ns")
    for name, v in attn.items():
        log(f"  attention: {name:32s} {v if v is not None else '-':>8} ns after the last QKV store")
    print(json.dumps(out), flush=True)


def prefill_main(args):
    """Batched prefills of the Qwen2.5-0.5B-shape decoder for kernel traces:
    the 40-token prompt five times and a 4064-token prompt three times
    (wall-clock times printed; the kernel durations come from the trace)."""
    import numpy as np

    from runtime.qwen_engine import QwenDecoderEngine
    from runtime.synthetic import QWEN25_05B, SyntheticModel

    model = SyntheticModel(QWEN25_05B, seed=0)
    meta = model.metadata
    rng = np.random.default_rng(12)
    short = [int(t) for t in rng.integers(0, meta["vocab_size"], PROMPT)]
    long_prompt = [int(t) for t in rng.integers(0, meta["vocab_size"], 4064)]
    engine = QwenDecoderEngine(model, context_length=4096)
    out = {"workload": "prefill", "prompt_40_ms": [], "prompt_4064_ms": []}
    try:
        engine.prefill(short)
        for _ in range(5):
            t0 = time.perf_counter()
            engine.prefill(short, want_logits_array=False)
            out["prompt_40_ms"].append(round((time.perf_counter() - t0) * 1e3, 3))
        for _ in range(3):
            t0 = time.perf_counter()
            engine.prefill(long_prompt, want_logits_array=False)
            out["prompt_4064_ms"].append(round((time.perf_counter() - t0) * 1e3, 3))
    finally:
        engine.close()
    attn = 4.0 * meta["attention_heads"] * meta["head_dim"] * meta["layers"] * 4064 * 4065 / 2
    out["flops_4064"] = 2.0 * 4064 * layer_params(meta) + attn
    out["flops_40"] = 2.0 * PROMPT * layer_params(meta)
    print(json.dumps(out), flush=True)


MOE_COPIES = 3  # device copies of the MoE block cycled by the timed calls (3 x 1.14 GB)
MOE_BATCHES = 8  # distinct random token batches per copy


def moe_call_bytes(shape, unique_routed, tokens):
    """Algorithmic HBM bytes of one MoE block call: the router, the gate/up and
    down weights of every routed expert the batch selects (each read once) and
    of the shared experts, the bf16 input and output rows, the routing."""
    H, I, E, S, k = (shape[n] for n in ("hidden", "intermediate", "experts", "shared", "top_k"))
    expert = (2 * I * H + H * I) * 2
    return E * H * 2 + (unique_routed + S) * expert + 2 * tokens * H * 2 + 8 * tokens * k


def moe_main(args):
    """The routed-expert block (config: hidden 2048, 64 routed experts + 2
    shared of SwiGLU intermediate 1408, top-6 from a softmax router, bf16
    N(0, 0.02) weights, tokens N(0, 1)) at 1, 2, 4, 8 and 16 tokens.  Each
    timed call runs hk_moe_forward (router, top-k, grouped expert GEMMs,
    combine) on one of three device copies of the block and one of eight
    token batches, so no call finds its experts in the 256 MB Infinity Cache
    from the call before; HIP events around the calls; bytes are each call's
    own selection (its distinct routed experts)."""
    import ctypes

    import numpy as np

    from runtime import hip
    from runtime.bf16 import to_bits
    from runtime.moe import MOE_2048_64X1408, MoEBlock, synthetic_moe

    shape = MOE_2048_64X1408
    H, k = shape["hidden"], shape["top_k"]
    hip.init(0)
    lib = hip.lib()
    log("building the MoE block (64 + 2 experts of 2048 -> 1408 -> 2048)")
    router, gate_up, down = synthetic_moe(shape, seed=0)
    blocks = [MoEBlock(router, gate_up, down, top_k=k, shared=shape["shared"], max_tokens=16)
              for _ in range(MOE_COPIES)]
    rng = np.random.default_rng(21)
    xs = to_bits(rng.standard_normal((MOE_BATCHES, 16, H), dtype=np.float32))
    xbuf = hip.DeviceBuffer.from_array(xs)
    ybuf = hip.DeviceBuffer(2 * 16 * H)
    ids = hip.DeviceBuffer(4 * 16 * k)
    xptr = lambda r: xbuf.ptr + r * 16 * H * 2

    def call(b, r, tokens, with_ids=False):
        hip.check(lib.hk_moe_forward(blocks[b]._moe, ctypes.c_void_p(xptr(r)), tokens, ybuf.ptr,
                                     ids.ptr if with_ids else None, None, None), "hk_moe_forward")

    n = max(args.kernel_launches, MOE_COPIES * MOE_BATCHES)
    rows = []
    for tokens in (1, 2, 4, 8, 16):
        nbytes = []
        for r in range(MOE_BATCHES):  # each batch's selection (the copies route alike)
            call(0, r, tokens, with_ids=True)
            hip.check(lib.hk_stream_sync(None), "sync")
            sel = ids.read(np.int32, tokens * k)
            nbytes.append(moe_call_bytes(shape, len(set(sel.tolist())), tokens))
        order = [(i % MOE_COPIES, (i // MOE_COPIES) % MOE_BATCHES) for i in range(n)]
        for b, r in order:  # warm
            call(b, r, tokens)
        e0, e1 = hip.Event(), hip.Event()
        e0.record(None)
        for b, r in order:
            call(b, r, tokens)
        e1.record(None)
        hip.check(lib.hk_stream_sync(None), "sync")
        us = e0.elapsed_ms(e1) * 1e3 / n
        mean_bytes = sum(nbytes[r] for _, r in order) / n
        gbs = mean_bytes / (us * 1e-6) / 1e9
        rows.append({"tokens": tokens, "us_per_call": round(us, 2), "bytes_per_call": int(mean_bytes),
                     "hbm_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"MoE block, {tokens} token(s): {us:.1f} us per call, {mean_bytes / 1e6:.1f} MB, "
            f"{gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of the HBM peak)")
    best = max(rows, key=lambda r: r["frac"])
    result = {
        "metric": "MoE block calls/s at 16 tokens, experts from HBM",
        "value": round(1e6 / rows[-1]["us_per_call"], 1),
        "unit": "calls/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": n,
        "ms_per_step": round(rows[-1]["us_per_call"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "routed-expert block: hidden 2048, 64 routed + 2 shared experts, SwiGLU "
            "intermediate 1408, top-6 softmax router, bf16 N(0,0.02) weights, tokens N(0,1); calls "
            f"cycle {MOE_COPIES} device copies of the block x {MOE_BATCHES} token batches",
            **shape,
        },
        "by_tokens": rows,
        "roofline": {
            "bound": "hbm",
            "kernel": "the whole hk_moe_forward call (router, plan, grouped gate/up + SwiGLU, down, "
            f"combine) at {best['tokens']} token(s)",
            "achieved": best["hbm_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": best["frac"],
            "traffic": None,
        },
    }
    if not args.no_cpu_baseline:
        from threadpoolctl import threadpool_limits

        from oracle.moe import moe_forward

        log("timing the CPU oracle (one token per call)")
        calls, t0 = 0, time.perf_counter()
        with threadpool_limits(limits=1):
            while time.perf_counter() - t0 < 10.0 or calls == 0:
                moe_forward(xs[calls % MOE_BATCHES, :1], router, gate_up, down, top_k=k, shared=shape["shared"])
                calls += 1
        elapsed = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(calls / elapsed, 3), "unit": "calls/s (1 token)", "cores": 1,
                                  "kind": "port",
                                  "sample": f"{calls} one-token block calls through oracle/moe.py, one BLAS thread"}
    for b in blocks:
        b.close()
    print(json.dumps(result), flush=True)


EXPERTS, EXPERT_ROWS, EXPERT_COLS = 8, 2048, 2048  # the reference's 8 expert slots of 2048 x 2048
EXPERT_POOL = 128  # experts resident on the device: 512 MiB of int8, twice the 256 MB Infinity Cache
GROUP_HIDDEN, GROUP_MID = 2048, 1408  # an 8-expert group of the 64-expert H2048/I1408 MoE


QUANT_POOLS = {"q4_k": (12, 144, 256), "q6_k": (14, 210, 160)}  # ggml type, block bytes, resident experts


def quant_launch_bytes(block_bytes):
    """Algorithmic bytes of one quantised MUL_MAT_ID launch over 8 slots:
    the experts' GGML blocks, the bf16 input row per slot, float32 outputs."""
    per_slot = EXPERT_ROWS * (EXPERT_COLS // 256) * block_bytes + 2 * EXPERT_COLS + 4 * EXPERT_ROWS
    return EXPERTS * per_slot


def quant_mul_mat_id(experts, rng, x, n):
    """Q4_K / Q6_K MUL_MAT_ID launches rotating over more experts than the
    Infinity Cache holds (random valid blocks: random quants and scales,
    small fp16 d)."""
    import numpy as np

    out = {}
    for name, (gtype, block_bytes, pool) in QUANT_POOLS.items():
        nb = EXPERT_COLS // 256
        blocks = rng.integers(0, 256, (pool * EXPERT_ROWS, nb, block_bytes), dtype=np.uint8)
        d_at = (0, 2) if gtype == 12 else (208,)
        for off in d_at:
            blocks[..., off:off + 2] = rng.uniform(0.001, 0.01, (pool * EXPERT_ROWS, nb)).astype(
                np.float16).view(np.uint8).reshape(pool * EXPERT_ROWS, nb, 2)
        qset = experts.GgmlExperts.quant(gtype, blocks, pool, EXPERT_ROWS, EXPERT_COLS)
        del blocks
        qset.mul_mat_id(x, np.arange(EXPERTS, dtype=np.int32))
        rotating = (np.arange(n)[:, None] * EXPERTS + np.arange(EXPERTS)[None, :]) % pool
        qset.repeat_ms(rotating)  # warm
        ms = qset.repeat_ms(rotating)
        nbytes = quant_launch_bytes(block_bytes)
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"{name} MUL_MAT_ID 8x2048x2048: kernel {ms * 1e3:.2f} us ({gbs:.0f} GB/s) rotating over {pool} experts")
        out[name] = {"kernel_us": round(ms * 1e3, 3), "bytes_per_launch": nbytes, "achieved_gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "resident_experts": pool}
        qset.close()
    return out


def expert_launch_bytes():
    """Algorithmic HBM bytes of one MUL_MAT_ID launch over 8 slots: int8
    weights and float32 row scales of 8 experts, the bf16 input row read by
    every slot, and 8 float32 output rows."""
    per_slot = EXPERT_ROWS * EXPERT_COLS + 4 * EXPERT_ROWS + 2 * EXPERT_COLS + 4 * EXPERT_ROWS
    return EXPERTS * per_slot


def experts_cpu_baseline(weights, x, budget_s=10.0):
    """The oracle's expert projection (pre-quantised, one BLAS thread) on the
    same 8-slot call, repeated for about ``budget_s`` seconds."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import experts as ox

    packed = [ox.requantize_rows(weights[e]) for e in range(EXPERTS)]
    calls, t0 = 0, time.perf_counter()
    with threadpool_limits(limits=1):
        while time.perf_counter() - t0 < budget_s or calls == 0:
            for q, s in packed:
                ox.project(q, s, x)
            calls += 1
    elapsed = time.perf_counter() - t0
    return {"value": round(calls / elapsed, 3), "unit": "calls/s", "cores": 1, "kind": "port",
            "sample": f"{calls} MUL_MAT_ID calls (8 x {EXPERT_ROWS} x {EXPERT_COLS}, weights "
            "pre-quantised) through oracle/experts.py with one BLAS thread"}


def experts_main(args):
    """Expert shims: the MUL_MAT_ID kernel over 8-expert slices of 128
    resident 2048 x 2048 W8 experts, rotating so that no launch finds its
    weights in the Infinity Cache (timed with HIP events); the host-pointer
    call rate of both contracts; and the oracle on the host."""
    import numpy as np

    from runtime import experts, hip

    hip.init(0)
    rng = np.random.default_rng(5)
    log(f"requantising {EXPERT_POOL} x {EXPERT_ROWS} x {EXPERT_COLS} expert weights")
    w = rng.standard_normal((EXPERT_POOL, EXPERT_ROWS, EXPERT_COLS), dtype=np.float32)
    w *= np.float32(0.02)
    x = rng.normal(0, 1, EXPERT_COLS).astype(np.float32)
    ids = np.arange(EXPERTS, dtype=np.int32)
    ggml = experts.GgmlExperts(w)
    for _ in range(max(args.warmup, 1)):
        ggml.mul_mat_id(x, ids)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ggml.mul_mat_id(x, ids)
    call_s = (time.perf_counter() - t0) / args.steps
    n = args.kernel_launches
    rotating = (np.arange(n)[:, None] * EXPERTS + np.arange(EXPERTS)[None, :]) % EXPERT_POOL
    same = np.tile(ids, (n, 1))
    ggml.repeat_ms(rotating)  # warm
    kernel_ms = ggml.repeat_ms(rotating)
    warm_ms = ggml.repeat_ms(same)
    nbytes = expert_launch_bytes()
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    log(f"MUL_MAT_ID 8x2048x2048: kernel {kernel_ms * 1e3:.2f} us ({achieved:.0f} GB/s) rotating over "
        f"{EXPERT_POOL} experts, {warm_ms * 1e3:.2f} us on the same 8; call {call_s * 1e6:.1f} us host-inclusive")

    quant = quant_mul_mat_id(experts, rng, x, n)

    # Colibri expert group: 8 experts of 2048 -> 1408 -> 2048, one row each
    experts.coli_init(0)
    mk = lambda shape: rng.normal(0, 0.02, shape).astype(np.float32)
    g = [experts.ColiTensor(mk((GROUP_MID, GROUP_HIDDEN)), None, 0, GROUP_HIDDEN, GROUP_MID) for _ in range(8)]
    u = [experts.ColiTensor(mk((GROUP_MID, GROUP_HIDDEN)), None, 0, GROUP_HIDDEN, GROUP_MID) for _ in range(8)]
    d = [experts.ColiTensor(mk((GROUP_HIDDEN, GROUP_MID)), None, 0, GROUP_MID, GROUP_HIDDEN) for _ in range(8)]
    gx = rng.normal(0, 1, 8 * GROUP_HIDDEN).astype(np.float32)
    for _ in range(max(args.warmup, 1)):
        experts.expert_group(g, u, d, gx)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        experts.expert_group(g, u, d, gx)
    group_s = (time.perf_counter() - t0) / args.steps
    log(f"Colibri expert group 8 x (2048->1408->2048): {group_s * 1e6:.1f} us per call host-inclusive")
    for t in g + u + d:
        t.close()
    experts.coli_shutdown()

    traffic = None
    tfile = ROOT / "profiles" / "traffic_expert_w8_mul_mat_id.json"
    if tfile.is_file():
        traffic = json.loads(tfile.read_text()).get("traffic_bytes_per_launch")
    result = {
        "metric": "MUL_MAT_ID expert GEMV launches/s, 8 x 2048 x 2048 W8 experts per launch from HBM",
        "value": round(1e3 / kernel_ms, 1),
        "unit": "launches/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kernel_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights, f32 accumulate",
        "data": "synthetic",
        "config": {
            "workload": "GGML MUL_MAT_ID, 8 ids per launch over 128 resident experts of 2048 x 2048 "
            "(N(0,0.02) weights requantised to int8 + row scale), one float32 input row, launch i "
            "using experts 8i..8i+7 mod 128; Colibri expert group of 8 experts 2048 -> 1408 -> 2048",
            "experts_per_launch": EXPERTS, "resident_experts": EXPERT_POOL, "rows": EXPERT_ROWS,
            "cols": EXPERT_COLS,
        },
        "kernel_us_same_experts": round(warm_ms * 1e3, 3),
        "call_us_host_inclusive": round(call_s * 1e6, 2),
        "coli_group_us_host_inclusive": round(group_s * 1e6, 2),
        "quant_mul_mat_id": quant,
        "roofline": {
            "bound": "hbm",
            "kernel": f"expert_w8_kernel, one launch per MUL_MAT_ID call (bytes/launch {nbytes})",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
    }
    if not args.no_cpu_baseline:
        log("timing the CPU oracle")
        result["cpu_baseline"] = experts_cpu_baseline(w[:EXPERTS], x)
    ggml.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
