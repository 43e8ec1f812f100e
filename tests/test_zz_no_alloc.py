"""hk_attention_decode_noalloc (the attention entry point that allocates
nothing: its scratch is a static device array) against hk_attention_decode on
the same inputs, through the C ABI.  Both launch the same kernel with the same
grid, so outputs and the KV append agree bit for bit.  Two calls in a row, the
second smaller, check that the shared scratch carries nothing over."""

import numpy as np
import pytest

from _util import announce
from oracle import bf16

pytestmark = pytest.mark.gpu


def _dev(array):
    from runtime import hip

    return hip.DeviceBuffer.from_array(np.ascontiguousarray(array))


def _inputs(q_heads, kv_heads, ctx, position, seed):
    from runtime.qwen_engine import rope_tables

    rng = np.random.default_rng(seed)
    cos, sin = rope_tables(1e6, 64, ctx)
    kc = np.zeros((kv_heads, ctx, 64), np.uint16)
    vc = np.zeros((kv_heads, ctx, 64), np.uint16)
    kc[:, :position] = bf16.to_bits(rng.normal(0, 1, (kv_heads, position, 64)).astype(np.float32))
    vc[:, :position] = bf16.to_bits(rng.normal(0, 1, (kv_heads, position, 64)).astype(np.float32))
    qkv = bf16.to_bits(rng.normal(0, 1, (q_heads + 2 * kv_heads) * 64).astype(np.float32))
    return qkv, cos, sin, kc, vc


def _run(hk_lib, entry, q_heads, kv_heads, ctx, position, inputs):
    from runtime import hip

    qkv, cos, sin, kc, vc = inputs
    QKV, COS, SIN, KC, VC = _dev(qkv), _dev(cos), _dev(sin), _dev(kc), _dev(vc)
    OUT = hip.DeviceBuffer(2 * q_heads * 64)
    fn = getattr(hk_lib, entry)
    hip.check(fn(QKV.ptr, COS.ptr, SIN.ptr, KC.ptr, VC.ptr, position, ctx, q_heads, kv_heads, 64, OUT.ptr, None),
              entry)
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    return (OUT.read(np.uint16, q_heads * 64), KC.read(np.uint16, kc.size), VC.read(np.uint16, vc.size))


# (q_heads, kv_heads, context, position): a long context whose heads merge 16
# split-KV chunks, then a smaller call (fewer heads, one chunk), then a
# mid-size one with three chunks
CASES = [(14, 2, 4096, 4000), (9, 3, 300, 100), (14, 2, 1024, 700)]


def test_noalloc_attention_matches_allocating_entry_point(hk_lib):
    for i, (hq, hkv, ctx, pos) in enumerate(CASES):
        announce(f"attention noalloc call {i}: Hq={hq} Hkv={hkv} ctx={ctx} p={pos}")
        inputs = _inputs(hq, hkv, ctx, pos, 100 + i)
        want = _run(hk_lib, "hk_attention_decode", hq, hkv, ctx, pos, inputs)
        got = _run(hk_lib, "hk_attention_decode_noalloc", hq, hkv, ctx, pos, inputs)
        for g, w, name in zip(got, want, ("out", "kcache", "vcache")):
            np.testing.assert_array_equal(g, w, err_msg=f"call {i}: {name}")
        assert np.any(got[0] != 0)


def test_noalloc_attention_rejects_contexts_beyond_its_scratch(hk_lib):
    from runtime import hip

    announce("attention noalloc: size limit")
    # 64 heads x 256 chunks x 264 bytes of partials: above the 1 MiB scratch
    qkv = _dev(np.zeros((64 + 2 * 4) * 64, np.uint16))
    tab = _dev(np.zeros(32, np.float32))
    cache = _dev(np.zeros(64, np.uint16))
    out = hip.DeviceBuffer(2 * 64 * 64)
    rc = hk_lib.hk_attention_decode_noalloc(qkv.ptr, tab.ptr, tab.ptr, cache.ptr, cache.ptr, 0, 65536, 64, 4,
                                            64, out.ptr, None)
    assert rc == hip.HK_ERR_INVALID
    assert "1 MiB" in hip.last_error()
