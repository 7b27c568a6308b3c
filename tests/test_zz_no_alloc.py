"""gh_attention_decode_noalloc (the no-allocation decode attention) against gh_attention_decode:
the same kernels and split counts over a fixed device scratch array, so the outputs are
bit-identical. Two calls in a row, the second smaller (fewer positions, fewer heads), leave
the array's counters clear for the next; launches needing more scratch than the array holds
are rejected.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from graph_horizon_amd import GhError
from graph_horizon_amd import _ffi as F

pytestmark = pytest.mark.gpu


def _kv(hip, layers, ctx, kvh, rng):
    n = layers * ctx * kvh * 128
    kc = O.f16(rng.standard_normal(n).astype(np.float32))
    vc = O.f16(rng.standard_normal(n).astype(np.float32))
    return F.GhKv(hip.from_host(kc), hip.from_host(vc), F.KV_F16, layers, ctx, kvh, 128, 128)


def _decode(hip, name, kv, q_heads, pos, layer, qb):
    ob = hip.alloc_buffer(q_heads * 128 * 2)
    hip._run(name, C.byref(ob), C.byref(qb), C.byref(kv), q_heads, pos, layer)
    out = hip.download(ob, np.uint16, q_heads * 128)
    hip.free_buffer(ob)
    return out


@pytest.mark.parametrize("splits", [0, 32])
def test_noalloc_decode_matches_allocating_entry_point(hip, splits):
    rng = np.random.default_rng(77 + splits)
    hip.set_attention_splits(splits)
    try:
        # first call: 32 q / 8 kv heads (GQA 4) at the last position of a 4096-position cache;
        # second call, smaller: 8 q / 8 kv heads (GQA 1) at position 100
        for q_heads, kv_heads, ctx, pos, layer in ((32, 8, 4096, 4095, 1), (8, 8, 512, 100, 0)):
            kv = _kv(hip, 2, ctx, kv_heads, rng)
            qb = hip.from_host(O.f16(rng.standard_normal(q_heads * 128).astype(np.float32)))
            want = _decode(hip, "gh_attention_decode", kv, q_heads, pos, layer, qb)
            got = _decode(hip, "gh_attention_decode_noalloc", kv, q_heads, pos, layer, qb)
            assert np.array_equal(got, want), (q_heads, pos)
            for b in (qb, kv.k, kv.v):
                hip.free_buffer(b)
    finally:
        hip.set_attention_splits(0)


def test_noalloc_rejects_launches_beyond_its_scratch(hip):
    """128 query heads x 32 splits need 2 MiB of partials (> the 1 MiB array): GH_E_RANGE, and
    the array still serves the next call."""
    rng = np.random.default_rng(5)
    kv = _kv(hip, 1, 2048, 16, rng)
    qb = hip.from_host(O.f16(rng.standard_normal(128 * 128).astype(np.float32)))
    hip.set_attention_splits(32)
    try:
        with pytest.raises(GhError) as e:
            _decode(hip, "gh_attention_decode_noalloc", kv, 128, 2047, 0, qb)
        assert e.value.code == -5  # GH_E_RANGE
        got = _decode(hip, "gh_attention_decode_noalloc", kv, 16, 2047, 0, qb)
        want = _decode(hip, "gh_attention_decode", kv, 16, 2047, 0, qb)
        assert np.array_equal(got, want)
    finally:
        hip.set_attention_splits(0)
    for b in (qb, kv.k, kv.v):
        hip.free_buffer(b)


def test_noalloc_grows_no_backend_scratch():
    """The entry point's whole scratch is its fixed array: on a fresh backend (no attention
    has run, so it holds no merge counters yet) two no-allocation calls at 32 splits leave the
    backend's workspace, counter slots and generation exactly as they were. The allocating
    entry point then creates the counters, so the check does see an allocation when one
    happens."""
    from graph_horizon_amd import HipBackend

    rng = np.random.default_rng(9)
    with HipBackend(0) as fresh:
        fresh.set_attention_splits(32)
        before = fresh.scratch_info()
        assert before[1] == 0, before
        outs = []
        for q_heads, kv_heads, ctx, pos in ((32, 8, 4096, 4095), (8, 8, 512, 100)):
            kv = _kv(fresh, 1, ctx, kv_heads, rng)
            qb = fresh.from_host(O.f16(rng.standard_normal(q_heads * 128).astype(np.float32)))
            outs.append((kv, qb, q_heads, pos,
                         _decode(fresh, "gh_attention_decode_noalloc", kv, q_heads, pos, 0, qb)))
        assert fresh.scratch_info() == before
        for kv, qb, q_heads, pos, got in outs:
            want = _decode(fresh, "gh_attention_decode", kv, q_heads, pos, 0, qb)
            assert np.array_equal(got, want)
        assert fresh.scratch_info()[1] > 0
        for kv, qb, *_ in outs:
            for b in (qb, kv.k, kv.v):
                fresh.free_buffer(b)
