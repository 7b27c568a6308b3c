"""Prefill attention on the matrix cores (gh_attention_prefill with n >= 32 rows, G = 4)
against the oracle, and against the reference's own prefill-attention test vectors.

Bars:
  * oracle (attention/mod.rs:582-725 restated): |got - want| <= 1e-3·|want| + 1e-5 — outputs
    are convex combinations of V rows; P·V runs with FP16 hi + lo probabilities, so the only
    FP16 rounding left is the output's (2^-11 relative);
  * the reference's Vulkan prefill test (vulkan/mod.rs:935-1110): its q/k/v generators, shapes
    (q_heads 4, kv_heads 1, head_dim 128; contexts 2048 / 8192 / 28000, n = 64 / 32 / 16 at the
    end of the context) and its bar |got - want| <= 2e-2 + 2e-2·|want| (vulkan/mod.rs:1245-1258),
    against both the per-row decode path and the CPU softmax.
"""
import numpy as np
import pytest

import oracle as O
from graph_horizon_amd import _ffi as F

pytestmark = pytest.mark.gpu


def _kv(hip, layers, ctx, kvh, kc, vc):
    return F.GhKv(hip.from_host(kc), hip.from_host(vc), F.KV_F16, layers, ctx, kvh, 128, 128)


def _free(hip, *bufs):
    for b in bufs:
        hip.free_buffer(b)


def _close(got, want, what, rel=1e-3, floor=1e-5):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    tol = rel * np.abs(want) + floor
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside, worst " \
        f"{np.max(np.abs(got - want) / tol):.3f}x tol"


@pytest.mark.parametrize("ctx,base,n,layer", [
    (512, 0, 32, 0),      # one query block, first tile only
    (512, 0, 100, 1),     # ragged rows
    (1024, 300, 200, 1),  # base inside a key tile, query blocks straddling tiles
    (2048, 0, 512, 0),    # the model's prefill chunk
    (4096, 4000, 96, 1),  # late chunk of a long context
])
def test_prefill_attention_matches_oracle(hip, ctx, base, n, layer):
    rng = np.random.default_rng(ctx + base + n)
    layers, qh, kvh = 2, 32, 8
    kc = O.f16(rng.standard_normal(layers * ctx * kvh * 128).astype(np.float32))
    vc = O.f16(rng.standard_normal(layers * ctx * kvh * 128).astype(np.float32))
    q = O.f16(rng.standard_normal(n * qh * 128).astype(np.float32))
    kv = _kv(hip, layers, ctx, kvh, kc, vc)
    qb, ob = hip.from_host(q), hip.alloc_buffer(n * qh * 128 * 2)
    hip.attention_prefill(ob, qb, kv, qh, base, n, layer)
    got = O.f32(hip.download(ob, np.uint16, n * qh * 128))
    want = O.f32(O.attention_prefill(q, kc, vc, 128, kvh, qh, base, n, layer, ctx))
    assert np.isfinite(got).all()
    _close(got, want, f"ctx {ctx} base {base} n {n}")
    _free(hip, qb, ob, kv.k, kv.v)


def test_prefill_attention_c4_2048(hip):
    """BASELINE config 4 prefill: 2048 causal rows, 32 q / 8 kv heads, head_dim 128; 48 rows
    (first, last and spread) checked against the oracle's decode of that row (prefill row r ==
    decode at base + r, attention/mod.rs:920-1024)."""
    n, ctx, qh, kvh = 2048, 2048, 32, 8
    rng = np.random.default_rng(2048)
    kc = O.f16(rng.standard_normal(ctx * kvh * 128).astype(np.float32))
    vc = O.f16(rng.standard_normal(ctx * kvh * 128).astype(np.float32))
    q = O.f16(rng.standard_normal(n * qh * 128).astype(np.float32))
    kv = _kv(hip, 1, ctx, kvh, kc, vc)
    qb, ob = hip.from_host(q), hip.alloc_buffer(n * qh * 128 * 2)
    hip.attention_prefill(ob, qb, kv, qh, 0, n, 0)
    got = O.f32(hip.download(ob, np.uint16, n * qh * 128)).reshape(n, qh * 128)
    assert np.isfinite(got).all()
    rows = sorted(set([0, 1, 31, 32, 63, 64, 1023, 2046, 2047] + list(rng.integers(0, n, 39))))
    for r in rows:
        want = O.f32(O.attention_decode(q[r * qh * 128:(r + 1) * qh * 128], kc, vc, 128, kvh, qh,
                                        r, 0, ctx))
        _close(got[r], want, f"row {r}")
    _free(hip, qb, ob, kv.k, kv.v)


def _reference_case(ctx_total):
    """attention_prefill_decode_for_scheme inputs (vulkan/mod.rs:955-1000), one layer."""
    qh, hd = 4, 128
    pos = np.arange(ctx_total)[:, None]
    i = np.arange(hd)[None, :]
    k = (((pos * 7 + i) % 13).astype(np.float32) * np.float32(0.025) - np.float32(0.12))
    v = (((pos * 11 + i) % 19).astype(np.float32) * np.float32(0.02) - np.float32(0.15))
    return qh, O.f16(k.reshape(-1)), O.f16(v.reshape(-1))


@pytest.mark.parametrize("context", [2048, 8192, 28000])
def test_reference_prefill_attention_vectors(hip, context):
    qh, kc, vc = _reference_case(context)
    kv = _kv(hip, 1, context, 1, kc, vc)
    for n in (64, 32, 16):  # n = 16 runs the per-row split-K path
        base = context - n
        idx = np.arange(n * qh * 128)
        q = O.f16(((idx % 17).astype(np.float32) * np.float32(0.03) - np.float32(0.22)))
        qb, pb, db = hip.from_host(q), hip.alloc_buffer(q.nbytes), hip.alloc_buffer(q.nbytes)
        hip.attention_prefill(pb, qb, kv, qh, base, n, 0)
        for r in range(n):
            qr = hip.view(qb, r * qh * 256, qh * 256)
            dr = hip.view(db, r * qh * 256, qh * 256)
            hip.attention_decode(dr, qr, kv, qh, base + r, 0)
        got_p = O.f32(hip.download(pb, np.uint16, q.size)).astype(np.float64)
        got_d = O.f32(hip.download(db, np.uint16, q.size)).astype(np.float64)
        # CPU softmax in fp64 over the FP16 inputs (the reference test's own CPU oracle)
        kf = O.f32(kc).astype(np.float64).reshape(context, 128)
        vf = O.f32(vc).astype(np.float64).reshape(context, 128)
        qf = O.f32(q).astype(np.float64).reshape(n, qh, 128)
        cpu = np.empty((n, qh, 128))
        for r in range(n):
            s = qf[r] @ kf[:base + r + 1].T / np.sqrt(128.0)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            cpu[r] = (p / p.sum(axis=1, keepdims=True)) @ vf[:base + r + 1]
        cpu = cpu.reshape(-1)
        for what, a, b in (("prefill vs decode", got_p, got_d), ("prefill vs cpu", got_p, cpu),
                           ("decode vs cpu", got_d, cpu)):
            err = np.abs(a - b)
            ok = err <= 2e-2 + 2e-2 * np.abs(b)
            assert ok.all(), f"ctx {context} n {n} {what}: {(~ok).sum()} outside"
            # and the repository's own bar on the same data
            _close(a, b, f"ctx {context} n {n} {what}", rel=1e-3, floor=1e-5)
        _free(hip, qb, pb, db)
    _free(hip, kv.k, kv.v)


@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 8), (16, 8), (64, 8)], ids=["g4", "g1", "g2", "g8"])
def test_decode_every_forced_split_count(hip, qh, kvh):
    """Decode attention with each split count 1..32 forced (gh_set_attention_splits), for each
    GQA group size: the split partials cross workgroups through agent-scope atomics and the
    last workgroup of each (row, kv head) merges them. Positions below, at and across chunk
    boundaries, and counts above the row's chunk count. Same bar as the oracle decode test."""
    rng = np.random.default_rng(321 + qh)
    ctx, layers = 2048, 2
    kc = O.f16(rng.standard_normal(layers * ctx * kvh * 128).astype(np.float32))
    vc = O.f16(rng.standard_normal(layers * ctx * kvh * 128).astype(np.float32))
    kv = _kv(hip, layers, ctx, kvh, kc, vc)
    q = O.f16(rng.standard_normal(qh * 128).astype(np.float32))
    qb, ob = hip.from_host(q), hip.alloc_buffer(qh * 128 * 2)
    cases = [(0, 0), (63, 1), (64, 0), (700, 1), (2047, 1)]
    want = {c: O.f32(O.attention_decode(q, kc, vc, 128, kvh, qh, c[0], c[1], ctx)) for c in cases}
    modes = [False, True] if hip.xcd_count else [False]
    try:
        for splits in range(1, 33):
            hip.set_attention_splits(splits)
            for pos, layer in cases:
                bits = []
                for xcd in modes:  # the split merge through device memory, then one XCD's L2
                    hip.set_attention_xcd_merge(xcd)
                    hip.attention_decode(ob, qb, kv, qh, pos, layer)
                    bits.append(hip.download(ob, np.uint16, qh * 128))
                    _close(O.f32(bits[-1]), want[(pos, layer)], f"splits {splits} pos {pos} xcd {xcd}")
                assert all(np.array_equal(b, bits[0]) for b in bits), f"merge forms differ: {splits} {pos}"
    finally:
        hip.set_attention_splits(0)
        hip.set_attention_xcd_merge(bool(hip.xcd_count))
    _free(hip, qb, ob, kv.k, kv.v)


def test_xcd_probe_confirms_the_mi355x_dispatch():
    """The start-up probe sees the eight XCDs of an MI355X (256 CUs) in one partition and
    workgroup i of each probed launch on XCD i mod 8, so decode attention merges its splits
    through one XCD's L2 by default."""
    from graph_horizon_amd import HipBackend

    with HipBackend() as b:
        print(f"xcd_count {b.xcd_count}")
        assert b.xcd_count == 8


@pytest.mark.parametrize("qh,kvh,n", [(12, 3, 7), (64, 8, 5), (32, 8, 20), (16, 16, 3)],
                         ids=["g4-kv3", "g8", "g4-rows20", "g1-kv16"])
def test_multi_row_decode_kernels_xcd_grid(hip, qh, kvh, n):
    """Rows below the matrix-core prefill's minimum (or groups it does not serve) run the
    decode kernels with several query rows. In the XCD-local grid the (row, kv head) pairs fill
    z-groups of xcds, the last one partly (kv_heads 3: 21 pairs): both merge forms give the
    same bits, within the oracle bar, at every split count the row lengths allow."""
    if not hip.xcd_count:
        pytest.skip("dispatch placement not confirmed on this device")
    rng = np.random.default_rng(qh * 7 + kvh + n)
    ctx, base = 1024, 600
    kc = O.f16(rng.standard_normal(ctx * kvh * 128).astype(np.float32))
    vc = O.f16(rng.standard_normal(ctx * kvh * 128).astype(np.float32))
    q = O.f16(rng.standard_normal(n * qh * 128).astype(np.float32))
    kv = _kv(hip, 1, ctx, kvh, kc, vc)
    qb, ob = hip.from_host(q), hip.alloc_buffer(n * qh * 128 * 2)
    want = O.f32(O.attention_prefill(q, kc, vc, 128, kvh, qh, base, n, 0, ctx))
    try:
        for splits in (0, 1, 5, 11):
            hip.set_attention_splits(splits)
            bits = []
            for xcd in (False, True):
                hip.set_attention_xcd_merge(xcd)
                hip.attention_prefill(ob, qb, kv, qh, base, n, 0)
                bits.append(hip.download(ob, np.uint16, n * qh * 128))
                _close(O.f32(bits[-1]), want, f"splits {splits} xcd {xcd}")
            assert np.array_equal(bits[0], bits[1]), f"merge forms differ at {splits} splits"
    finally:
        hip.set_attention_splits(0)
        hip.set_attention_xcd_merge(True)
    _free(hip, qb, ob, kv.k, kv.v)


def test_greedy_graph_with_forced_splits_matches_stream(hip):
    """A replayed decode graph whose attention grid is fixed at 32 splits (most of them idle at
    short positions) gives the tokens of the same steps launched on the stream."""
    from graph_horizon_amd import HipModel, synth

    shape = synth.SHAPES["tiny"]
    outs = []
    hip.set_attention_splits(32)
    try:
        for flags in (0, F.MODEL_NO_GRAPH):
            gm = HipModel(hip, synth.model_config(shape, 2304, 16, flags=flags))
            for layer, tid, fmt, data in synth.model_tensors(shape, 36):
                gm.load_tensor(layer, tid, fmt, data)
            gm.prefill(list(range(1, 60)), 0)
            outs.append(gm.decode_greedy(9, 59, 40))
            gm.close()
    finally:
        hip.set_attention_splits(0)
    assert np.array_equal(outs[0], outs[1])


def test_graph_replay_ignores_partials_of_earlier_steps(hip):
    """A replayed decode graph whose attention grid is fixed at 4 splits (forced: one step
    graph over the whole 256-position context), while the splits in use follow the position.
    A run that crosses position 64 (two splits in use) leaves real partials and merge state
    behind; replaying the first steps again (one split in use) must give the first run's
    tokens."""
    from graph_horizon_amd import HipModel, synth

    shape = synth.SHAPES["tiny"]
    hip.set_attention_splits(4)
    try:
        gm = HipModel(hip, synth.model_config(shape, 256, 64))
        for layer, tid, fmt, data in synth.model_tensors(shape, 33):
            gm.load_tensor(layer, tid, fmt, data)
        prompt = [3, 99, 1500, 42]
        gm.prefill(prompt, 0)
        first = gm.read_argmax()
        short = gm.decode_greedy(first, 4, 8)
        gm.prefill(prompt, 0)
        long = gm.decode_greedy(first, 4, 70)
        gm.prefill(prompt, 0)
        again = gm.decode_greedy(first, 4, 8)
        gm.close()
    finally:
        hip.set_attention_splits(0)
    assert np.array_equal(long[:8], short) and np.array_equal(again, short)
