"""The graph driver at the benchmark's real widths (8B-shaped: d 4096, FFN 12288; 14B-shaped:
d 5120, FFN 16384; both 32/8 heads x 128, vocab 131072, Q4_K_M formats), two blocks deep so
the CPU oracle keeps up: batched prefill, then greedy decode through the replayed HIP graph,
teacher-forced against the oracle (the parity.rs protocol, >= 99 % top-1 agreement).
"""
import dataclasses

import numpy as np
import pytest

import oracle as O
from agreement import assert_agreement
from graph_horizon_amd import HipModel, synth
from test_oracle import oracle_model

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["8b", "14b"])
def test_full_width_blocks_decode_matches_oracle(hip, name):
    shape = dataclasses.replace(synth.SHAPES[name], name=f"{name}-2", block_count=2)
    seed, ctx = 77, 160
    tensors = list(synth.model_tensors(shape, seed))
    gm = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=64))
    for layer, tid, fmt, data in tensors:
        gm.load_tensor(layer, tid, fmt, data)
    om, _ = oracle_model(shape, seed, ctx, tensors)
    del tensors
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, shape.vocab_size, 40)]
    gm.prefill(prompt, 0)
    om.prefill(prompt, 0, 64)
    got, want = gm.read_logits(), om.logits()
    assert np.isfinite(got).all()
    scale = np.abs(want).max()
    assert np.max(np.abs(got - want)) <= 2e-2 * max(scale, 1.0), np.max(np.abs(got - want))
    first = int(np.argmax(want))
    steps = 48
    toks = gm.decode_greedy(first, len(prompt), steps)
    tok, ora = first, []
    for i in range(steps):
        om.token(tok, len(prompt) + i)
        ora.append(om.logits())
        tok = int(toks[i])
    assert_agreement(toks, ora, f"{shape.name} {steps} greedy steps")
    gm.close()
    om.close()


def test_8b_full_depth_greedy_64_matches_oracle(hip):
    """The whole 8B-shaped decoder (34 blocks, the bench's model): a 64-token prompt, then 64
    greedy decode steps through the replayed HIP graph, teacher-forced against the oracle
    (generation/tests.rs:375-416, >= 99 % top-1 agreement). The oracle resumes from the
    device's KV cache of the first 63 prompt positions: it recomputes the prompt's last row
    (logits and every layer's K/V row against the device prefill's) and each decode step."""
    shape = synth.SHAPES["8b"]
    seed, ctx, n, steps = 808, 192, 64, 64
    tensors = list(synth.model_tensors(shape, seed))
    print("8b full depth: model generated", flush=True)
    gm = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=n))
    for layer, tid, fmt, data in tensors:
        gm.load_tensor(layer, tid, fmt, data)
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, shape.vocab_size, n)]
    gm.prefill(prompt, 0)
    prefill_logits = gm.read_logits()
    assert np.isfinite(prefill_logits).all()
    kv = gm.kv()
    m = shape.block_count * ctx * shape.kv_head_count * shape.head_dim
    k_dev, v_dev = hip.download(kv.k, np.uint16, m), hip.download(kv.v, np.uint16, m)
    first = gm.read_argmax()
    toks = gm.decode_greedy(first, n, steps)
    gm.close()
    print("8b full depth: device done", flush=True)

    om, _ = oracle_model(shape, seed, ctx, tensors)
    del tensors
    om.load_kv(k_dev, v_dev, ctx, n - 1)
    om.token(prompt[-1], n - 1)
    want = om.logits()
    scale = max(float(np.abs(want).max()), 1.0)
    err = float(np.max(np.abs(prefill_logits - want)))
    print(f"8b full depth: prompt row max |logit diff| {err:.4g} of scale {scale:.4g}", flush=True)
    assert err <= 2e-2 * scale
    kvw = shape.kv_head_count * shape.head_dim
    for role, dev in ((0, k_dev), (1, v_dev)):
        ora = O.f32(om.kv(role)).reshape(shape.block_count, ctx, kvw)[:, n - 1].astype(np.float64)
        got = O.f32(dev).reshape(shape.block_count, ctx, kvw)[:, n - 1].astype(np.float64)
        assert np.max(np.abs(got - ora)) <= 2e-2 * max(np.abs(ora).max(), 1.0), role
    tok, ora = first, [want]
    for i in range(steps):
        om.token(tok, n + i)
        ora.append(om.logits())
        tok = int(toks[i])
    om.close()
    # the prefill's argmax and the 64 greedy tokens against the oracle's logits at each step
    assert_agreement([first] + [int(t) for t in toks], ora, "8b full depth, 64 greedy steps")


@pytest.mark.parametrize("n", [100, 160, 300])
@pytest.mark.parametrize("name", ["8b", "14b"])
def test_full_width_prefill_driver_matches_op_by_op(hip, name, n):
    """The driver's fused prefill at the real widths, 300 rows in one chunk (a partial second
    256-token tile, over the FP16 weight copies), 160 rows (one partial 256-token tile, where
    the separate gate/up GEMMs split K and the driver's paired gate/up launch does not) or 100
    rows (one partial 128-token tile of the
    dequantizing kernels, no copies) — Q/K/V in one mixed-format GEMM with its RoPE split reduce writing K/V into
    the cache, the O and down projections' split sums folded into the residual and the
    RMSNorm, SiLU in the up GEMM, 16-row attention blocks — against every trait op recorded
    separately over the C ABI (prefill::record_batch): logits, the last row's residual and the
    cache. The fused Q/K/V launch splits K differently (2 against 4 and 8), so a few values
    round to the neighbouring FP16; one block keeps that from being amplified by a second
    block of random weights (whose residual grows to thousands and whose attention is nearly
    one-hot), and every difference is bounded against the tensor's scale. On the 8B shape at
    100 rows (one 128-token tile) Q/K/V, O and down split K alike in the fused and the separate
    launches on MI355X's 256 CUs (Q/K/V five splits each); gate and up run in the fused
    driver's one paired launch (gh_gemm3_swiglu_r96_t128, K unsplit) against two GEMMs of two
    splits each op by op, a re-association of each FP32 sum that leaves every FP16 output of
    these weights unchanged: the driver is bit-identical there."""
    from graph_over_abi import AbiGraph

    shape = dataclasses.replace(synth.SHAPES[name], name=f"{name}-1", block_count=1)
    seed, ctx = 91, 320
    tensors = list(synth.model_tensors(shape, seed))
    ref = AbiGraph(hip, shape, seed, ctx, tensors=tensors)
    gm = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=512))
    for layer, tid, fmt, data in tensors:
        gm.load_tensor(layer, tid, fmt, data)
    del tensors
    toks = [int(t) for t in np.random.default_rng(seed).integers(0, shape.vocab_size, n)]
    want = ref.prefill(toks, 0)
    gm.prefill(toks, 0)
    got = gm.read_logits()
    assert np.isfinite(got).all()
    d = shape.embedding_length
    if name == "8b" and n <= 128:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert np.array_equal(gm.read_x().view(np.uint32), ref.prefill_x[(n - 1) * d:].view(np.uint32))
    scale = max(np.abs(want).max(), 1.0)
    assert np.max(np.abs(got - want)) <= 2e-3 * scale, np.max(np.abs(got - want)) / scale
    xw = ref.prefill_x[(n - 1) * d:].astype(np.float64)
    xg = gm.read_x().astype(np.float64)
    assert np.max(np.abs(xg - xw)) <= 2e-3 * max(np.abs(xw).max(), 1.0)
    kv = gm.kv()
    m = shape.block_count * ctx * shape.kv_head_count * shape.head_dim
    for role in ("k", "v"):
        a = hip.download(getattr(kv, role), np.uint16, m).view(np.float16).astype(np.float64)
        b = hip.download(getattr(ref.kv, role), np.uint16, m).view(np.float16).astype(np.float64)
        a = a.reshape(shape.block_count, ctx, -1)[:, :n]
        b = b.reshape(shape.block_count, ctx, -1)[:, :n]
        err = np.abs(a - b)
        assert err.max() <= 2e-3 * np.abs(b).max(), (role, float(err.max()), float(np.abs(b).max()))
        assert np.mean(err > 0) < 1e-2, (role, float(np.mean(err > 0)))  # isolated FP16 flips (0.2 %)
    gm.close()


@pytest.mark.parametrize("n", [160, 300, 2048])
@pytest.mark.parametrize("name", ["8b", "14b"])
def test_prefill_fp16_weight_copies_are_bit_identical(hip, name, n):
    """The FP16 copies of the layer matrices (made before the first prefill with chunks of more
    than 128 rows) hold the values the dequantizing GEMM producers stage, and the all-waves-MFMA
    kernels that read them sum in the same k order over the same tiles and splits: the prefill
    leaves the same logits, residual row and K/V cache bits as with GH_MODEL_NO_F16_WEIGHTS.
    160 rows fill one 256-token tile (the rest clamped to the last row); 300 rows run gate/up
    in 96-row tiles and the mixed Q/K/V launch, O and the Q6_K down in 128-row tiles with split
    K (2, 4 and 4 splits); 2048 rows run every GEMM in 128-row tiles, unsplit."""
    from graph_horizon_amd import _ffi as F

    shape = dataclasses.replace(synth.SHAPES[name], name=f"{name}-1", block_count=1)
    seed, ctx = 17, max(320, n)
    tensors = list(synth.model_tensors(shape, seed))
    toks = [int(t) for t in np.random.default_rng(seed).integers(0, shape.vocab_size, n)]
    outs = []
    for flags in (0, F.MODEL_NO_F16_WEIGHTS):
        gm = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=max(512, n), flags=flags))
        for layer, tid, fmt, data in tensors:
            gm.load_tensor(layer, tid, fmt, data)
        gm.prefill(toks, 0)
        kv = gm.kv()
        m = shape.block_count * ctx * shape.kv_head_count * shape.head_dim
        outs.append((gm.read_logits().view(np.uint32), gm.read_x().view(np.uint32),
                     hip.download(kv.k, np.uint16, m), hip.download(kv.v, np.uint16, m)))
        gm.close()
    for got, want, what in zip(outs[0], outs[1], ("logits", "x", "k", "v")):
        assert np.array_equal(got, want), what


def test_prefill_fp16_weight_copies_follow_reloaded_weights(hip):
    """The FP16 copies are a cache of the layer matrices: reloading a matrix after a prefill
    made them (gh_model_load_tensor) drops every copy, and the next prefill dequantizes the new
    weights again. A model that prefilled with one set of weights, then had block 0's Q, gate
    and down matrices replaced, prefills the same prompt bit for bit like a fresh model built
    with the new weights."""
    from graph_horizon_amd import _ffi as F

    shape = synth.SHAPES["small"]
    ctx, n = 320, 300
    old = list(synth.model_tensors(shape, 23))
    new = list(synth.model_tensors(shape, 24))
    swap = {(0, F.T_ATTN_Q), (0, F.T_FFN_GATE), (0, F.T_FFN_DOWN)}
    mixed = [nt if (nt[0], nt[1]) in swap else ot for ot, nt in zip(old, new)]
    toks = [int(t) for t in np.random.default_rng(5).integers(0, shape.vocab_size, n)]

    gm = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=512))
    for layer, tid, fmt, data in old:
        gm.load_tensor(layer, tid, fmt, data)
    gm.prefill(toks, 0)
    before = gm.read_logits().view(np.uint32).copy()
    for layer, tid, fmt, data in mixed:
        if (layer, tid) in swap:
            gm.load_tensor(layer, tid, fmt, data)
    gm.prefill(toks, 0)
    got = (gm.read_logits().view(np.uint32).copy(), gm.read_x().view(np.uint32).copy())
    gm.close()

    ref = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=512))
    for layer, tid, fmt, data in mixed:
        ref.load_tensor(layer, tid, fmt, data)
    ref.prefill(toks, 0)
    want = (ref.read_logits().view(np.uint32), ref.read_x().view(np.uint32))
    ref.close()
    assert not np.array_equal(before, want[0])  # the swap changes the result
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
