"""GPU checks that do not route through the oracle's own formulas: the reference's op trace,
closed-form one-layer models (dedicated and tied output), the tied output against the oracle,
and exhaustive FP16 widening / narrowing sweeps on the device.
"""
import json
import os

import numpy as np
import pytest

import closed_form as CF
from agreement import assert_agreement
import oracle as O
from graph_horizon_amd import HipModel, synth
from graph_horizon_amd import _ffi as F

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_op_trace.json")


def _load(gm, ts):
    for layer, tid, fmt, data in ts:
        gm.load_tensor(layer, tid, fmt, data)


# ---------------------------------------------------------------- op trace over the C ABI
@pytest.mark.parametrize("row", [0, 1, 2])
def test_abi_op_trace_matches_reference(hip, row):
    """forward::token recorded op by op over the C ABI (tests/graph_over_abi.py, which the
    fused driver is bit-identical to) logs exactly the reference's shape-recorder trace for
    each REFERENCE_ROWS entry's block count and output kind (graph/shape.rs:389-446)."""
    from graph_over_abi import AbiGraph
    from test_oracle import expected_op_trace

    with open(GOLDEN) as f:
        golden = json.load(f)
    blocks, _, _, dedicated = golden["reference_rows"][row]
    shape = synth.Shape("trace", blocks, 256, 256, head_count=2, kv_head_count=1, vocab_size=64)
    g = AbiGraph(hip, shape, 70 + row, 8, tied=not dedicated)
    trace = []
    g.token(3, 0, trace=trace)
    assert trace == expected_op_trace(golden, blocks, dedicated)


# ---------------------------------------------------------------- closed-form one-layer models
@pytest.mark.parametrize("variant", ["zero_ffn", "zero_o"])
@pytest.mark.parametrize("tied", [False, True], ids=["dedicated", "tied"])
def test_closed_form_one_layer_model(hip, variant, tied):
    """The fused decode driver's logits equal the fp64 closed form (tests/closed_form.py) of a
    one-layer model with a zero down (zero_ffn) or O (zero_o) matrix, for the dedicated and
    the tied output; a wiring mistake would be 5x the tolerance or more (shown on the CPU in
    test_oracle.py)."""
    ts = CF.tensors(variant, tied, 80 + 2 * (variant == "zero_o") + tied)
    gm = HipModel(hip, synth.model_config(CF.SHAPE, 32, 16))
    _load(gm, ts)
    for token in (5, 2000):
        gm.token(token, 0)
        got = gm.read_logits()
        want = CF.logits(ts, variant, token)
        err = CF.error(got, want)
        assert err < CF.TOL, (variant, tied, token, err)
    gm.close()


# ---------------------------------------------------------------- tied output vs the oracle
def test_tied_output_matches_oracle(hip):
    """tail.rs:43-58: with no output matrix the logits read token_embd. The driver (decode
    steps and the replayed greedy graph) against the oracle on the same tied model."""
    from test_oracle import oracle_model

    shape = synth.SHAPES["tiny"]
    ts = [t for t in synth.model_tensors(shape, 90) if not (t[0] == F.NO_LAYER and t[1] == F.T_OUTPUT)]
    gm = HipModel(hip, synth.model_config(shape, 128, 16))
    _load(gm, ts)
    om, _ = oracle_model(shape, 0, 128, generated=ts)
    for p, t in enumerate([7, 1500, 33, 2047, 640]):
        gm.token(t, p)
        om.token(t, p)
        want = om.logits()
        # the tied logits are token_embd rows (16x the output matrix's scale here): the
        # model tolerance 2e-2 relative, with the absolute floor scaled by their RMS
        rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
        assert np.allclose(gm.read_logits(), want, rtol=2e-2, atol=2e-2 * rms), p
    # replayed greedy graph, teacher-forced against the oracle
    first = int(np.argmax(om.logits()))
    toks = gm.decode_greedy(first, 5, 24)
    tok, ora = first, []
    for i in range(24):
        om.token(tok, 5 + i)
        ora.append(om.logits())
        tok = int(toks[i])
    assert_agreement(toks, ora, "tied output, 24 greedy steps", min_frac=1.0)
    gm.close()
    om.close()


# ---------------------------------------------------------------- FP16 conversion on the device
def test_f16_widening_all_patterns_on_device(hip):
    """All 65,536 FP16 patterns widened on the device (v_cvt_f32_f16 inside gh_residual_add,
    x = -0.0, so x + f32(y) = f32(y) exactly): bit-identical to numpy's binary16 widening for
    every non-NaN pattern (signed zeros, subnormals, infinities) and to the oracle's
    residual_add for every pattern; NaNs stay NaN (backend/f16.rs:11-37, cpu/f16.rs:131-168)."""
    y = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = np.full(65536, -0.0, np.float32)
    xb, yb = hip.from_host(x), hip.from_host(y)
    hip.residual_add(xb, yb, 65536)
    got = hip.download(xb, np.float32, 65536)
    want = x.copy()
    O.lib().gho_residual_add(want.ctypes.data, y.ctypes.data, 65536)
    nan = np.isnan(y.view(np.float16))
    assert np.array_equal(got.view(np.uint32)[~nan],
                          y.view(np.float16).astype(np.float32).view(np.uint32)[~nan])
    assert np.all(np.isnan(got[nan]))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    hip.free_buffer(xb)
    hip.free_buffer(yb)


def test_f16_narrowing_sweep_on_device(hip):
    """FP32 -> FP16 narrowing on the device (v_cvt_f16_f32 in gh_silu_mul's final rounding):
    for gate values g >= 16, f16(silu(g)) = g exactly, so the kernel stores f16(g * u) with
    g * u an exact FP32 product. u runs over all 65,536 patterns against four g values, which
    covers overflow to infinity, subnormal results, exact ties, signed zeros, infinities and
    NaNs. Bit-identical to numpy's round-half-even narrowing of the same product (non-NaN)
    and to the oracle's silu_mul for every element, NaN payloads included: the reference
    writes FP16 buffers through F16C vcvtps2ph in 8-element chunks (backend/cpu/f16.rs:86-102),
    which keeps a NaN's sign and top payload bits, as the device conversion does."""
    u = np.tile(np.arange(65536, dtype=np.uint32).astype(np.uint16), 4)
    gv = np.array([16.0, 17.5, 1000.0, 60000.0], np.float16)
    assert np.array_equal((gv.astype(np.float64) / (1.0 + np.exp(-gv.astype(np.float64)))).astype(np.float16), gv)
    g = np.repeat(gv, 65536).view(np.uint16)
    gb, ub, ob = hip.from_host(g), hip.from_host(u), hip.alloc_buffer(g.size * 2)
    hip.silu_mul(ob, gb, ub, g.size)
    got = hip.download(ob, np.uint16, g.size)
    with np.errstate(over="ignore", invalid="ignore"):
        prod = g.view(np.float16).astype(np.float32) * u.view(np.float16).astype(np.float32)
        want = prod.astype(np.float16).view(np.uint16)
    nan = np.isnan(prod)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7E00) == 0x7E00)  # quiet NaNs
    assert np.array_equal(got, O.silu_mul(g, u))
    # the sweep reaches the cases it is for
    half = (prod.view(np.uint32) & 0x1FFF) == 0x1000
    with np.errstate(over="ignore"):
        assert (np.isinf(prod.astype(np.float16)) & np.isfinite(prod)).any()  # overflow
    assert (np.abs(prod) < 2.0 ** -14).any() and half.sum() > 100       # subnormals, ties
    for b in (gb, ub, ob):
        hip.free_buffer(b)


# ---------------------------------------------------------------- RoPE tables
def test_model_rope_table_survives_other_yarn_calls(hip):
    """A model's decode reads its own YaRN table: gh_rope_yarn with other parameters (which
    rebuilds the backend's table, here for 6000 positions) between two decode steps, graph
    replay included, leaves the model's logits equal to the oracle's."""
    from graph_horizon_amd import GhError, Yarn
    from test_oracle import oracle_model

    shape = synth.SHAPES["tiny"]
    gm = HipModel(hip, synth.model_config(shape, 64, 16))
    for layer, tid, fmt, data in synth.model_tensors(shape, 91):
        gm.load_tensor(layer, tid, fmt, data)
    om, _ = oracle_model(shape, 91, 64)
    other = Yarn(rope_dim=64, original_context=4096, freq_base=1e4, factor=4.0, beta_fast=16.0,
                 beta_slow=2.0, log_multiplier=0.5, q_temperature_scale=0.3)
    x = hip.from_host(np.zeros(4 * 128, np.uint16))
    for pos, tok in enumerate([5, 600, 1999]):
        hip.rope_yarn(x, 4, 128, 6000 - pos, other, F.ROPE_QUERY)
        gm.token(tok, pos)
        om.token(tok, pos)
        assert np.allclose(gm.read_logits(), om.logits(), rtol=2e-2, atol=2e-2), pos
    hip.rope_yarn(x, 4, 128, 10, other, F.ROPE_KEY)
    toks = gm.decode_greedy(7, 3, 4)
    hip.rope_yarn(x, 4, 128, 7, Yarn(**synth.yarn_params(shape)), F.ROPE_KEY)
    again = gm.decode_greedy(7, 3, 4)
    assert np.array_equal(toks, again)
    # positions past the table limit (MAX_CONTEXT) are rejected, including u32 wrap-around
    for pos in (262144, 0xFFFFFFFF):
        with pytest.raises(GhError):
            hip.rope_yarn(x, 4, 128, pos, other, F.ROPE_QUERY)
    hip.free_buffer(x)
    gm.close()
    om.close()
