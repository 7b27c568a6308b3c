"""The fused paths past YaRN's original context, where the query post-scale is active.

The decode QKV GEMV epilogue and the prefill Q/K/V split reduce both rotate Q and K from the
RoPE table and scale Q alone by ln(floor(pos / 16384) + 1) * 0.1 + 1 (backend/rope.rs:91-100,
graph/block.rs:66-83, graph/prefill/layer.rs:79-89). Each scenario (yarn_long.SCENARIOS) puts a
prefill chunk or a run of greedy decode steps across position 16384 over a seeded KV cache:
  * the fused driver against every trait op recorded separately over the C ABI (whose
    standalone RoPE is bit-exact against the oracle at 16384 and 20000): logits, residual row
    and K/V cache rows bit for bit, after the prefill and after each teacher-forced step;
  * the graph-replayed greedy tokens against the stream-launched steps' argmax;
  * the oracle: logits within yarn_long.LOGIT_TOL of the logit scale (planted post-scale
    mistakes move them by more than three times that, test_oracle.py) and the new K/V rows
    within FP16 rounding;
  * at the 8B width (one block), the same against the oracle, where the fused Q/K/V launch
    splits K differently from the separate GEMMs (FP32 re-association only).
"""
import numpy as np
import pytest

import oracle as O
from graph_horizon_amd import HipModel, synth
import yarn_long as Y
from agreement import assert_agreement

pytestmark = pytest.mark.gpu


def _model(hip, shape, ts, base, ctx=Y.CTX):
    gm = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=512))
    for layer, tid, fmt, data in ts:
        gm.load_tensor(layer, tid, fmt, data)
    k, v = Y.seeded_kv(shape, base, ctx)
    kv = gm.kv()
    hip.upload(kv.k, k)
    hip.upload(kv.v, v)
    return gm


def _cache(hip, kv, shape, ctx):
    n = shape.block_count * ctx * shape.kv_head_count * shape.head_dim
    kvw = shape.kv_head_count * shape.head_dim
    return (hip.download(kv.k, np.uint16, n).reshape(shape.block_count, ctx, kvw),
            hip.download(kv.v, np.uint16, n).reshape(shape.block_count, ctx, kvw))


def _kv_close(got, want, lo, hi, what):
    g = O.f32(got[:, lo:hi]).astype(np.float64)
    w = O.f32(want.reshape(got.shape)[:, lo:hi]).astype(np.float64)
    # the projections sum in another order than the oracle's AVX2 loops, so many values round
    # to a neighbouring FP16 (a third of the K values of the tiny model's small-scale Q/K
    # weights, whose sums cancel heavily); a post-scale on K would move every row past 16384
    # by 7 %, tens of times both bounds
    err = np.abs(g - w)
    scale = max(np.abs(w).max(), 1.0)
    assert err.max() <= 4e-3 * scale, (what, float(err.max()), scale)
    assert err.mean() <= 5e-4 * scale, (what, float(err.mean()), scale)


@pytest.mark.parametrize("scenario", Y.SCENARIOS, ids=lambda s: f"n{s[0]}-base{s[1]}")
def test_fused_paths_across_16384_tiny(hip, scenario):
    from graph_over_abi import AbiGraph

    shape = synth.SHAPES["tiny"]
    n, base, steps = scenario
    ts = Y.tensors(shape)
    toks = Y.prompt(shape, n)
    print(f"long context: tiny n={n} base={base} steps={steps}", flush=True)
    gm = _model(hip, shape, ts, base)
    ref = AbiGraph(hip, shape, Y.SEED, Y.CTX, tensors=ts)
    k, v = Y.seeded_kv(shape, base)
    hip.upload(ref.kv.k, k)
    hip.upload(ref.kv.v, v)

    want = ref.prefill(toks, base)
    gm.prefill(toks, base)
    got = gm.read_logits()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    d = shape.embedding_length
    assert np.array_equal(gm.read_x().view(np.uint32), ref.prefill_x[(n - 1) * d:].view(np.uint32))
    first = gm.read_argmax()
    greedy = gm.decode_greedy(first, base + n, steps)  # the replayed step graph

    # the same steps launched op by op (fused kernels on the stream) against the trait ops,
    # teacher-forced on the graph's tokens
    tok, step_logits = first, []
    for i in range(steps):
        gm.token(tok, base + n + i)
        lg = gm.read_logits()
        w = ref.token(tok, base + n + i)
        assert np.array_equal(lg.view(np.uint32), w.view(np.uint32)), i
        assert int(np.argmax(lg)) == int(greedy[i]) or np.sort(lg)[-1] == np.sort(lg)[-2], i
        step_logits.append(lg)
        tok = int(greedy[i])
    end = base + n + steps
    gk, gv = _cache(hip, gm.kv(), shape, Y.CTX)
    rk, rv = _cache(hip, ref.kv, shape, Y.CTX)
    assert np.array_equal(gk[:, :end], rk[:, :end]) and np.array_equal(gv[:, :end], rv[:, :end])
    gm.close()

    # the oracle, teacher-forced on the device's tokens
    of, ol, ok, ov, _ = Y.oracle_run(shape, ts, scenario, forced=[first] + [int(t) for t in greedy])
    errs = [Y.logit_err(a, b) for a, b in zip([got] + step_logits, [of] + ol)]
    print(f"  max logit error / scale: {max(errs):.3g} (bar {Y.LOGIT_TOL})", flush=True)
    assert max(errs) <= Y.LOGIT_TOL, errs
    _kv_close(gk, ok, base, end, "K")
    _kv_close(gv, ov, base, end, "V")
    assert_agreement([first] + [int(t) for t in greedy], [of] + ol, f"tiny n={n} base={base}",
                     min_frac=1.0)


def test_fused_paths_across_16384_8b_width(hip):
    """One 8B-wide block (d 4096, FFN 12288, 32/8 heads), a 40-row prefill across 16384 and
    four greedy steps after it, against the oracle."""
    shape = Y.one_block("8b")
    scenario = (40, 16350, 4)
    n, base, steps = scenario
    ctx = 16448
    ts = Y.tensors(shape)
    print("long context: 8b-1 n=40 base=16350", flush=True)
    gm = _model(hip, shape, ts, base, ctx)
    gm.prefill(Y.prompt(shape, n), base)
    got = gm.read_logits()
    first = gm.read_argmax()
    greedy = gm.decode_greedy(first, base + n, steps)
    tok, step_logits = first, []
    for i in range(steps):
        gm.token(tok, base + n + i)
        step_logits.append(gm.read_logits())
        tok = int(greedy[i])
    gk, gv = _cache(hip, gm.kv(), shape, ctx)
    gm.close()
    of, ol, ok, ov, _ = Y.oracle_run(shape, ts, scenario, forced=[first] + [int(t) for t in greedy], ctx=ctx)
    errs = [Y.logit_err(a, b) for a, b in zip([got] + step_logits, [of] + ol)]
    print(f"  max logit error / scale: {max(errs):.3g} (bar {Y.LOGIT_TOL})", flush=True)
    assert max(errs) <= Y.LOGIT_TOL, errs
    end = base + n + steps
    _kv_close(gk, ok, base, end, "K")
    _kv_close(gv, ov, base, end, "V")
    assert_agreement([first] + [int(t) for t in greedy], [of] + ol, "8b-1 n=40", min_frac=1.0)
