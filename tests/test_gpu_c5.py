"""BASELINE configs[4] at its stated workload: the 14B-shaped Q4_K_M decoder (40 blocks, d 5120,
FFN 16384, 32/8 heads x 128, vocab 131072; attn_v / ffn_down / output Q6_K, the rest Q4_K)
with a 512-token random-id prompt and 256 greedy decode steps through the replayed HIP graph
(generation/mod.rs:75-148).

The CPU oracle cannot prefill 512 tokens through 40 blocks within a test (about 12 s per
block), so it resumes from the device's prefilled KV cache: seeded with the device's K/V of
positions < p, it recomputes position p through all 40 blocks itself — the prompt's last row
(its logits and its K/V entries against the device prefill's) and 64 decode steps
teacher-forced on the device's greedy tokens (>= 99 % top-1 agreement; near ties, counted and
printed, excepted).
"""
import numpy as np
import pytest

import oracle as O
from agreement import assert_agreement
from graph_horizon_amd import HipModel, synth
from graph_horizon_amd import _ffi as F
from test_oracle import oracle_model

pytestmark = pytest.mark.gpu

PROMPT, STEPS, CTX = 512, 256, 1024
ORACLE_STEPS = 64


def _close(got, want, what, rel=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    scale = max(float(np.abs(want).max()), 1.0)
    err = float(np.max(np.abs(got - want)))
    assert err <= rel * scale, f"{what}: max |diff| {err:.4g} > {rel} x {scale:.4g}"


def _kv_host(hip, kv, shape):
    n = shape.block_count * CTX * shape.kv_head_count * shape.head_dim
    return hip.download(kv.k, np.uint16, n), hip.download(kv.v, np.uint16, n)


def test_c5_14b_prompt_512_greedy_256(hip):
    shape = synth.SHAPES["14b"]
    seed = 1405
    tensors = list(synth.model_tensors(shape, seed))
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, shape.vocab_size, PROMPT)]

    gm = HipModel(hip, synth.model_config(shape, CTX, prefill_rows=PROMPT))
    for layer, tid, fmt, data in tensors:
        gm.load_tensor(layer, tid, fmt, data)
    gm.prefill(prompt, 0)
    prefill_logits = gm.read_logits()
    assert np.isfinite(prefill_logits).all()
    k_dev, v_dev = _kv_host(hip, gm.kv(), shape)
    first = gm.read_argmax()
    toks = gm.decode_greedy(first, PROMPT, STEPS)
    assert np.isfinite(gm.read_logits()).all()
    assert ((toks >= 0) & (toks < shape.vocab_size)).all()

    # the same prompt in two prefill calls (256 + 256 rows, the second attending across the
    # first's KV) gives the one-batch logits within the model tolerance
    gm.prefill(prompt[:PROMPT // 2], 0)
    gm.prefill(prompt[PROMPT // 2:], PROMPT // 2)
    _close(gm.read_logits(), prefill_logits, "chunked vs single-chunk prefill")
    gm.close()

    # the decode steps launched on the stream (no graph) reproduce the graph's tokens
    sm = HipModel(hip, synth.model_config(shape, CTX, prefill_rows=PROMPT, flags=F.MODEL_NO_GRAPH))
    for layer, tid, fmt, data in tensors:
        sm.load_tensor(layer, tid, fmt, data)
    sm.prefill(prompt, 0)
    assert np.array_equal(sm.read_logits().view(np.uint32), prefill_logits.view(np.uint32))
    assert np.array_equal(sm.decode_greedy(first, PROMPT, 32), toks[:32])
    sm.close()

    # oracle, resumed from the device's cache of the first 511 prompt positions
    om, _ = oracle_model(shape, seed, CTX, tensors)
    del tensors
    om.load_kv(k_dev, v_dev, CTX, PROMPT - 1)
    om.token(prompt[-1], PROMPT - 1)
    _close(prefill_logits, om.logits(), "prompt's last row vs oracle")
    ora = [om.logits()]
    # the row's K and V in every layer (K after RoPE), within the FP16 model tolerance
    kv_row = shape.kv_head_count * shape.head_dim
    for role, dev in ((0, k_dev), (1, v_dev)):
        want = O.f32(om.kv(role)).reshape(shape.block_count, CTX, kv_row)[:, PROMPT - 1]
        got = O.f32(dev).reshape(shape.block_count, CTX, kv_row)[:, PROMPT - 1]
        _close(got, want, f"KV role {role} at position {PROMPT - 1}")
    # 64 decode steps teacher-forced on the device's tokens
    tok = first
    for i in range(ORACLE_STEPS):
        om.token(tok, PROMPT + i)
        ora.append(om.logits())
        tok = int(toks[i])
    om.close()
    assert_agreement([first] + [int(t) for t in toks[:ORACLE_STEPS]], ora,
                     f"C5 14B, prompt row and {ORACLE_STEPS} greedy steps")
