"""Shared set-up of the long-context parity checks: positions past YaRN's original context.

The query post-scale of backend/rope.rs:91-100 is ln(floor(pos / 16384) + 1) * 0.1 + 1 for the
query role and 1 for the key role, so it only departs from 1 from position 16384 on. These
scenarios put a prefill chunk or a run of decode steps across 16384, over a KV cache whose
earlier positions are seeded (no 16K-token prompt has to be run first).

Two choices keep a post-scale mistake visible in the logits:
  * the Q and K projections' block scales are divided by QK_DIV, so scores q.k/sqrt(128) have a
    spread of a few units and the softmax is not one-hot (a one-hot softmax ignores a change of
    temperature);
  * the seeded K/V rows have the statistics of the model's own K/V rows at that scale.
tests/test_oracle.py::test_long_context_checks_catch_post_scale_mistakes plants the mistakes in
the oracle and shows that they move the logits by several times LOGIT_TOL.
"""
from __future__ import annotations

import dataclasses

import numpy as np

import oracle as O
from graph_horizon_amd import synth
from graph_horizon_amd import _ffi as F

CTX = 16512
QK_DIV = 8.0
K_STD, V_STD = 1.5, 4.0
SEED = 61
LOGIT_TOL = 1.5e-2  # max |diff| of the logits, relative to the largest |logit| (at least 1)

# (prefill rows, base position, decode steps after it): the prefill crosses 16384 with a
# 128-token-tile chunk (40 rows) and with a 256-token-tile chunk over the FP16 weight copies
# (137 rows); the 8-row chunk ends below 16384 and its decode steps cross it.
SCENARIOS = [(40, 16350, 4), (8, 16370, 10), (137, 16300, 3)]


def tensors(shape, seed=SEED):
    """synth.model_tensors with the Q and K matrices' block scales divided by QK_DIV."""
    rng = np.random.default_rng(seed + 1)
    out = []
    for layer, tid, fmt, data in synth.model_tensors(shape, seed):
        if layer != F.NO_LAYER and tid in (F.T_ATTN_Q, F.T_ATTN_K):
            ind, outd = synth.tensor_dims(shape, tid)
            data = synth.quant_blocks(rng, fmt, outd, ind, synth.model_d_std(ind) / QK_DIV)
        out.append((layer, tid, fmt, data))
    return out


def seeded_kv(shape, base, ctx=CTX, seed=5):
    """FP16 K and V caches ([layer][ctx][kv_heads * head_dim]) with positions < base filled."""
    rng = np.random.default_rng(seed)
    kvw = shape.kv_head_count * shape.head_dim
    k = np.zeros((shape.block_count, ctx, kvw), np.uint16)
    v = np.zeros_like(k)
    k[:, :base] = O.f16(rng.standard_normal(shape.block_count * base * kvw) * K_STD).reshape(
        shape.block_count, base, kvw)
    v[:, :base] = O.f16(rng.standard_normal(shape.block_count * base * kvw) * V_STD).reshape(
        shape.block_count, base, kvw)
    return k.reshape(-1), v.reshape(-1)


def prompt(shape, n):
    return [int(t) for t in np.random.default_rng(n).integers(0, shape.vocab_size, n)]


def logit_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want))) / max(float(np.abs(want).max()), 1.0)


def one_block(name):
    return dataclasses.replace(synth.SHAPES[name], name=f"{name}-1", block_count=1)


def oracle_run(shape, ts, scenario, forced=None, plant=O.PLANT_NONE, ctx=CTX):
    """The oracle over one scenario: prefill logits, the K/V cache, and the logits of each
    decode step fed `forced` tokens (the oracle's own argmax chain when None). Returns
    (prefill_logits, [step logits], k_cache, v_cache, tokens fed)."""
    from test_oracle import oracle_model

    n, base, steps = scenario
    k, v = seeded_kv(shape, base, ctx)
    om, _ = oracle_model(shape, SEED, ctx, generated=ts)
    om.set_plant(plant)
    om.load_kv(k, v, ctx, base)
    om.prefill(prompt(shape, n), base, 512)
    first = om.logits()
    fed, step_logits = [], []
    tok = int(np.argmax(first)) if forced is None else int(forced[0])
    for i in range(steps):
        fed.append(tok)
        om.token(tok, base + n + i)
        lg = om.logits()
        step_logits.append(lg)
        if forced is None:
            tok = int(np.argmax(lg))
        elif i + 1 < steps:
            tok = int(forced[i + 1])
    kc, vc = om.kv(0), om.kv(1)
    om.close()
    return first, step_logits, kc, vc, fed
