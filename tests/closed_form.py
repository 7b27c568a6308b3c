"""Closed-form one-layer models (test helper, not collected).

A one-layer Ministral-shaped model whose FFN down matrix (or attention O matrix) is all zeros
has logits that follow from a few dense products, so they can be computed in fp64 with numpy
from the dequantized weights alone — no graph code, no attention kernel, no GEMV kernel:

  x0 = embed(token)                                   (the dequantized token row, FP32)
  zero_ffn:  at position 0 the softmax has one term of weight exp(0) = 1, so each query head
             h attends exactly V of its kv head h // G:
             n0 = f16(rmsnorm(x0, attn_norm)), v = f16(W_v n0), a[h] = v[h // G],
             x1 = x0 + f32(f16(W_o a))             (the FFN adds f16(0) = 0)
  zero_o:    x0 passes the attention block unchanged (f16(W_o a) = 0);
             n1 = f16(rmsnorm(x0, ffn_norm)), g = f16(W_gate n1), u = f16(W_up n1),
             x1 = x0 + f32(f16(W_down f16(f16(silu(g)) u)))
  logits = W_out f16(rmsnorm(x1, output_norm)), W_out = output, or token_embd when tied.

The FP16 rounding points are the contract's (graph/block.rs:17-107, mlp.rs:12-61,
tail.rs:22-59, activation.rs:16-29). The dense products run in fp64, so a model's FP32
result differs only where an FP16 intermediate lands on the other side of a rounding
boundary; a wiring mistake (K for V, a swapped norm, gate/up exchanged, a dropped residual,
the wrong output matrix) moves the logits by orders of magnitude more (`plant` shows it).
"""
from __future__ import annotations

import numpy as np

import oracle as O
from graph_horizon_amd import synth
from graph_horizon_amd import _ffi as F

SHAPE = synth.Shape("closed-form", 1, 512, 1024, head_count=8, kv_head_count=2, vocab_size=2048)
EPS = 1e-5
# |model - closed form| <= TOL * (|closed form| + rms(closed form)): FP16 boundary flips only
# (measured up to 3e-4 on the oracle; planted wiring mistakes measure 0.026 and up)
TOL = 2e-3


def tensors(variant: str, tied: bool, seed: int):
    """synth.model_tensors of SHAPE with the down (zero_ffn) or O (zero_o) matrix zeroed and,
    when tied, no output matrix."""
    zero_tid = {"zero_ffn": F.T_FFN_DOWN, "zero_o": F.T_ATTN_OUTPUT}[variant]
    rng = np.random.default_rng(seed + 1000)
    d = SHAPE.embedding_length
    out = []
    for layer, tid, fmt, data in synth.model_tensors(SHAPE, seed):
        if layer == F.NO_LAYER and tid == F.T_OUTPUT and tied:
            continue
        if layer != F.NO_LAYER and tid == zero_tid:
            data = np.zeros_like(data)
        elif fmt == F.FMT_F32:
            # norm weights far apart (a swapped norm must show), FP32 in the file
            data = (1.0 + 0.4 * rng.standard_normal(d)).astype(np.float32)
        elif tid == F.T_TOKEN_EMBD:
            # embedding rows at the branch's scale (a dropped residual must show)
            data = synth.q4k_blocks(rng, SHAPE.vocab_size, d, synth.model_d_std(d) * 64.0)
        out.append((layer, tid, fmt, data))
    return out


def _table(ts):
    return {(layer, tid): (fmt, data) for layer, tid, fmt, data in ts}


def _dense(t, layer, tid):
    fmt, data = t[(layer, tid)]
    if layer == F.NO_LAYER:
        ind, outd = SHAPE.embedding_length, SHAPE.vocab_size
    else:
        ind, outd = synth.tensor_dims(SHAPE, tid)
    return O.dequant(fmt, data, outd, ind).astype(np.float64)


def _f16(x):
    """fp64 -> FP16 (numpy's correctly rounded, round-half-even narrowing) -> fp64."""
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def _rms(x, w32):
    """rmsnorm_x (normalization.rs:12-40) in fp64 with the FP16 weight the model loads."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w32, np.float32).astype(np.float16).astype(np.float64)
    return _f16(x / np.sqrt(np.mean(x * x) + EPS) * w)


def logits(ts, variant: str, token: int, plant: str | None = None):
    """The closed-form logits of the one-layer model at position 0. `plant` injects one wiring
    mistake (for showing that the check catches it): 'k_for_v', 'norm_swap', 'gate_up_swap',
    'drop_residual', 'wrong_output'."""
    t = _table(ts)
    s = SHAPE
    group = s.head_count // s.kv_head_count
    norm = lambda tid: t[(0, tid)][1]  # noqa: E731
    x0 = _dense(t, F.NO_LAYER, F.T_TOKEN_EMBD)[token].astype(np.float32)
    attn_norm, ffn_norm = F.T_ATTN_NORM, F.T_FFN_NORM
    if plant == "norm_swap":
        attn_norm, ffn_norm = ffn_norm, attn_norm
    if variant == "zero_ffn":
        n0 = _rms(x0, norm(attn_norm))
        v = _f16(_dense(t, 0, F.T_ATTN_K if plant == "k_for_v" else F.T_ATTN_V) @ n0)
        v = v.reshape(s.kv_head_count, s.head_dim)
        a = np.concatenate([v[h // group] for h in range(s.head_count)])
        branch = _f16(_dense(t, 0, F.T_ATTN_OUTPUT) @ a)
    else:
        n1 = _rms(x0, norm(ffn_norm))
        g = _f16(_dense(t, 0, F.T_FFN_GATE) @ n1)
        u = _f16(_dense(t, 0, F.T_FFN_UP) @ n1)
        if plant == "gate_up_swap":
            g, u = u, g
        act = _f16(_f16(g / (1.0 + np.exp(-g))) * u)
        branch = _f16(_dense(t, 0, F.T_FFN_DOWN) @ act)
    x1 = branch.astype(np.float32) if plant == "drop_residual" else x0 + branch.astype(np.float32)
    tied = (F.NO_LAYER, F.T_OUTPUT) not in t
    use_embd = tied != (plant == "wrong_output")
    if use_embd:
        w_out = _dense(t, F.NO_LAYER, F.T_TOKEN_EMBD)
    elif (F.NO_LAYER, F.T_OUTPUT) in t:
        w_out = _dense(t, F.NO_LAYER, F.T_OUTPUT)
    else:  # tied model, planted mistake: any other matrix of the vocabulary's shape
        w_out = _dense(t, F.NO_LAYER, F.T_TOKEN_EMBD)[::-1]
    return w_out @ _rms(x1, t[(F.NO_LAYER, F.T_OUTPUT_NORM)][1])


def error(got, want):
    """max |got - want| / (|want| + rms(want)): below TOL for a correct model."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want) / (np.abs(want) + np.sqrt(np.mean(want * want)))))


def oracle_cfg(kv_context: int = 32) -> O.ModelCfg:
    s = SHAPE
    return O.ModelCfg(s.block_count, 32768, s.embedding_length, s.feed_forward_length,
                      s.head_count, s.kv_head_count, s.head_dim, s.head_dim, s.vocab_size, EPS,
                      O.Yarn(**synth.yarn_params(s)))


def oracle_model(ts, kv_context: int = 32) -> O.Model:
    table = {("g", tid) if layer == F.NO_LAYER else (layer, tid): (fmt, data)
             for layer, tid, fmt, data in ts}
    return O.Model(oracle_cfg(kv_context), table, kv_context)
