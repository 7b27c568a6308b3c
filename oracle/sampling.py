"""Host token sampling, sampling.rs:1-203 restated in Python — TEST INFRASTRUCTURE.

Only tests/ may import this module. FP32 throughout, with sequential sums as the reference's
iterator folds; exp is the C library's expf (the reference's f32::exp lowers to it on Linux),
called through ctypes. Pinned in tests/test_sampling.py by the reference's own sampling tests
(sampling.rs:206-298), by the xorshift64* generator's uniformity, and by the empirical draw
frequencies against the closed-form softmax / nucleus / min-p distributions.
"""
from __future__ import annotations

import ctypes as C
import ctypes.util
import numpy as np

_libm = C.CDLL(ctypes.util.find_library("m"))
_libm.expf.restype = C.c_float
_libm.expf.argtypes = [C.c_float]
F32 = np.float32
MASK = (1 << 64) - 1
MAX_DEVICE_K = 128
GREEDY, TOPK, FALLBACK = 0, 1, 2


def expf(x) -> F32:
    return F32(_libm.expf(float(F32(x))))


def rng_seed(seed: int) -> int:
    """Rng::new, sampling.rs:20-26."""
    return ((seed ^ 0x9E3779B97F4A7C15) | 1) & MASK


def rng_next(state: int):
    """Rng::next_f32, sampling.rs:28-36: (new state, uniform in [0, 1) from the top 24 bits)."""
    x = state
    x ^= x >> 12
    x = (x ^ (x << 25)) & MASK
    x ^= x >> 27
    return x, F32(((x * 0x2545F4914F6CDD1D) & MASK) >> 40) / F32(1 << 24)


def total_key(v) -> int:
    b = int(np.asarray(v, dtype=F32).view(np.int32))
    return b ^ ((b >> 31) & 0x7FFFFFFF)


def order_key(c):
    """(logit desc by f32 total order, index asc) as an ascending sort key."""
    return (-total_key(c[1]), c[0])


def plan(p) -> tuple[int, int]:
    """sampling::plan, sampling.rs:180-192."""
    if F32(p["repeat_penalty"]) != F32(1.0):
        return FALLBACK, 0
    if F32(p["temperature"]) <= 0:
        return GREEDY, 0
    if 0 < p["top_k"] <= MAX_DEVICE_K:
        return TOPK, p["top_k"]
    return FALLBACK, 0


def argmax(logits) -> int:
    best, best_val = 0, F32(-np.inf)
    for i, v in enumerate(logits):
        if v > best_val:
            best, best_val = i, v
    return best


def sample_from_candidates(cand, p, state: int):
    """sampling.rs:99-155: softmax, top-p, min-p, inverse-CDF draw. Returns (token, state)."""
    if not cand:
        return 0, state
    cand = list(cand)
    mx = F32(cand[0][1])
    probs = [expf(F32(F32(l) - mx)) for _, l in cand]
    s = F32(0)
    for pr in probs:
        s = F32(s + pr)
    probs = [F32(pr / s) for pr in probs]
    if F32(p["top_p"]) < F32(1.0):
        cum, cut = F32(0), len(probs)
        for i, pr in enumerate(probs):
            cum = F32(cum + pr)
            if cum >= F32(p["top_p"]):
                cut = i + 1
                break
        cand, probs = cand[:cut], probs[:cut]
    if F32(p["min_p"]) > 0:
        thr = F32(F32(p["min_p"]) * probs[0])
        keep = 0
        while keep < len(probs) and probs[keep] >= thr:
            keep += 1
        keep = max(keep, 1)
        cand, probs = cand[:keep], probs[:keep]
    s = F32(0)
    for pr in probs:
        s = F32(s + pr)
    state, u = rng_next(state)
    r = F32(u * s)
    acc = F32(0)
    for i, pr in enumerate(probs):
        acc = F32(acc + pr)
        if r < acc:
            return cand[i][0], state
    return cand[-1][0], state


def sample(logits, p, recent, state: int):
    """sampling::sample, sampling.rs:40-94 (logits: float32 array, mutated). (token, state)."""
    rp = F32(p["repeat_penalty"])
    if rp != F32(1.0):
        for t in recent:
            if t < len(logits):
                v = logits[t]
                logits[t] = F32(v / rp) if v > 0 else F32(v * rp)
    if F32(p["temperature"]) <= 0:
        return argmax(logits), state
    inv = F32(F32(1.0) / F32(p["temperature"]))
    cand = [(i, F32(v * inv)) for i, v in enumerate(logits) if np.isfinite(v)]
    if not cand:
        return argmax(logits), state
    cand.sort(key=order_key)
    if 0 < p["top_k"] < len(cand):
        cand = cand[:p["top_k"]]
    return sample_from_candidates(cand, p, state)
