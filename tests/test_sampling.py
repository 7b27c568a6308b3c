"""Host sampling of the graph driver (gh_sample*, sampling.rs:1-203) on the CPU.

libgh_hip.so's host functions against the Python restatement (oracle/sampling.py), which is
pinned here by the reference's own sampling tests (sampling.rs:206-298), by the generator's
uniformity, and by the empirical draw frequencies against the closed-form distributions.
"""
import ctypes as C

import numpy as np
import pytest

from graph_horizon_amd import _ffi as F
from oracle import sampling as S

F32 = np.float32


@pytest.fixture(scope="module")
def lib():
    return F.lib()


def params(temperature=0.0, top_p=1.0, top_k=0, min_p=0.0, repeat_penalty=1.0, seed=0):
    return dict(temperature=temperature, top_p=top_p, top_k=top_k, min_p=min_p,
                repeat_penalty=repeat_penalty, seed=seed)


def gh(p):
    return F.GhSampling(p["temperature"], p["top_p"], p["top_k"], p["min_p"], p["repeat_penalty"],
                        p["seed"])


def lib_sample(lib, logits, p, recent, state):
    l = np.ascontiguousarray(logits, dtype=F32).copy()
    r = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32))
    st = C.c_uint64(state)
    tok = C.c_uint32()
    sp = gh(p)
    assert lib.gh_sample(l.ctypes.data, l.size, C.byref(sp), r.ctypes.data if r.size else None, r.size,
                         C.byref(st), C.byref(tok)) == 0
    return tok.value, st.value, l


def lib_tail(lib, cand, p, state):
    idx = np.array([c[0] for c in cand], dtype=np.uint32)
    val = np.array([c[1] for c in cand], dtype=F32)
    st = C.c_uint64(state)
    tok = C.c_uint32()
    sp = gh(p)
    assert lib.gh_sample_from_candidates(idx.ctypes.data, val.ctypes.data, idx.size, C.byref(sp),
                                         C.byref(st), C.byref(tok)) == 0
    return tok.value, st.value


# ---- the reference's sampling tests (sampling.rs:206-298), on the oracle and the library
def test_reference_temperature_zero_is_exact_argmax(lib):
    l = np.array([0.1, 2.5, -1.0, 2.4], F32)
    assert S.sample(l.copy(), params(), [], S.rng_seed(0))[0] == 1
    assert lib_sample(lib, l, params(), [], S.rng_seed(0))[0] == 1


def test_reference_sampling_is_deterministic_for_a_seed(lib):
    p = params(temperature=1.0)
    l = np.array([1.0, 2.0, 3.0, 0.5], F32)
    draws = {S.sample(l.copy(), p, [], S.rng_seed(42))[0] for _ in range(3)}
    draws |= {lib_sample(lib, l, p, [], S.rng_seed(42))[0] for _ in range(3)}
    assert len(draws) == 1


def test_reference_top_k_one_collapses_to_argmax(lib):
    p = params(temperature=1.0, top_k=1)
    l = np.array([0.0, 5.0, 1.0], F32)
    assert S.sample(l.copy(), p, [], S.rng_seed(7))[0] == 1
    assert lib_sample(lib, l, p, [], S.rng_seed(7))[0] == 1


def test_reference_sample_equals_shared_tail(lib):
    p = params(temperature=0.8, top_p=0.95, min_p=0.05)
    logits = np.array([1.0, 2.0, 3.0, 0.5, -1.0, 4.0, 2.5], F32)
    seed = S.rng_seed(123)
    via_sample = lib_sample(lib, logits, p, [], seed)[0]
    inv = F32(1.0) / F32(0.8)
    cand = sorted([(i, F32(v * inv)) for i, v in enumerate(logits)], key=S.order_key)
    assert lib_tail(lib, cand, p, seed)[0] == via_sample
    assert S.sample_from_candidates(cand, p, seed)[0] == via_sample


def test_reference_plan_routes_paths(lib):
    def plan(p):
        k = C.c_uint32()
        sp = gh(p)
        return lib.gh_sampling_plan(C.byref(sp), C.byref(k)), k.value
    cases = [(params(), (F.SAMPLE_GREEDY, 0)), (params(temperature=1.0, top_k=40), (F.SAMPLE_TOPK, 40)),
             (params(temperature=1.0, top_k=129), (F.SAMPLE_FALLBACK, 0)),
             (params(repeat_penalty=1.1), (F.SAMPLE_FALLBACK, 0)),
             (params(temperature=1.0, top_k=0), (F.SAMPLE_FALLBACK, 0))]
    for p, want in cases:
        assert plan(p) == want
        assert S.plan(p) == want


# ---- the generator
def test_rng_matches_and_is_uniform(lib):
    for seed in (0, 1, 42, 2 ** 63 + 5):
        st = C.c_uint64(lib.gh_rng_seed(seed))
        assert st.value == S.rng_seed(seed) and st.value & 1
        ost = S.rng_seed(seed)
        for _ in range(64):
            u = lib.gh_rng_next_f32(C.byref(st))
            ost, ou = S.rng_next(ost)
            assert st.value == ost and F32(u) == ou
    st = S.rng_seed(9)
    us = []
    for _ in range(200000):
        st, u = S.rng_next(st)
        us.append(u)
    us = np.array(us, dtype=np.float64)
    assert us.min() >= 0 and us.max() < 1
    counts = np.histogram(us, bins=64, range=(0, 1))[0]
    chi2 = ((counts - 200000 / 64) ** 2 / (200000 / 64)).sum()
    assert chi2 < 120, chi2  # 63 degrees of freedom: p ~ 1e-5 at 120
    assert abs(us.mean() - 0.5) < 0.003


# ---- the library against the oracle over random cases
@pytest.mark.parametrize("seed", range(12))
def test_library_matches_oracle(lib, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 400))
    logits = (rng.standard_normal(n) * rng.uniform(0.5, 6)).astype(F32)
    logits[rng.integers(0, n, n // 6)] = logits[rng.integers(0, n, n // 6)]  # exact ties
    if seed % 3 == 0:
        logits[rng.integers(0, n, 3)] = [np.inf, -np.inf, np.nan]
    p = params(temperature=float(rng.choice([0.0, 0.3, 0.8, 1.0, 1.7])),
               top_p=float(rng.choice([1.0, 0.9, 0.5])), top_k=int(rng.choice([0, 1, 5, 40, 1000])),
               min_p=float(rng.choice([0.0, 0.05, 0.2])),
               repeat_penalty=float(rng.choice([1.0, 1.1, 1.3])), seed=int(rng.integers(0, 2 ** 32)))
    recent = rng.integers(0, n + 5, int(rng.integers(0, 30))).tolist()
    st = S.rng_seed(p["seed"])
    lst = st
    for _ in range(20):
        ol = logits.copy()
        want, st = S.sample(ol, p, recent, st)
        got, lst, ll = lib_sample(lib, logits, p, recent, lst)
        assert got == want and lst == st
        assert np.array_equal(ll.view(np.uint32), ol.view(np.uint32))  # penalty applied alike


# ---- the draws follow the closed-form distributions (pins softmax, nucleus, min-p, CDF)
def test_draw_frequencies(lib):
    l = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0], F32)
    for p, support in [(params(temperature=1.0, seed=1), None),
                       (params(temperature=0.7, top_p=0.8, seed=2), "top_p"),
                       (params(temperature=1.0, min_p=0.2, seed=3), "min_p")]:
        z = np.exp(l.astype(np.float64) / p["temperature"])
        prob = z / z.sum()
        if support == "top_p":
            keep = int(np.searchsorted(np.cumsum(prob), p["top_p"]) + 1)
            prob[keep:] = 0
        elif support == "min_p":
            prob[prob < p["min_p"] * prob[0]] = 0
        prob /= prob.sum()
        st = S.rng_seed(p["seed"])
        draws = 30000
        counts = np.zeros(l.size)
        for _ in range(draws):
            t, st, _ = lib_sample(lib, l, p, [], st)
            counts[t] += 1
        assert (counts[prob == 0] == 0).all()
        nz = prob > 0
        sd = np.sqrt(draws * prob[nz] * (1 - prob[nz])) + 1
        assert (np.abs(counts[nz] - draws * prob[nz]) < 5 * sd).all(), (counts, draws * prob)
