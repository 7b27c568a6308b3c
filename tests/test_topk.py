"""read_topk's ordering and the device top-k's key scheme, on the CPU.

The reference's order (cpu/readback.rs:59-69, sampling.rs) is `(logit desc by f32::total_cmp,
index asc)`. total_cmp is pinned here by its definition (the f32 bit pattern as i32, with the
low 31 bits flipped when negative), independently of the oracle's C++; the device kernels'
64-bit key and its inverse (kernels/glue.hip: gh_topk_partial / gh_topk_final) are pinned by
running the same stripe/merge decomposition in numpy.
"""
import numpy as np
import pytest

import oracle as O

SPECIALS = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001, 0x7F800000, 0xFF800000,
                     0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x3F800000, 0xBF800000],
                    dtype=np.uint32)  # ±NaN (two payloads), ±inf, ±0, ±denormal, ±1


def total_cmp_key(bits):
    """Rust f32::total_cmp: i32 of the bits, low 31 bits flipped for negative values."""
    b = np.asarray(bits, dtype=np.uint32).astype(np.int64)
    i = np.where(b >= 1 << 31, b - (1 << 32), b)
    return np.where(i < 0, i ^ 0x7FFFFFFF, i)


def want_topk(bits, k):
    key = total_cmp_key(bits)
    order = sorted(range(len(bits)), key=lambda j: (-int(key[j]), j))[:min(k, len(bits))]
    return [(j, int(bits[j])) for j in order]


def as_bits(pairs):
    return [(i, int(np.asarray(v, dtype=np.float32).view(np.uint32))) for i, v in pairs]


def _logits(rng, n, specials=True):
    bits = rng.standard_normal(n).astype(np.float32).view(np.uint32).copy()
    bits[rng.integers(0, n, n // 5)] = bits[rng.integers(0, n, n // 5)]  # many exact ties
    if specials:
        bits[rng.integers(0, n, 3 * SPECIALS.size)] = np.repeat(SPECIALS, 3)
    return bits


@pytest.mark.parametrize("n,k", [(12, 12), (12, 5), (300, 40), (5000, 128), (5000, 200)])
def test_oracle_topk_is_total_cmp_order(n, k):
    rng = np.random.default_rng(n + k)
    bits = SPECIALS.copy() if n == 12 else _logits(rng, n)
    got = as_bits(O.topk(bits.view(np.float32), k))
    assert got == want_topk(bits, k)


# ---- the device scheme, restated in numpy ----
def device_key(bits):
    b = np.asarray(bits, dtype=np.uint64)
    ordv = np.where(b >> 31 == 1, b ^ 0xFFFFFFFF, b ^ 0x80000000)
    return ((~ordv & 0xFFFFFFFF) << 32) | np.arange(b.size, dtype=np.uint64)


def device_value_bits(key):
    ordv = (~(key >> 32)) & 0xFFFFFFFF
    return np.where(ordv >> 31 == 1, ordv ^ 0x80000000, ordv ^ 0xFFFFFFFF)


def device_topk(bits, k, chunk=2048, max_stripes=128):
    n = bits.size
    k = min(k, n)
    width = 1 << (k - 1).bit_length()
    chunks = -(-n // chunk)
    per = chunk * -(-chunks // max_stripes)
    stripes = -(-n // per)
    keys = device_key(bits)
    pad = np.uint64(0xFFFFFFFFFFFFFFFF)
    lists = []
    for s in range(stripes):
        r = np.full(width, pad, dtype=np.uint64)
        for c in range(s * per, min(n, (s + 1) * per), chunk):
            blk = np.full(chunk, pad, dtype=np.uint64)
            part = keys[c:min(n, s * per + per, c + chunk)]
            blk[:part.size] = part
            blk.sort()
            r = np.sort(np.minimum(r, blk[:width][::-1]))
        lists.append(r)
    m = 1 << (stripes - 1).bit_length()
    lists += [np.full(width, pad, dtype=np.uint64)] * (m - stripes)
    while len(lists) > 1:
        h = len(lists) // 2
        lists = [np.sort(np.minimum(lists[i], lists[i + h][::-1])) for i in range(h)]
    top = lists[0][:k]
    return [(int(t & 0xFFFFFFFF), int(v)) for t, v in zip(top, device_value_bits(top))]


@pytest.mark.parametrize("n,k", [(5, 3), (12, 12), (3000, 1), (3000, 64), (131072, 40),
                                 (300001, 128), (700000, 100)])
def test_device_scheme_matches_oracle(n, k):
    rng = np.random.default_rng(n * 7 + k)
    bits = SPECIALS.copy() if n == 12 else _logits(rng, n, specials=n > 5)
    want = as_bits(O.topk(bits.view(np.float32), k))
    assert device_topk(bits, k) == want
