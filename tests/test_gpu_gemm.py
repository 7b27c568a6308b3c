"""Matrix-core prefill GEMM (gh_matmul_batched with n >= 8 tokens) against the oracle.

Bars:
  * kernel arithmetic: against an fp64 product of the FP16-rounded reference-dequantized
    weights (the GEMM's stated operands), |got - want| <= 1e-3·|want| + 2e-6·Σ|terms| — FP32
    accumulation plus the FP16 rounding of the output (2^-11 relative at most);
  * reference CPU kernel (q4k.rs:218-325 / q6k.rs:157-235 restated in the oracle) on the same
    seeded inputs: the bar above widened by + 2^-12·Σ|terms| for the FP16 rounding of the
    weights. Each rounded weight is within 2^-11 of its FP32 value (the worst-case envelope
    2^-11·Σ|terms|); the errors of thousands of independently rounded weights cancel, and
    the measured deviation (printed, run with -s) stays far below half that envelope;
  * the reference's own prefill parity tests (vulkan/kernels/matmul/prefill/mod.rs:160-300,
    330-450): their weight/activation generators and shapes, their bar
    |got - want| <= 5e-2 or <= 5e-3·max(|want|, 1) (mod.rs:275,440).
"""
import numpy as np
import pytest

import oracle as O
from graph_horizon_amd import synth
from graph_horizon_amd import _ffi as F

pytestmark = pytest.mark.gpu


def _f16_weights(fmt, w, rows, in_dim):
    deq = O.dequant(fmt, w, rows, in_dim)  # bit-exact reference dequantization (FP32)
    return deq.astype(np.float16).astype(np.float64)  # round-to-nearest-even to FP16


def _run(hip, fmt, rows, in_dim, n, seed, d_std=0.02):
    rng = np.random.default_rng(seed)
    w = synth.quant_blocks(rng, fmt, rows, in_dim, d_std)
    a16 = O.f16(rng.standard_normal(n * in_dim).astype(np.float32))
    wb = hip.load_weight(fmt, w, in_dim, rows)
    ab = hip.from_host(a16)
    ob = hip.alloc_buffer(n * rows * 2)
    hip.matmul_batched(ob, ab, wb, in_dim, rows, n)
    got = O.f32(hip.download(ob, np.uint16, n * rows)).reshape(n, rows).astype(np.float64)
    for b in (wb, ab, ob):
        hip.free_buffer(b)
    return w, a16, got


def _check_fp64(fmt, w, a16, got, rows, in_dim, n, what, f16_weights=True):
    w16 = (_f16_weights(fmt, w, rows, in_dim) if f16_weights
           else O.dequant(fmt, w, rows, in_dim).astype(np.float64))
    a = O.f32(a16).astype(np.float64).reshape(n, in_dim)
    want = a @ w16.T
    scale = np.abs(a) @ np.abs(w16).T
    tol = 1e-3 * np.abs(want) + 2e-6 * scale
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside, worst " \
        f"{np.max(np.abs(got - want) / tol):.3f}x tol"


def _check_reference(fmt, w, a16, got, rows, in_dim, n, what, tokens=None):
    tokens = range(n) if tokens is None else tokens
    deq = O.dequant(fmt, w, rows, in_dim).astype(np.float64)
    worst = 0.0
    for t in tokens:
        x = a16[t * in_dim:(t + 1) * in_dim]
        want = O.f32(O.matmul_batched(fmt, x, w, in_dim, rows, 1)).astype(np.float64)
        terms = np.abs(deq) @ np.abs(O.f32(x).astype(np.float64))
        tol = 1e-3 * np.abs(want) + (2e-6 + 2.0 ** -12) * terms
        dev = np.abs(got[t] - want)
        worst = max(worst, float(np.max(np.maximum(dev - 1e-3 * np.abs(want), 0.0) / terms)))
        bad = dev > tol
        assert not bad.any(), f"{what} token {t}: {bad.sum()} outside the FP16-weight envelope"
    print(f"{what}: worst deviation from the reference kernel beyond the output rounding "
          f"= {worst:.3e}·Σ|terms| (envelope 2^-11 = {2.0 ** -11:.3e}, bar 2^-12 + 2e-6)")


def _reference_bar(got, want, what):
    err = np.abs(got - want)
    ok = (err <= 5e-2) | (err <= 5e-3 * np.maximum(np.abs(want), 1.0))
    assert ok.all(), f"{what}: {(~ok).sum()} of {ok.size} outside the reference prefill bar"


@pytest.mark.parametrize("fmt,rows,in_dim,n", [
    (F.FMT_Q4_K, 128, 256, 8),      # smallest: one tile, four units, no split
    (F.FMT_Q4_K, 300, 1024, 37),    # ragged rows and tokens
    (F.FMT_Q6_K, 300, 1024, 130),   # ragged, two token tiles
    (F.FMT_Q4_K, 200, 4096, 129),   # split-K
    (F.FMT_Q6_K, 130, 12288, 64),   # down-projection depth, 16 splits
    (F.FMT_Q6_K, 1024, 5120, 200),  # 14B-shaped V projection
    # 256 tokens and more: the warp-specialized kernels
    (F.FMT_Q4_K, 96, 256, 257),     # smallest: one row tile, a one-token second token tile
    (F.FMT_Q4_K, 1000, 2048, 300),  # narrow output, 96-row tiles, split-K, ragged rows/tokens
    (F.FMT_Q6_K, 2000, 3072, 256),  # one token tile, ragged rows
    (F.FMT_Q6_K, 640, 8448, 700),   # 132 units: 16 splits shrunk to 15 (none empty)
    (F.FMT_Q4_K, 4096, 4096, 384),  # 128-row tiles with split-K
])
def test_gemm_parity(hip, fmt, rows, in_dim, n):
    w, a16, got = _run(hip, fmt, rows, in_dim, n, 7 + rows + n)
    assert np.isfinite(got).all()
    _check_fp64(fmt, w, a16, got, rows, in_dim, n, f"{fmt} {rows}x{in_dim} n={n}")
    _check_reference(fmt, w, a16, got, rows, in_dim, n, f"{fmt} {rows}x{in_dim}",
                     tokens=range(0, n, max(1, n // 8)))


@pytest.mark.parametrize("fmt,rows,in_dim", [(F.FMT_Q4_K, 12288, 4096), (F.FMT_Q6_K, 4096, 12288)])
def test_gemm_c3_full_size(hip, fmt, rows, in_dim):
    """The 512-token prefill GEMMs at full size (gate/up and down of the 8B-shaped block)."""
    n = 512
    w, a16, got = _run(hip, fmt, rows, in_dim, n, 4242 + fmt)
    assert np.isfinite(got).all()
    _check_fp64(fmt, w, a16, got, rows, in_dim, n, f"C3 {fmt} {rows}x{in_dim}")
    _check_reference(fmt, w, a16, got, rows, in_dim, n, f"C3 {fmt}", tokens=[0, 1, 255, 511])


def test_gemm_equals_gemv_within_tolerance_at_threshold(hip):
    """n = 7 runs the GEMV (exact quant arithmetic), n = 8 the GEMM (FP16 weight tiles): each
    meets the fp64 bar of its own operands on the same data."""
    fmt, rows, in_dim = F.FMT_Q4_K, 256, 2048
    rng = np.random.default_rng(99)
    w = synth.quant_blocks(rng, fmt, rows, in_dim, 0.02)
    a16 = O.f16(rng.standard_normal(8 * in_dim).astype(np.float32))
    wb, ab = hip.load_weight(fmt, w, in_dim, rows), hip.from_host(a16)
    ob = hip.alloc_buffer(8 * rows * 2)
    for n in (7, 8):
        hip.matmul_batched(ob, ab, wb, in_dim, rows, n)
        got = O.f32(hip.download(ob, np.uint16, n * rows)).reshape(n, rows).astype(np.float64)
        _check_fp64(fmt, w, a16[:n * in_dim], got, rows, in_dim, n, f"n={n}", f16_weights=n >= 8)
    for b in (wb, ab, ob):
        hip.free_buffer(b)


def _lcg(count, seed=0x9E3779B9):
    """The reference test generator, seed = seed * 1664525 + 1013904223 (mod 2^32), as the
    array of its first `count` outputs (blocks of M steps advanced with the M-step map)."""
    a, c, m, M = 1664525, 1013904223, 0xFFFFFFFF, 65536
    first = np.empty(M, np.uint64)
    for i in range(M):
        seed = (seed * a + c) & m
        first[i] = seed
    am, cm = 1, 0  # s -> am·s + cm is M steps
    for _ in range(M):
        am, cm = (am * a) & m, (cm * a + c) & m
    out = np.empty(((count + M - 1) // M) * M, np.uint64)
    blk = first
    for b in range(len(out) // M):
        out[b * M:(b + 1) * M] = blk
        blk = (blk * np.uint64(am) + np.uint64(cm)) & np.uint64(m)
    return out[:count]


def _reference_q4k_case(in_dim, out_dim, n):
    """q4k_cpu_oracle inputs (prefill/mod.rs:190-215): LCG bytes, d = 0.03, dmin = 0.01,
    activations (rng >> 8) / u32::MAX - 0.5 in FP32, narrowed to FP16 for the device."""
    nbytes = out_dim * (in_dim // 256) * 144
    stream = _lcg(nbytes + n * in_dim)
    q = ((stream[:nbytes] >> np.uint64(16)) & np.uint64(0xFF)).astype(np.uint8)
    blocks = q.reshape(-1, 144)
    blocks[:, 0:2] = np.frombuffer(np.float16(0.03).tobytes(), np.uint8)
    blocks[:, 2:4] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    vals = (stream[nbytes:] >> np.uint64(8)).astype(np.float32)
    act = vals / np.float32(4294967295.0) - np.float32(0.5)
    return q, O.f16(act.astype(np.float32))


def _reference_q6k_case(in_dim, out_dim, n):
    """q6k_cpu_oracle inputs (prefill/mod.rs:360-385): byte i of block b = 17 i + b (mod 256),
    scales i % 7 + 1, d = 0.01; activations (i % 31) / 32 - 0.5."""
    nblk = out_dim * (in_dim // 256)
    q = np.zeros((nblk, 210), np.uint8)
    idx = np.arange(192, dtype=np.uint32)
    for b in range(nblk):
        q[b, :192] = ((idx * 17) + (b & 0xFF)) & 0xFF
    q[:, 192:208] = (np.arange(16) % 7 + 1).astype(np.uint8)
    q[:, 208:210] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    act = (np.arange(n * in_dim) % 31).astype(np.float32) / np.float32(32.0) - np.float32(0.5)
    return q.reshape(-1), O.f16(act)


@pytest.mark.parametrize("fmt,in_dim,out_dim,n", [
    (F.FMT_Q4_K, 4096, 70, 37),       # batched_q4k_small_output_matches_cpu_oracle
    (F.FMT_Q4_K, 14336, 4096, 16),    # batched_q4k_large_k (more tokens than the reference's 3)
    (F.FMT_Q4_K, 5120, 16384, 8),     # batched_q4k_14b gate/up
    (F.FMT_Q4_K, 16384, 5120, 8),     # batched_q4k_14b down
    (F.FMT_Q6_K, 3072, 70, 16),       # batched_q6k_matches_cpu_oracle
    (F.FMT_Q6_K, 3072, 3072, 8),      # batched_q6k_matrix2
    (F.FMT_Q6_K, 5120, 1024, 8),      # batched_q6k_14b V
    (F.FMT_Q6_K, 16384, 5120, 8),     # batched_q6k_14b down
])
def test_gemm_reference_prefill_vectors(hip, fmt, in_dim, out_dim, n):
    make = _reference_q4k_case if fmt == F.FMT_Q4_K else _reference_q6k_case
    w, a16 = make(in_dim, out_dim, n)
    wb, ab = hip.load_weight(fmt, w, in_dim, out_dim), hip.from_host(a16)
    ob = hip.alloc_buffer(n * out_dim * 2)
    hip.matmul_batched(ob, ab, wb, in_dim, out_dim, n)
    got = O.f32(hip.download(ob, np.uint16, n * out_dim)).reshape(n, out_dim).astype(np.float64)
    want = O.f32(O.matmul_batched(fmt, a16, w, in_dim, out_dim, n)).reshape(n, out_dim)
    assert np.isfinite(got).all()
    _reference_bar(got, want.astype(np.float64), f"{fmt} {in_dim}->{out_dim} n={n}")
    for b in (wb, ab, ob):
        hip.free_buffer(b)
