"""Parity of the gfx950 backend (through the C ABI) against the CPU oracle on seeded inputs.

Bars (stated per test):
  * bit-exact: dequantized weights, KV writes, embedding rows, residual add, RoPE, argmax/top-k;
  * matvec/GEMM and attention: |got - want| <= 1e-3·|want| + 2e-6·Σ|terms| (FP32 accumulation;
    the second term only matters for outputs whose terms cancel);
  * FP16 glue with a transcendental or a reduction (silu_mul, rmsnorm): within 1 FP16 ulp.
"""
import math

import numpy as np
import pytest

import oracle as O
from graph_horizon_amd import GhError, Yarn, synth
from graph_horizon_amd import _ffi as F
from agreement import assert_agreement

pytestmark = pytest.mark.gpu

REL = 1e-3
FLOOR = 2e-6


def f16(x):
    return O.f16(np.asarray(x, dtype=np.float32))


def up(hip, arr):
    return hip.from_host(np.ascontiguousarray(arr))


def assert_close_terms(got, want, scale, rel=REL, what=""):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    tol = rel * np.abs(want) + FLOOR * np.asarray(scale, np.float64)
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tolerance, worst " \
        f"{np.max(np.abs(got - want) / np.maximum(tol, 1e-30)):.3f}x tol"


def ulp_diff(a16, b16):
    a = a16.astype(np.int32)
    b = b16.astype(np.int32)
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


def term_scale(fmt, w, x16, rows, in_dim):
    deq = O.dequant(fmt, w, rows, in_dim).astype(np.float64)
    return np.abs(deq * O.f32(x16).astype(np.float64)[None]).sum(axis=1)


# ---------------------------------------------------------------- dequant
@pytest.mark.parametrize("fmt,rows,in_dim", [(F.FMT_Q4_K, 48, 4096), (F.FMT_Q6_K, 48, 4096),
                                              (F.FMT_Q6_K, 16, 5120), (F.FMT_Q4_K, 8, 12288),
                                              (F.FMT_Q6_K, 8, 12288)])
def test_dequant_bit_exact(hip, fmt, rows, in_dim):
    rng = np.random.default_rng(100 + fmt + in_dim)
    w = synth.quant_blocks(rng, fmt, rows, in_dim, 0.02)
    wb = hip.load_weight(fmt, w, in_dim, rows)
    out = hip.alloc_buffer(rows * in_dim * 4)
    hip.dequant_rows(out, wb, 0, rows)
    got = hip.download(out, np.float32, rows * in_dim).reshape(rows, in_dim)
    want = O.dequant(fmt, w, rows, in_dim)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a window of rows (row0 > 0) decodes the same bytes
    hip.dequant_rows(out, wb, rows // 2, rows - rows // 2)
    part = hip.download(out, np.float32, (rows - rows // 2) * in_dim).reshape(-1, in_dim)
    assert np.array_equal(part.view(np.uint32), want[rows // 2:].view(np.uint32))
    hip.free_buffer(out)
    hip.free_buffer(wb)


def test_reference_golden_blocks_on_device(hip, goldens):
    """The reference's hand-derived Q4_K / Q6_K blocks decode to the expected values on gfx950."""
    g = goldens["q4_k_golden_vector"]
    blk = (np.float16(g["d"]).tobytes() + np.float16(g["dmin"]).tobytes() + bytes(g["scales"])
           + bytes([g["qs_byte"]] * 128))
    wb = hip.load_weight(F.FMT_Q4_K, np.frombuffer(blk, np.uint8), 256, 1)
    out = hip.alloc_buffer(1024)
    hip.dequant_rows(out, wb, 0, 1)
    got = hip.download(out, np.float32, 256)
    assert np.array_equal(got, np.repeat(np.float32(g["per_sub_block"]), 32))
    g6 = goldens["q6_k_golden_vector"]
    raw = bytes([g6["ql_byte"]] * 128 + [g6["qh_byte"]] * 64) + np.int8(g6["scales"]).tobytes()
    raw += np.float16(g6["d"]).tobytes()
    wb6 = hip.load_weight(F.FMT_Q6_K, np.frombuffer(raw, np.uint8), 256, 1)
    hip.dequant_rows(out, wb6, 0, 1)
    got6 = hip.download(out, np.float32, 256)
    for i, want in g6["anchors"]:
        assert got6[i] == want
    for b in (wb, wb6, out):
        hip.free_buffer(b)


# ---------------------------------------------------------------- GEMV
def _gemv(hip, fmt, rows, in_dim, seed, f32_out, d_std=0.02):
    rng = np.random.default_rng(seed)
    w = synth.quant_blocks(rng, fmt, rows, in_dim, d_std)
    x16 = f16(rng.standard_normal(in_dim))
    wb = hip.load_weight(fmt, w, in_dim, rows)
    xb = up(hip, x16)
    yb = hip.alloc_buffer(rows * 4)
    if f32_out:
        hip.logits(yb, xb, wb, in_dim, rows)
        got = hip.download(yb, np.float32, rows)
        want = O.logits(fmt, x16, w, in_dim, rows)
    else:
        hip.matmul(yb, xb, wb, in_dim, rows)
        got = O.f32(hip.download(yb, np.uint16, rows))
        want = O.f32(O.matmul(fmt, x16, w, in_dim, rows))
    scale = term_scale(fmt, w, x16, rows, in_dim)
    for b in (wb, xb, yb):
        hip.free_buffer(b)
    return got, want, scale


def test_q4k_gemv_c1_logits(hip):
    """Q4_K 4096x4096, |N(0,0.02)| d/dmin, x ~ N(0,1), FP32 output."""
    got, want, scale = _gemv(hip, F.FMT_Q4_K, 4096, 4096, 1, True)
    assert_close_terms(got, want, scale, what="Q4_K 4096x4096")


# the decode-step projections of one 8B-shaped block
C2 = [("q", F.FMT_Q4_K, 4096, 4096), ("k", F.FMT_Q4_K, 1024, 4096), ("v", F.FMT_Q6_K, 1024, 4096),
      ("o", F.FMT_Q4_K, 4096, 4096), ("gate", F.FMT_Q4_K, 12288, 4096),
      ("up", F.FMT_Q4_K, 12288, 4096), ("down", F.FMT_Q6_K, 4096, 12288)]


@pytest.mark.parametrize("name,fmt,rows,in_dim", C2, ids=[c[0] for c in C2])
def test_c2_block_projection_matmul_f16(hip, name, fmt, rows, in_dim):
    got, want, scale = _gemv(hip, fmt, rows, in_dim, 7 + rows + in_dim, False)
    assert_close_terms(got, want, scale, what=name)


@pytest.mark.parametrize("fmt,rows,in_dim", [(F.FMT_Q6_K, 8192, 4096), (F.FMT_Q6_K, 2048, 5120),
                                              (F.FMT_Q4_K, 333, 5120), (F.FMT_Q4_K, 7, 256),
                                              (F.FMT_Q6_K, 3, 14336),
                                              # direct kernel, several tasks per wave (2-4,
                                              # unequal): the next task is prefetched
                                              (F.FMT_Q4_K, 20000, 4096), (F.FMT_Q6_K, 9001, 2048),
                                              (F.FMT_Q4_K, 12287, 4096)])  # ragged last task
def test_gemv_logits_shapes(hip, fmt, rows, in_dim):
    got, want, scale = _gemv(hip, fmt, rows, in_dim, 3 + rows, True)
    assert_close_terms(got, want, scale, what=f"{fmt} {rows}x{in_dim}")


@pytest.mark.parametrize("fmt", [F.FMT_Q4_K, F.FMT_Q6_K])
def test_matmul_batched(hip, fmt):
    rng = np.random.default_rng(55)
    in_dim, rows, n = 1024, 300, 5
    w = synth.quant_blocks(rng, fmt, rows, in_dim, 0.02)
    a16 = f16(rng.standard_normal(n * in_dim))
    wb, ab, ob = hip.load_weight(fmt, w, in_dim, rows), up(hip, a16), hip.alloc_buffer(n * rows * 2)
    hip.matmul_batched(ob, ab, wb, in_dim, rows, n)
    got = O.f32(hip.download(ob, np.uint16, n * rows)).reshape(n, rows)
    want = O.f32(O.matmul_batched(fmt, a16, w, in_dim, rows, n)).reshape(n, rows)
    deq = O.dequant(fmt, w, rows, in_dim).astype(np.float64)
    for i in range(n):
        scale = np.abs(deq * O.f32(a16[i * in_dim:(i + 1) * in_dim])[None]).sum(axis=1)
        assert_close_terms(got[i], want[i], scale, what=f"token {i}")
    for b in (wb, ab, ob):
        hip.free_buffer(b)


# ---------------------------------------------------------------- glue
def test_rmsnorm_within_one_ulp(hip):
    rng = np.random.default_rng(5)
    dim, rows = 5120, 4
    x = (rng.standard_normal(rows * dim) * 3).astype(np.float32)
    w = f16(1.0 + 0.05 * rng.standard_normal(dim))
    xb, wb, ob = up(hip, x), up(hip, w), hip.alloc_buffer(rows * dim * 2)
    hip.rmsnorm_x(ob, xb, wb, dim, 1e-5, rows)
    got = hip.download(ob, np.uint16, rows * dim)
    assert ulp_diff(got, O.rmsnorm_x(x, w, dim, 1e-5, rows)).max() <= 1
    for b in (xb, wb, ob):
        hip.free_buffer(b)


YARN = Yarn(rope_dim=128, original_context=16384, freq_base=1e6, factor=16.0, beta_fast=32.0,
            beta_slow=1.0, log_multiplier=1.0, q_temperature_scale=0.1)


@pytest.mark.parametrize("pos", [0, 1, 127, 128, 4095, 16384, 20000])
def test_rope_bit_exact(hip, pos):
    rng = np.random.default_rng(pos)
    heads = 32
    x = f16(rng.standard_normal(heads * 128))
    for role in (F.ROPE_QUERY, F.ROPE_KEY):
        xb = up(hip, x)
        hip.rope_yarn(xb, heads, 128, pos, YARN, role)
        got = hip.download(xb, np.uint16, heads * 128)
        want = O.rope_yarn(x, heads, 128, pos, O.Yarn(128, 16384, 1e6, 16.0, 32.0, 1.0, 1.0, 0.1), role)
        assert np.array_equal(got, want), (pos, role)
        hip.free_buffer(xb)


def test_rope_batched_matches_per_row(hip):
    rng = np.random.default_rng(9)
    rows, qh, kvh, base = 7, 32, 8, 16380
    q, k = f16(rng.standard_normal(rows * qh * 128)), f16(rng.standard_normal(rows * kvh * 128))
    qb, kb = up(hip, q), up(hip, k)
    hip.rope_yarn_batched(qb, kb, qh, kvh, 128, base, rows, YARN)
    gq, gk = hip.download(qb, np.uint16, q.size), hip.download(kb, np.uint16, k.size)
    oy = O.Yarn(128, 16384, 1e6, 16.0, 32.0, 1.0, 1.0, 0.1)
    for r in range(rows):
        assert np.array_equal(gq[r * qh * 128:(r + 1) * qh * 128],
                              O.rope_yarn(q[r * qh * 128:(r + 1) * qh * 128], qh, 128, base + r, oy, 0))
        assert np.array_equal(gk[r * kvh * 128:(r + 1) * kvh * 128],
                              O.rope_yarn(k[r * kvh * 128:(r + 1) * kvh * 128], kvh, 128, base + r, oy, 1))
    hip.free_buffer(qb)
    hip.free_buffer(kb)


def test_silu_mul_within_one_ulp(hip):
    rng = np.random.default_rng(6)
    n = 16384 * 3 + 17
    g, u = f16(rng.standard_normal(n) * 4), f16(rng.standard_normal(n) * 4)
    gb, ub, ob = up(hip, g), up(hip, u), hip.alloc_buffer(n * 2)
    hip.silu_mul(ob, gb, ub, n)
    d = ulp_diff(hip.download(ob, np.uint16, n), O.silu_mul(g, u))
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    for b in (gb, ub, ob):
        hip.free_buffer(b)


def test_residual_add_bit_exact(hip):
    rng = np.random.default_rng(7)
    n = 5120
    x = rng.standard_normal(n).astype(np.float32)
    y = f16(rng.standard_normal(n))
    xb, yb = up(hip, x), up(hip, y)
    hip.residual_add(xb, yb, n - 3)  # only the first n-3 elements change
    got = hip.download(xb, np.float32, n)
    want = x.copy()
    O.lib().gho_residual_add(want.ctypes.data, y.ctypes.data, n - 3)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    hip.free_buffer(xb)
    hip.free_buffer(yb)


@pytest.mark.parametrize("fmt", [F.FMT_Q4_K, F.FMT_Q6_K])
def test_embed_bit_exact(hip, fmt):
    rng = np.random.default_rng(8)
    vocab, d = 1000, 5120
    w = synth.quant_blocks(rng, fmt, vocab, d, 0.02)
    wb, xb = hip.load_weight(fmt, w, d, vocab), hip.alloc_buffer(d * 4)
    for tok in (0, 1, 517, vocab - 1):
        hip.embed(xb, wb, tok, d)
        want = np.empty(d, np.float32)
        assert O.lib().gho_embed(want.ctypes.data, fmt, w.ctypes.data, tok, d) == 0
        assert np.array_equal(hip.download(xb, np.float32, d).view(np.uint32), want.view(np.uint32))
    with pytest.raises(GhError):
        hip.embed(xb, wb, vocab, d)
    hip.free_buffer(wb)
    hip.free_buffer(xb)


def _kv(hip, layers, ctx, kvh, kc=None, vc=None):
    n = layers * ctx * kvh * 128
    kb = up(hip, kc) if kc is not None else hip.alloc_buffer(n * 2)
    vb = up(hip, vc) if vc is not None else hip.alloc_buffer(n * 2)
    return F.GhKv(kb, vb, F.KV_F16, layers, ctx, kvh, 128, 128)


def test_kv_write_bytes(hip):
    rng = np.random.default_rng(10)
    layers, ctx, kvh = 3, 50, 8
    kc = f16(rng.standard_normal(layers * ctx * kvh * 128))
    vc = f16(rng.standard_normal(layers * ctx * kvh * 128))
    kv = _kv(hip, layers, ctx, kvh, kc, vc)
    rows, layer, pos = 3, 2, 40
    k, v = f16(rng.standard_normal(rows * kvh * 128)), f16(rng.standard_normal(rows * kvh * 128))
    kb, vb = up(hip, k), up(hip, v)
    off = O.lib().gho_kv_payload_offset(layer, pos, kvh, 128, ctx)
    hip.kv_write(kv, kb, vb, off, off, rows * kvh)
    gk = hip.download(kv.k, np.uint16, kc.size)
    gv = hip.download(kv.v, np.uint16, vc.size)
    wk, wv = kc.copy(), vc.copy()
    wk[off // 2: off // 2 + k.size] = k
    wv[off // 2: off // 2 + v.size] = v
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
    with pytest.raises(GhError):  # past the end of the cache
        hip.kv_write(kv, kb, vb, kc.nbytes - 2, 0, rows * kvh)
    with pytest.raises(GhError):  # an offset whose sum with the length wraps around 2^64
        hip.kv_write(kv, kb, vb, 2**64 - 2, 0, rows * kvh)
    with pytest.raises(GhError):
        hip.kv_write(kv, kb, vb, 0, 2**64 - 1024, rows * kvh)
    for b in (kb, vb, kv.k, kv.v):
        hip.free_buffer(b)


def test_view_alignment(hip):
    """min_buffer_offset_alignment (contract.rs:56) is 16, and views at other offsets are
    rejected (the kernels read rows with 16-byte loads)."""
    assert hip.min_buffer_offset_alignment() == 16
    b = hip.alloc_buffer(4096)
    assert hip.view(b, 32, 64).addr == b.addr + 32
    for off in (2, 4, 8, 24):
        with pytest.raises(GhError):
            hip.view(b, off, 64)
    with pytest.raises(GhError):
        hip.view(b, 4096 - 16, 32)  # beyond the buffer
    hip.free_buffer(b)


def test_create_leaves_no_hip_error():
    """gh_create resolves each kernel by trying the modules in turn; the misses must not stay
    behind as the thread's last HIP error, which another HIP user in the same process (torch
    checks hipGetLastError after its own calls) would report as its own failure."""
    import ctypes

    from graph_horizon_amd import HipBackend

    rt = ctypes.CDLL("libamdhip64.so")
    rt.hipGetLastError()  # whatever came before
    b = HipBackend(0)
    try:
        assert rt.hipGetLastError() == 0
    finally:
        b.close()


# ---------------------------------------------------------------- attention
def _attn_case(hip, ctx, layers, seed, qh=32, kvh=8):
    rng = np.random.default_rng(seed)
    kc = f16(rng.standard_normal(layers * ctx * kvh * 128))
    vc = f16(rng.standard_normal(layers * ctx * kvh * 128))
    return kc, vc, _kv(hip, layers, ctx, kvh, kc, vc), rng


@pytest.mark.parametrize("ctx,pos,layer", [(4096, 4095, 1), (32768, 32767, 0), (4096, 0, 0),
                                           (4096, 63, 1), (4096, 64, 1), (4096, 1000, 0)])
def test_attention_decode(hip, ctx, pos, layer):
    """32 q / 8 kv heads, head_dim 128, f16 KV, ctx 4096 and 32768."""
    kc, vc, kv, rng = _attn_case(hip, ctx, 2, ctx + pos)
    q = f16(rng.standard_normal(32 * 128))
    qb, ob = up(hip, q), hip.alloc_buffer(32 * 128 * 2)
    hip.attention_decode(ob, qb, kv, 32, pos, layer)
    got = O.f32(hip.download(ob, np.uint16, 32 * 128))
    want = O.f32(O.attention_decode(q, kc, vc, 128, 8, 32, pos, layer, ctx))
    # outputs are convex combinations of V rows (|v| ~ 1): absolute floor 1e-5
    assert_close_terms(got, want, np.full(got.shape, 5.0), what=f"ctx {ctx} pos {pos}")
    for b in (qb, ob, kv.k, kv.v):
        hip.free_buffer(b)


@pytest.mark.parametrize("base,n", [(0, 1), (0, 37), (100, 64), (300, 200)])
def test_attention_prefill(hip, base, n):
    ctx = 512
    kc, vc, kv, rng = _attn_case(hip, ctx, 2, base + n)
    q = f16(rng.standard_normal(n * 32 * 128))
    qb, ob = up(hip, q), hip.alloc_buffer(n * 32 * 128 * 2)
    hip.attention_prefill(ob, qb, kv, 32, base, n, 1)
    got = O.f32(hip.download(ob, np.uint16, n * 32 * 128))
    want = O.f32(O.attention_prefill(q, kc, vc, 128, 8, 32, base, n, 1, ctx))
    assert_close_terms(got, want, np.full(got.shape, 5.0), what=f"prefill {base}+{n}")
    with pytest.raises(GhError):  # beyond the context
        hip.attention_prefill(ob, qb, kv, 32, ctx - n + 1, n, 1)
    for b in (qb, ob, kv.k, kv.v):
        hip.free_buffer(b)


# ---------------------------------------------------------------- read-back
def test_argmax_and_topk(hip):
    rng = np.random.default_rng(12)
    vocab = 131072
    cases = [rng.standard_normal(vocab).astype(np.float32)]
    tie = rng.standard_normal(vocab).astype(np.float32)
    tie[[77, 5000, 130000]] = 9.0
    cases.append(tie)
    nan = rng.standard_normal(vocab).astype(np.float32)
    nan[::7] = np.nan
    cases.append(nan)
    cases.append(np.full(vocab, -np.inf, np.float32))
    for l in cases:
        lb = up(hip, l)
        assert hip.read_argmax(lb, vocab) == O.argmax(l)
        assert _topk_bits(hip.read_topk(lb, vocab, 40)) == _topk_bits(O.topk(l, 40))
        hip.free_buffer(lb)


def _topk_bits(pairs):
    return [(i, int(np.asarray(v, dtype=np.float32).view(np.uint32))) for i, v in pairs]


@pytest.mark.parametrize("vocab,ks", [
    (5, [1, 3, 99]),                 # the reference's readback test vector sizes; k > vocab
    (3000, [1, 64, 128, 129]),       # two chunks of 2048; k = 129 takes the host path
    (131072, [1, 40, 100, 128]),     # the vocabulary of the 8B/14B shapes: 64 stripes
    (700001, [128, 2]),              # stripes of several 2048-logit chunks (114 stripes)
])
def test_topk_device_bit_exact(hip, vocab, ks):
    """Device top-k vs the oracle (cpu/readback.rs:59-69 order): indices and raw logit bits
    identical, with exact ties, ±0, ±inf, denormals and NaNs of both signs and two payloads."""
    rng = np.random.default_rng(vocab)
    if vocab == 5:
        bits = np.array([0.1, 2.5, 2.5, -1.0, 2.4], dtype=np.float32).view(np.uint32)
    else:
        bits = rng.standard_normal(vocab).astype(np.float32).view(np.uint32).copy()
        bits[rng.integers(0, vocab, vocab // 5)] = bits[rng.integers(0, vocab, vocab // 5)]
        specials = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001, 0x7F800000,
                             0xFF800000, 0, 0x80000000, 1, 0x80000001], dtype=np.uint32)
        bits[rng.integers(0, vocab, 3 * specials.size)] = np.repeat(specials, 3)
        fin = bits.view(np.float32)[np.isfinite(bits.view(np.float32))]
        bits[rng.integers(0, vocab, 50)] = np.float32(fin.max()).view(np.uint32)  # ties at the top
    l = bits.view(np.float32)
    lb = up(hip, l)
    for k in ks:
        got = _topk_bits(hip.read_topk(lb, vocab, k))
        want = _topk_bits(O.topk(l, k))
        assert len(got) == min(k, vocab)
        assert got == want, f"vocab {vocab} k {k}"
    hip.free_buffer(lb)


# ---------------------------------------------------------------- graph driver (whole model)
def _models(hip, shape_name, seed, kv_context, prefill_rows=64):
    from graph_horizon_amd import HipModel
    from test_oracle import oracle_model

    shape = synth.SHAPES[shape_name]
    gm = HipModel(hip, synth.model_config(shape, kv_context, prefill_rows))
    for layer, tid, fmt, data in synth.model_tensors(shape, seed):
        gm.load_tensor(layer, tid, fmt, data)
    om, _ = oracle_model(shape, seed, kv_context)
    return gm, om


def test_model_decode_tokens_match_oracle(hip):
    gm, om = _models(hip, "tiny", 31, 128)
    toks = [1, 500, 2047, 33, 900, 12, 7, 1999]
    dev, ora = [], []
    for p, t in enumerate(toks):
        gm.token(t, p)
        om.token(t, p)
        got, want = gm.read_logits(), om.logits()
        assert np.allclose(got, want, rtol=2e-2, atol=2e-2), p
        dev.append(gm.read_argmax())
        ora.append(want)
    assert_agreement(dev, ora, "tiny decode", min_frac=1.0)
    gm.close()
    om.close()


def test_model_prefill_matches_oracle(hip):
    gm, om = _models(hip, "tiny", 32, 256, prefill_rows=48)
    toks = list(np.random.default_rng(3).integers(0, 2048, 100))
    gm.prefill(toks, 0)
    om.prefill(toks, 0, 48)
    got, want = gm.read_logits(), om.logits()
    assert np.allclose(got, want, rtol=2e-2, atol=2e-2)
    gm.close()
    om.close()


@pytest.mark.parametrize("n", [8, 32, 128])
def test_model_prefill_short_chunk_matches_oracle(hip, n):
    """A prompt of n rows in one chunk (8: the smallest GEMM batch; 32; 128: one full 128-token
    tile) on the small shape (the down GEMM splits K, its residual tail summing the splits),
    against the oracle's prefill of the same prompt: the logits and every K/V cache row the
    chunk wrote."""
    shape, ctx = synth.SHAPES["small"], 160
    gm, om = _models(hip, "small", 33, ctx, prefill_rows=128)
    toks = list(np.random.default_rng(50 + n).integers(0, shape.vocab_size, n))
    gm.prefill(toks, 0)
    om.prefill(toks, 0, 128)
    got, want = gm.read_logits(), om.logits()
    assert np.abs(want).max() > 0.1
    assert np.allclose(got, want, rtol=2e-2, atol=2e-2)
    kv = gm.kv()
    kvw = shape.kv_head_count * shape.head_dim
    m = shape.block_count * ctx * kvw
    for role, buf in ((0, kv.k), (1, kv.v)):
        dev = O.f32(hip.download(buf, np.uint16, m)).reshape(shape.block_count, ctx, kvw)[:, :n]
        ora = O.f32(om.kv(role)).reshape(shape.block_count, ctx, kvw)[:, :n]
        assert np.max(np.abs(dev - ora)) <= 2e-2 * max(float(np.abs(ora).max()), 1.0), role
    gm.close()
    om.close()


def test_model_prefill_policy_chunks(hip):
    """prefill_rows = 0 takes gh_prefill_rows (2048-row chunks): a 2500-token prompt in two
    chunks (2048 + 452 rows, the second attending across the first) gives the logits and KV
    of 512-row chunking within the model tolerance."""
    from graph_horizon_amd import HipModel
    shape = synth.SHAPES["tiny"]
    ctx = 2600
    assert hip.lib.gh_prefill_rows(hip.h, shape.block_count, ctx) == 2048
    toks = list(np.random.default_rng(4).integers(0, shape.vocab_size, 2500))
    logits = []
    for rows in (0, 512):
        gm = HipModel(hip, synth.model_config(shape, ctx, rows))
        for layer, tid, fmt, data in synth.model_tensors(shape, 35):
            gm.load_tensor(layer, tid, fmt, data)
        gm.prefill(toks, 0)
        logits.append(gm.read_logits())
        gm.close()
    assert np.allclose(logits[0], logits[1], rtol=2e-2, atol=2e-2)


def test_greedy_decode_graph_replay_teacher_forced(hip):
    """64-step greedy decode through the replayed HIP graph; each step's argmax is checked
    against the oracle fed the same (teacher-forced) token history (parity.rs protocol)."""
    gm, om = _models(hip, "tiny", 33, 256)
    prompt = [3, 99, 1500, 42]
    gm.prefill(prompt, 0)
    om.prefill(prompt, 0, 64)
    first = int(np.argmax(om.logits()))
    steps = 64
    toks = gm.decode_greedy(first, len(prompt), steps)
    tok, ora = first, []
    for i in range(steps):
        om.token(tok, len(prompt) + i)
        ora.append(om.logits())
        tok = int(toks[i])
    assert_agreement(toks, ora, "tiny 64-step greedy")
    # replaying the graph from the same state reproduces the host-driven path
    gm.prefill(prompt, 0)
    again = gm.decode_greedy(first, len(prompt), 8)
    assert np.array_equal(again, toks[:8])
    gm.close()
    om.close()


def test_model_rejects_bad_inputs(hip):
    gm, om = _models(hip, "tiny", 34, 16)
    om.close()
    with pytest.raises(GhError):
        gm.token(2048, 0)  # beyond vocabulary
    with pytest.raises(GhError):
        gm.token(1, 16)  # beyond the KV context
    with pytest.raises(GhError):
        gm.prefill([], 0)
    gm.close()


@pytest.mark.parametrize("ctx,prompt,steps", [(64, 3, 20), (300, 60, 80)])
def test_greedy_decode_stream_launch_equals_graph(hip, ctx, prompt, steps):
    """GH_MODEL_NO_GRAPH launches the same step kernels directly: identical tokens. The second
    case decodes positions 60..139 of a 300-position cache, across the decode step graphs'
    position ranges (ends 64 and 128: 1, 2 and then 4 attention splits), both ways."""
    from graph_horizon_amd import HipModel

    shape = synth.SHAPES["tiny"]
    outs = []
    for flags in (0, F.MODEL_NO_GRAPH):
        gm = HipModel(hip, synth.model_config(shape, ctx, 64, flags=flags))
        for layer, tid, fmt, data in synth.model_tensors(shape, 35):
            gm.load_tensor(layer, tid, fmt, data)
        gm.prefill(list(range(4, 4 + prompt)), 0)
        outs.append(gm.decode_greedy(9, prompt, steps))
        gm.close()
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("shape_name", ["tiny", "small"])
def test_fused_decode_is_bit_identical_to_op_by_op(hip, shape_name):
    """The fused driver (RoPE + KV write in the QKV epilogue, residual in O/down, SwiGLU in
    gate/up) leaves the same bits as recording every trait op separately."""
    from graph_horizon_amd import HipModel
    from graph_over_abi import AbiGraph

    shape = synth.SHAPES[shape_name]
    ref = AbiGraph(hip, shape, 41, 64)
    gm = HipModel(hip, synth.model_config(shape, 64, 16))
    for layer, tid, fmt, data in synth.model_tensors(shape, 41):
        gm.load_tensor(layer, tid, fmt, data)
    for pos, tok in enumerate([11, 700, 3, 1999, 56]):
        want = ref.token(tok, pos)
        gm.token(tok, pos)
        got = gm.read_logits()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
        assert np.array_equal(gm.read_x().view(np.uint32), ref.read_x().view(np.uint32)), pos
    kv = gm.kv()
    n = shape.block_count * 64 * shape.kv_head_count * shape.head_dim
    for role in ("k", "v"):  # positions 0..4 of every layer were written
        a = hip.download(getattr(kv, role), np.uint16, n).reshape(shape.block_count, 64, -1)
        b = hip.download(getattr(ref.kv, role), np.uint16, n).reshape(shape.block_count, 64, -1)
        assert np.array_equal(a[:, :5], b[:, :5]), role
    gm.close()


@pytest.mark.parametrize("n", [8, 37, 128, 300])
@pytest.mark.parametrize("shape_name", ["tiny", "small"])
def test_prefill_driver_is_bit_identical_to_op_by_op(hip, shape_name, n):
    """The driver's prefill (one batch: GEMV for n < 8 rows, the MFMA GEMMs above, the
    warp-specialized ones from 256 rows, with the glue folded into GEMM epilogues and split
    reduces and Q/K/V in one launch) leaves the same logits and KV bits as recording every
    trait op separately (prefill::record_batch over the C ABI). The tiny shape's GEMMs run one
    K split each; the small shape's run one (two for down) at 8-128 rows and two (four for
    down) at 300, alike in the fused and the separate launches, so both sum in the same order.
    At 8-128 rows the driver's gate and up run as one paired launch (gh_gemm3_swiglu_r96_t128:
    48 gate + 48 up rows per tile, silu_mul in its epilogue; 22 and 43 tiles here, the last one
    partial) against two unsplit GEMMs and silu_mul op by op; at 300 rows they share one split
    reduce that applies silu_mul (gh_gemm_reduce_swiglu). Where the split counts differ
    (the 8B shape's Q/K/V launch against the three projections alone) the results differ only
    by FP32 re-association, checked against the oracle in test_gpu_model_shapes."""
    from graph_horizon_amd import HipModel
    from graph_over_abi import AbiGraph

    shape = synth.SHAPES[shape_name]
    ctx = 320
    ref = AbiGraph(hip, shape, 43, ctx)
    gm = HipModel(hip, synth.model_config(shape, ctx, 512))
    for layer, tid, fmt, data in synth.model_tensors(shape, 43):
        gm.load_tensor(layer, tid, fmt, data)
    toks = [int(t) for t in np.random.default_rng(n).integers(0, shape.vocab_size, n)]
    want = ref.prefill(toks, 0)
    gm.prefill(toks, 0)
    got = gm.read_logits()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    last_x = ref.prefill_x[(n - 1) * shape.embedding_length:]
    assert np.array_equal(gm.read_x().view(np.uint32), last_x.view(np.uint32))
    kv = gm.kv()
    m = shape.block_count * ctx * shape.kv_head_count * shape.head_dim
    for role in ("k", "v"):
        a = hip.download(getattr(kv, role), np.uint16, m).reshape(shape.block_count, ctx, -1)
        b = hip.download(getattr(ref.kv, role), np.uint16, m).reshape(shape.block_count, ctx, -1)
        assert np.array_equal(a[:, :n], b[:, :n]), role
    gm.close()


# ---------------------------------------------------------------- generation loop (§ sampling)
def _manual_generate(gm, prompt, p, max_tokens, context):
    """generation::drive restated over the driver's primitives with the oracle's sampling:
    the same decode kernels (one replayed graph step per token) and the same device reductions."""
    from oracle import sampling as S
    path, k = S.plan(p)
    st = S.rng_seed(p["seed"])
    recent = list(prompt)
    gm.prefill(prompt, 0)
    out = []
    while len(out) < max_tokens and len(prompt) + len(out) < context:
        if path == S.GREEDY:
            tok = gm.read_argmax()
        elif path == S.TOPK:
            inv = np.float32(1.0) / np.float32(p["temperature"])
            cand = [(i, np.float32(v * inv)) for i, v in gm.read_topk(k)]
            tok, st = S.sample_from_candidates(cand, p, st)
        else:
            tok, st = S.sample(gm.read_logits(), p, recent, st)
        out.append(tok)
        recent.append(tok)
        if len(out) < max_tokens and len(prompt) + len(out) < context:
            gm.decode_greedy(tok, len(prompt) + len(out) - 1, 1)
    return out


@pytest.mark.parametrize("p", [
    dict(temperature=0.0, top_p=1.0, top_k=0, min_p=0.0, repeat_penalty=1.0, seed=0),
    dict(temperature=0.9, top_p=0.95, top_k=40, min_p=0.02, repeat_penalty=1.0, seed=11),
    dict(temperature=1.2, top_p=1.0, top_k=128, min_p=0.0, repeat_penalty=1.0, seed=12),
    dict(temperature=0.8, top_p=0.9, top_k=0, min_p=0.05, repeat_penalty=1.15, seed=13),
], ids=["greedy", "device-topk40", "device-topk128", "fallback-penalty"])
def test_generate_matches_driver_loop(hip, p):
    """gh_model_generate (C++ loop, C++ sampling) == the same loop driven from Python with the
    oracle's sampling, token for token (the device reductions and logits are shared, so any
    difference is in the loop or the sampling restatement)."""
    gm, om = _models(hip, "tiny", 34, 96)
    om.close()
    prompt = [5, 77, 1024, 3, 650]
    got = gm.generate(prompt, F.GhSampling(**p), 24)
    want = _manual_generate(gm, prompt, p, 24, 96)
    assert [int(t) for t in got] == want
    # greedy generate == the graph-replayed greedy decode from the prefill's argmax
    if p["temperature"] == 0.0:
        gm.prefill(prompt, 0)
        first = gm.read_argmax()
        assert int(got[0]) == first
        assert [int(t) for t in gm.decode_greedy(first, len(prompt), 23)] == want[1:]
    # stops at the context and at eos
    short = gm.generate(prompt, F.GhSampling(**p), 500)
    assert len(short) == 96 - len(prompt)
    eos = int(got[3])
    stop = gm.generate(prompt, F.GhSampling(**p), 24, eos=eos)
    assert [int(t) for t in stop] == want[:want.index(eos)]
    gm.close()
