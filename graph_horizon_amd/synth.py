"""Seeded synthetic GGUF tensors for parity tests and benchmarks (no checkpoints offline).

Distributions (the benchmark configurations of the reference's hot path):
  Q4_K block (144 B): d, dmin = f16(|N(0, d_std)|); scales[12] uniform bytes (every 6-bit
      (sc, mn) uniform in 0..63); qs[128] uniform bytes (nibbles uniform in 0..15).
  Q6_K block (210 B): ql[128], qh[64] uniform bytes (quants uniform in -32..31);
      scales[16] = int8(clip(round(N(0, 16)), -128, 127)); d = f16(|N(0, d_std)|).
  Activations: f32 N(0, 1), rounded to FP16 at the boundary where the contract is FP16.
Generator: numpy.random.default_rng(seed) (PCG64); uniform bytes are its raw 64-bit outputs.

For whole-model runs `d_std = model_d_std(in_dim)` keeps every FP16 intermediate finite:
a weight row then has std ≈ 1/sqrt(in_dim), so unit-RMS inputs give unit-scale outputs.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _ffi as F

Q4K_BLOCK, Q6K_BLOCK = 144, 210


def to_f16(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def f16_bits(x) -> np.ndarray:
    return to_f16(x).view(np.uint16)


def uniform_bytes(rng: np.random.Generator, n: int) -> np.ndarray:
    """n uniform bytes: the generator's raw 64-bit words, little-endian."""
    return rng.bit_generator.random_raw((n + 7) // 8).view(np.uint8)[:n]


def q4k_blocks(rng: np.random.Generator, rows: int, in_dim: int, d_std: float = 0.02) -> np.ndarray:
    assert in_dim % 256 == 0
    nblk = rows * (in_dim // 256)
    blk = uniform_bytes(rng, nblk * Q4K_BLOCK).reshape(nblk, Q4K_BLOCK)
    dd = np.abs(rng.standard_normal((nblk, 2), dtype=np.float32) * np.float32(d_std))
    blk[:, 0:4] = dd.astype(np.float16).view(np.uint8).reshape(nblk, 4)
    return blk.reshape(-1)


def q6k_blocks(rng: np.random.Generator, rows: int, in_dim: int, d_std: float = 0.02,
               sc_std: float = 16.0) -> np.ndarray:
    assert in_dim % 256 == 0
    nblk = rows * (in_dim // 256)
    blk = uniform_bytes(rng, nblk * Q6K_BLOCK).reshape(nblk, Q6K_BLOCK)
    sc = np.clip(np.rint(rng.standard_normal((nblk, 16), dtype=np.float32) * sc_std), -128, 127)
    blk[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    d = np.abs(rng.standard_normal(nblk, dtype=np.float32) * np.float32(d_std))
    blk[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(nblk, 2)
    return blk.reshape(-1)


def quant_blocks(rng, fmt: int, rows: int, in_dim: int, d_std: float) -> np.ndarray:
    if fmt == F.FMT_Q4_K:
        return q4k_blocks(rng, rows, in_dim, d_std)
    if fmt == F.FMT_Q6_K:
        return q6k_blocks(rng, rows, in_dim, d_std)
    raise ValueError(fmt)


def model_d_std(in_dim: int) -> float:
    # std(w) ≈ 320·E|d| for both formats with the distributions above; E|N(0,s)| = 0.8 s.
    return 1.0 / (256.0 * float(np.sqrt(in_dim)))


@dataclass
class Shape:
    """A Ministral-shaped decoder (family/mistral/version.rs:40-44 rows, or smaller)."""
    name: str
    block_count: int
    embedding_length: int
    feed_forward_length: int
    head_count: int = 32
    kv_head_count: int = 8
    head_dim: int = 128
    vocab_size: int = 131072
    rope_theta: float = 1e6


SHAPES = {
    # 8B-shaped block with FFN 12288; 14B-shaped E2E decoder
    "8b": Shape("8b", 34, 4096, 12288),
    "14b": Shape("14b", 40, 5120, 16384),
    # small shapes for parity runs against the CPU oracle
    "tiny": Shape("tiny", 2, 512, 1024, head_count=8, kv_head_count=2, vocab_size=2048),
    "small": Shape("small", 2, 1024, 2048, head_count=8, kv_head_count=2, vocab_size=8192),
}

# Q4_K_M tensor formats: attn_v / ffn_down / output Q6_K, the rest Q4_K.
LAYER_FORMATS = {
    F.T_ATTN_Q: F.FMT_Q4_K, F.T_ATTN_K: F.FMT_Q4_K, F.T_ATTN_V: F.FMT_Q6_K,
    F.T_ATTN_OUTPUT: F.FMT_Q4_K, F.T_FFN_GATE: F.FMT_Q4_K, F.T_FFN_UP: F.FMT_Q4_K,
    F.T_FFN_DOWN: F.FMT_Q6_K,
}


def yarn_params(shape: Shape):
    """Ministral 3 style YaRN parameters (mistral3.rope.scaling.* metadata)."""
    return dict(rope_dim=shape.head_dim, original_context=16384, freq_base=shape.rope_theta,
                factor=16.0, beta_fast=32.0, beta_slow=1.0, log_multiplier=1.0,
                q_temperature_scale=0.1)


def model_config(shape: Shape, kv_context: int, prefill_rows: int = 0,
                 flags: int = 0) -> F.GhModelConfig:
    y = yarn_params(shape)
    return F.GhModelConfig(
        block_count=shape.block_count, context_length=max(kv_context, 32768),
        embedding_length=shape.embedding_length, feed_forward_length=shape.feed_forward_length,
        head_count=shape.head_count, kv_head_count=shape.kv_head_count,
        key_length=shape.head_dim, value_length=shape.head_dim, vocab_size=shape.vocab_size,
        rms_epsilon=1e-5, yarn=F.GhYarn(**y), kv_context=kv_context, prefill_rows=prefill_rows,
        flags=flags)


def tensor_dims(shape: Shape, tensor: int):
    d, ffn = shape.embedding_length, shape.feed_forward_length
    qw, kw = shape.head_count * shape.head_dim, shape.kv_head_count * shape.head_dim
    return {
        F.T_ATTN_Q: (d, qw), F.T_ATTN_K: (d, kw), F.T_ATTN_V: (d, kw),
        F.T_ATTN_OUTPUT: (qw, d), F.T_FFN_GATE: (d, ffn), F.T_FFN_UP: (d, ffn),
        F.T_FFN_DOWN: (ffn, d),
    }[tensor]


def model_tensors(shape: Shape, seed: int):
    """Yields (layer, tensor_id, fmt, data) for a random-init Q4_K_M model; norms are f32."""
    rng = np.random.default_rng(seed)
    d = shape.embedding_length
    yield (F.NO_LAYER, F.T_TOKEN_EMBD, F.FMT_Q4_K,
           q4k_blocks(rng, shape.vocab_size, d, model_d_std(d) * 16.0))
    for li in range(shape.block_count):
        for t in (F.T_ATTN_NORM, F.T_FFN_NORM):
            yield li, t, F.FMT_F32, (1.0 + 0.05 * rng.standard_normal(d)).astype(np.float32)
        for t, fmt in LAYER_FORMATS.items():
            ind, outd = tensor_dims(shape, t)
            yield li, t, fmt, quant_blocks(rng, fmt, outd, ind, model_d_std(ind))
    yield (F.NO_LAYER, F.T_OUTPUT_NORM, F.FMT_F32,
           (1.0 + 0.05 * rng.standard_normal(d)).astype(np.float32))
    yield (F.NO_LAYER, F.T_OUTPUT, F.FMT_Q6_K,
           q6k_blocks(rng, shape.vocab_size, d, model_d_std(d)))
