"""ctypes binding of the CPU oracle (oracle/libgh_oracle.so) — TEST INFRASTRUCTURE.

The oracle restates graph_horizon_engine's CPU backend (crates/graph_horizon_engine/src/
backend/cpu/**, backend/f16.rs, backend/rope.rs, kv_cache/layout.rs, family/mistral/graph/**)
in C++ with the reference's AVX2 operation order. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this module; the product never does.

Every function here was checked against what pins it (tests/test_oracle.py):
  f16 conversion      known answers of backend/f16.rs:86-112, exhaustive F16C comparison
  scale_min           exhaustive over all byte values vs the ggml bit specification
  Q4_K/Q6_K dequant   reference golden vectors (cpu/dequant.rs:462-495, 544-579) + closed form
  GEMV                fp64 brute force over dequant_row, scalar vs AVX2 vs batched invariants
  attention           hand-computed softmax (attention/mod.rs:816-846), serial reference,
                      prefill(n=1) == decode, fp64 softmax brute force
  RoPE / YaRN         rope.rs:166-214 unit magnitude, buckets, ramp; adjacent pairs
  silu_mul / rmsnorm  sequential FP16 rounding rule; RMSNorm formula in fp64
  argmax / top-k      readback.rs:77-100 tie-break cases
  KV layout           layout.rs:105-205 hand-computed byte regions
  graph               op trace == the reference's shape-recorder trace (graph/shape.rs:389-446),
                      dedicated and tied; closed-form one-layer models (zeroed FFN or zeroed
                      O projection) computed in fp64 from the pinned dequant; batched prefill
                      == sequential decode within abs 0.05 (generation/tests.rs:716-773)
  residual_add        closed form: numpy x + f32(y) bit for bit (±0, inf, NaN, prefix only)
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgh_oracle.so")

FMT_F32, FMT_F16, FMT_Q4_K, FMT_Q6_K = 0, 1, 12, 14
PLANT_NONE, PLANT_POST_SCALE_ON_K, PLANT_NO_POST_SCALE_ON_Q = 0, 1, 2
LAYER_TENSORS = 9


class Yarn(C.Structure):
    _fields_ = [("rope_dim", C.c_uint32), ("original_context", C.c_uint32),
                ("freq_base", C.c_float), ("factor", C.c_float), ("beta_fast", C.c_float),
                ("beta_slow", C.c_float), ("log_multiplier", C.c_float),
                ("q_temperature_scale", C.c_float)]


class ModelCfg(C.Structure):
    _fields_ = [("block_count", C.c_uint32), ("context_length", C.c_uint32),
                ("embedding_length", C.c_uint32), ("feed_forward_length", C.c_uint32),
                ("head_count", C.c_uint32), ("kv_head_count", C.c_uint32),
                ("key_length", C.c_uint32), ("value_length", C.c_uint32),
                ("vocab_size", C.c_uint32), ("rms_epsilon", C.c_float), ("yarn", Yarn)]


class Tensor(C.Structure):
    _fields_ = [("bytes", C.c_void_p), ("format", C.c_uint32)]


P, S, U32, U16, F32, I32, U64 = (C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint16, C.c_float,
                                 C.c_int, C.c_uint64)
_SIG = {
    "gho_set_threads": (None, [I32]),
    "gho_threads": (I32, []),
    "gho_f16_to_f32": (F32, [U16]),
    "gho_f32_to_f16": (U16, [F32]),
    "gho_f16_to_f32_slice": (None, [P, P, S]),
    "gho_f32_to_f16_slice": (None, [P, P, S]),
    "gho_scale_min": (None, [P, U32, C.POINTER(U32), C.POINTER(U32)]),
    "gho_dequant_row": (I32, [U32, P, S, S, P]),
    "gho_validate": (I32, [U32, S]),
    "gho_row_dot_q4k_scalar": (F32, [P, P, S, S]),
    "gho_row_dot_q4k_avx2": (F32, [P, P, S, S]),
    "gho_row_dot_q6k_scalar": (F32, [P, P, S, S]),
    "gho_row_dot_q6k_avx2": (F32, [P, P, S, S]),
    "gho_matmul": (I32, [U32, P, P, P, S, S]),
    "gho_logits": (I32, [U32, P, P, P, S, S]),
    "gho_matmul_batched": (I32, [U32, P, P, P, S, S, S]),
    "gho_row_dot_q4k_avx2_batched": (None, [P, P, S, S, P, S]),
    "gho_row_dot_q6k_avx2_batched": (None, [P, P, S, S, P, S]),
    "gho_attention_decode": (None, [P, P, P, P, S, S, S, S, S, S, S]),
    "gho_attention_prefill": (None, [P, P, P, P, S, S, S, S, S, S, S, S]),
    "gho_attention_decode_serial": (None, [P, P, P, P, S, S, S, S, S, S]),
    "gho_rmsnorm_x": (None, [P, P, P, S, F32, S]),
    "gho_silu_mul": (None, [P, P, P, S]),
    "gho_residual_add": (None, [P, P, S]),
    "gho_embed": (I32, [P, U32, P, S, S]),
    "gho_yarn_pair": (I32, [C.POINTER(Yarn), I32, S, S, C.POINTER(F32), C.POINTER(F32)]),
    "gho_yarn_post_scale": (F32, [C.POINTER(Yarn), I32, S]),
    "gho_yarn_correction_dims": (None, [C.POINTER(Yarn), C.POINTER(F32), C.POINTER(F32)]),
    "gho_rope_yarn": (I32, [P, S, S, S, C.POINTER(Yarn), I32]),
    "gho_argmax": (U32, [P, S]),
    "gho_topk": (S, [P, S, S, P, P]),
    "gho_kv_payload_offset": (U64, [S, S, S, S, S]),
    "gho_kv_buffer_bytes": (U64, [S, S, S, S]),
    "gho_model_create": (P, [C.POINTER(ModelCfg), C.POINTER(Tensor), C.POINTER(Tensor),
                             C.POINTER(Tensor), C.POINTER(Tensor), U32]),
    "gho_model_destroy": (None, [P]),
    "gho_model_token": (I32, [P, U32, U32]),
    "gho_model_prefill": (I32, [P, P, U32, U32, U32]),
    "gho_model_logits": (C.POINTER(F32), [P]),
    "gho_model_kv": (C.POINTER(U16), [P, I32]),
    "gho_model_x": (C.POINTER(F32), [P]),
    "gho_model_set_trace": (None, [P, I32]),
    "gho_model_load_kv": (I32, [P, P, P, U32, U32]),
    "gho_model_trace": (C.c_char_p, [P]),
    "gho_model_set_plant": (I32, [P, I32]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def f16(x) -> np.ndarray:
    """FP16 bits of x, narrowed RNE by the restated f32_to_f16 (backend/f16.rs:39-71)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
    out = np.empty(x.size, dtype=np.uint16)
    lib().gho_f32_to_f16_slice(_p(x), _p(out), x.size)
    return out


def f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16).reshape(-1))
    out = np.empty(h.size, dtype=np.float32)
    lib().gho_f16_to_f32_slice(_p(h), _p(out), h.size)
    return out


def dequant(fmt: int, w: np.ndarray, rows: int, in_dim: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty((rows, in_dim), dtype=np.float32)
    for r in range(rows):
        row = out[r]
        assert lib().gho_dequant_row(fmt, _p(w), r, in_dim, C.c_void_p(row.ctypes.data)) == 0
    return out


def matmul(fmt, a16, w, in_dim, out_dim) -> np.ndarray:
    a16 = np.ascontiguousarray(a16, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(out_dim, dtype=np.uint16)
    assert lib().gho_matmul(fmt, _p(out), _p(a16), _p(w), in_dim, out_dim) == 0
    return out


def logits(fmt, x16, w, in_dim, out_dim) -> np.ndarray:
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(out_dim, dtype=np.float32)
    assert lib().gho_logits(fmt, _p(out), _p(x16), _p(w), in_dim, out_dim) == 0
    return out


def matmul_batched(fmt, a16, w, in_dim, out_dim, n) -> np.ndarray:
    a16 = np.ascontiguousarray(a16, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(n * out_dim, dtype=np.uint16)
    assert lib().gho_matmul_batched(fmt, _p(out), _p(a16), _p(w), in_dim, out_dim, n) == 0
    return out


def attention_decode(q16, kc, vc, head_dim, kv_heads, q_heads, pos, layer, context):
    out = np.empty(q_heads * head_dim, dtype=np.uint16)
    lib().gho_attention_decode(_p(out), _p(np.ascontiguousarray(q16)), _p(kc), _p(vc), head_dim,
                               head_dim, kv_heads, q_heads, pos, layer, context)
    return out


def attention_prefill(q16, kc, vc, head_dim, kv_heads, q_heads, base, n, layer, context):
    out = np.empty(n * q_heads * head_dim, dtype=np.uint16)
    lib().gho_attention_prefill(_p(out), _p(np.ascontiguousarray(q16)), _p(kc), _p(vc), head_dim,
                                head_dim, kv_heads, q_heads, base, n, layer, context)
    return out


def rmsnorm_x(x, w16, dim, eps, rows):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows * dim, dtype=np.uint16)
    lib().gho_rmsnorm_x(_p(out), _p(x), _p(np.ascontiguousarray(w16)), dim, eps, rows)
    return out


def silu_mul(g16, u16):
    out = np.empty(g16.size, dtype=np.uint16)
    lib().gho_silu_mul(_p(out), _p(np.ascontiguousarray(g16)), _p(np.ascontiguousarray(u16)), g16.size)
    return out


def rope_yarn(x16, heads, head_dim, pos, yarn: Yarn, role):
    x = np.ascontiguousarray(x16, dtype=np.uint16).copy()
    assert lib().gho_rope_yarn(_p(x), heads, head_dim, pos, C.byref(yarn), role) == 0
    return x


def argmax(l) -> int:
    l = np.ascontiguousarray(l, dtype=np.float32)
    return int(lib().gho_argmax(_p(l), l.size))


def topk(l, k):
    l = np.ascontiguousarray(l, dtype=np.float32)
    idx = np.zeros(max(k, 1), dtype=np.uint32)
    val = np.zeros(max(k, 1), dtype=np.float32)
    n = lib().gho_topk(_p(l), l.size, k, _p(idx), _p(val))
    return [(int(i), v) for i, v in zip(idx[:n], val[:n])]  # np.float32: raw bits kept


class Model:
    """The oracle's graph restatement over host buffers (keeps the tensor arrays alive)."""

    def __init__(self, cfg: ModelCfg, tensors: dict, kv_context: int):
        self.cfg = cfg
        self.keep = []

        def t(key):
            if key not in tensors:
                return Tensor(None, 0)
            fmt, data = tensors[key]
            if fmt == FMT_F32:  # norms are narrowed to F16 at load (cpu/weights.rs:151-174)
                data, fmt = f16(data), FMT_F16
            data = np.ascontiguousarray(data)
            self.keep.append(data)
            return Tensor(data.ctypes.data, fmt)

        layers = (Tensor * (cfg.block_count * LAYER_TENSORS))()
        for li in range(cfg.block_count):
            for ti in range(LAYER_TENSORS):
                layers[li * LAYER_TENSORS + ti] = t((li, ti))
        emb, onorm, outp = t(("g", 16)), t(("g", 17)), t(("g", 18))
        self.h = lib().gho_model_create(C.byref(cfg), C.byref(emb), C.byref(onorm),
                                        C.byref(outp) if outp.bytes else None, layers, kv_context)
        self.kv_context = kv_context

    def close(self):
        if self.h:
            lib().gho_model_destroy(self.h)
            self.h = None

    def token(self, tok, pos):
        assert lib().gho_model_token(self.h, tok, pos) == 0

    def prefill(self, tokens, base, row_capacity):
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        assert lib().gho_model_prefill(self.h, _p(t), len(t), base, row_capacity) == 0

    def logits(self) -> np.ndarray:
        return np.ctypeslib.as_array(lib().gho_model_logits(self.h), (self.cfg.vocab_size,)).copy()

    def x(self) -> np.ndarray:
        return np.ctypeslib.as_array(lib().gho_model_x(self.h), (self.cfg.embedding_length,)).copy()

    def load_kv(self, k16, v16, src_context: int, positions: int):
        """Seed positions [0, positions) of every layer from caches of src_context positions."""
        k16 = np.ascontiguousarray(k16, dtype=np.uint16)
        v16 = np.ascontiguousarray(v16, dtype=np.uint16)
        assert lib().gho_model_load_kv(self.h, _p(k16), _p(v16), src_context, positions) == 0

    def set_trace(self, on: bool):
        lib().gho_model_set_trace(self.h, 1 if on else 0)

    def set_plant(self, plant: int):
        """Plant a known mistake (PLANT_*) to show that a parity check fails on it."""
        assert lib().gho_model_set_plant(self.h, plant) == 0

    def trace(self) -> list:
        return lib().gho_model_trace(self.h).decode().split("\n")[:-1]

    def kv(self, role) -> np.ndarray:
        n = self.cfg.block_count * self.kv_context * self.cfg.kv_head_count * self.cfg.key_length
        return np.ctypeslib.as_array(lib().gho_model_kv(self.h, role), (n,)).copy()
