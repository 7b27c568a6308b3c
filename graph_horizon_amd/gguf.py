"""GGUF model files: the native reader (gh_gguf_* in libgh_hip.so) and a GGUF v3 writer.

The reader is the C++ restatement of the engine's loader (gguf/loader/mod.rs, tensor_index.rs)
and of the dense mistral3 contract (family/mistral/config.rs, tensors.rs); it needs no GPU until
a model is loaded. The writer produces files in the same format (little-endian GGUF v3,
general.alignment-aligned data section) — for synthetic models, since no real checkpoint is
available offline.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

from . import _ffi as F
from . import synth

# GGUF metadata value types (loader/cursor.rs:86-127)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q4_K, GGML_Q6_K = 0, 1, 12, 14
_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
          8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
          14: (256, 210), 15: (256, 292)}


class GgufError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{F.STATUS.get(status, status)}: {message}")
        self.status = status
        self.message = message


def _check(rc: int):
    if rc != F.GH_OK:
        raise GgufError(rc, F.lib().gh_gguf_last_error().decode())


class GgufFile:
    """An open GGUF file (gh_gguf_open): header, metadata accessors and the tensor table."""

    def __init__(self, path: str):
        self.lib = F.lib()
        h = C.c_void_p()
        _check(self.lib.gh_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h
        v, tc, kc, do = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        _check(self.lib.gh_gguf_info(self.h, C.byref(v), C.byref(tc), C.byref(kc), C.byref(do)))
        self.version, self.tensor_count, self.kv_count, self.data_offset = (
            v.value, tc.value, kc.value, do.value)

    def close(self):
        if self.h:
            self.lib.gh_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor(self, index_or_name):
        if isinstance(index_or_name, str):
            i = C.c_uint64()
            _check(self.lib.gh_gguf_find(self.h, index_or_name.encode(), C.byref(i)))
            index_or_name = i.value
        info = F.GhGgufTensorInfo()
        _check(self.lib.gh_gguf_tensor(self.h, index_or_name, C.byref(info)))
        return {"name": info.name.decode(), "dims": list(info.dims[:info.n_dims]),
                "type": info.type, "offset": info.offset, "nbytes": info.nbytes,
                "data": info.data}

    def tensor_bytes(self, name: str) -> bytes:
        t = self.tensor(name)
        return C.string_at(t["data"], t["nbytes"])

    def tensors(self):
        return [self.tensor(i) for i in range(self.tensor_count)]

    def meta_u64(self, key: str) -> int:
        v = C.c_uint64()
        _check(self.lib.gh_gguf_meta_u64(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_f64(self, key: str) -> float:
        v = C.c_double()
        _check(self.lib.gh_gguf_meta_f64(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key: str):
        r = self.lib.gh_gguf_meta_str(self.h, key.encode())
        return None if r is None else r.decode()

    def meta_array_len(self, key: str) -> int:
        v = C.c_uint64()
        _check(self.lib.gh_gguf_meta_array_len(self.h, key.encode(), C.byref(v)))
        return v.value

    def model_config(self, kv_context: int, prefill_rows: int = 0, flags: int = 0) -> F.GhModelConfig:
        cfg = F.GhModelConfig()
        _check(self.lib.gh_gguf_model_config(self.h, kv_context, prefill_rows, C.byref(cfg)))
        cfg.flags = flags
        return cfg

    def check_model(self, cfg: F.GhModelConfig):
        _check(self.lib.gh_gguf_check_model(self.h, C.byref(cfg)))

    def load_model(self, model, cfg: F.GhModelConfig):
        """Uploads every tensor into a HipModel built with `cfg` (gh_gguf_load_model)."""
        _check(self.lib.gh_gguf_load_model(self.h, C.byref(cfg), model.h))


# ---- writer ----

def _pack_value(vtype: int, value) -> bytes:
    if vtype == STRING:
        b = value.encode()
        return struct.pack("<Q", len(b)) + b
    if vtype == ARRAY:
        elem, items = value
        return struct.pack("<IQ", elem, len(items)) + b"".join(_pack_value(elem, x) for x in items)
    return struct.pack(_SCALAR[vtype], value)


def _pack_string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def tensor_nbytes(dims, ggml_type: int) -> int:
    block, size = _BLOCK[ggml_type]
    n = int(np.prod(dims, dtype=np.uint64)) if dims else 1
    assert n % block == 0
    return n // block * size


def write_gguf(path: str, metadata, tensors, alignment: int = 32, version: int = 3):
    """metadata: [(key, vtype, value)]; ARRAY values are (elem_type, [items]).
    tensors: [(name, dims, ggml_type, bytes)] with GGUF dims (dims[0] = row length); data is
    laid out in order, each tensor aligned to `alignment`."""
    head = bytearray(b"GGUF")
    head += struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, value in metadata:
        head += _pack_string(key) + struct.pack("<I", vtype) + _pack_value(vtype, value)
    offsets, off = [], 0
    for name, dims, gtype, data in tensors:
        assert len(data) == tensor_nbytes(dims, gtype), name
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, dims, gtype, data), o in zip(tensors, offsets):
        head += _pack_string(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", gtype, o)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * ((-len(head)) % alignment))
        pos = 0
        for (name, dims, gtype, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + len(data)


_LAYER_NAMES = {F.T_ATTN_NORM: "attn_norm", F.T_ATTN_Q: "attn_q", F.T_ATTN_K: "attn_k",
                F.T_ATTN_V: "attn_v", F.T_ATTN_OUTPUT: "attn_output", F.T_FFN_NORM: "ffn_norm",
                F.T_FFN_GATE: "ffn_gate", F.T_FFN_UP: "ffn_up", F.T_FFN_DOWN: "ffn_down"}
_GLOBAL_NAMES = {F.T_TOKEN_EMBD: "token_embd", F.T_OUTPUT_NORM: "output_norm",
                 F.T_OUTPUT: "output"}


def tensor_name(layer: int, tensor: int) -> str:
    if layer == F.NO_LAYER:
        return _GLOBAL_NAMES[tensor] + ".weight"
    return f"blk.{layer}.{_LAYER_NAMES[tensor]}.weight"


def mistral3_metadata(shape: synth.Shape, context_length: int = 32768):
    """The mistral3 keys MistralConfig::from_metadata requires, for a synthetic shape (YaRN
    parameters as synth.yarn_params), with a placeholder token table of vocab_size entries."""
    y = synth.yarn_params(shape)
    a = "mistral3"
    return [
        ("general.architecture", STRING, a),
        ("general.alignment", U32, 32),
        (f"{a}.block_count", U32, shape.block_count),
        (f"{a}.context_length", U32, context_length),
        (f"{a}.embedding_length", U32, shape.embedding_length),
        (f"{a}.feed_forward_length", U32, shape.feed_forward_length),
        (f"{a}.vocab_size", U32, shape.vocab_size),
        (f"{a}.attention.head_count", U32, shape.head_count),
        (f"{a}.attention.head_count_kv", U32, shape.kv_head_count),
        (f"{a}.attention.key_length", U32, shape.head_dim),
        (f"{a}.attention.value_length", U32, shape.head_dim),
        (f"{a}.attention.layer_norm_rms_epsilon", F32, 1e-5),
        (f"{a}.attention.temperature_scale", F32, y["q_temperature_scale"]),
        (f"{a}.rope.dimension_count", U32, y["rope_dim"]),
        (f"{a}.rope.freq_base", F32, y["freq_base"]),
        (f"{a}.rope.scaling.type", STRING, "yarn"),
        (f"{a}.rope.scaling.factor", F32, y["factor"]),
        (f"{a}.rope.scaling.yarn_beta_fast", F32, y["beta_fast"]),
        (f"{a}.rope.scaling.yarn_beta_slow", F32, y["beta_slow"]),
        (f"{a}.rope.scaling.yarn_log_multiplier", F32, y["log_multiplier"]),
        (f"{a}.rope.scaling.original_context_length", U32, y["original_context"]),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(shape.vocab_size)])),
        ("tokenizer.ggml.bos_token_id", U32, 1),
        ("tokenizer.ggml.eos_token_id", U32, 2),
    ]


def gguf_tensors(shape: synth.Shape, tensors, tied: bool = False):
    """(layer, id, fmt, data) tuples (synth.model_tensors) as GGUF (name, dims, type, bytes)."""
    d = shape.embedding_length
    out = []
    for layer, tid, fmt, data in tensors:
        if tied and tid == F.T_OUTPUT:
            continue
        if tid in (F.T_ATTN_NORM, F.T_FFN_NORM, F.T_OUTPUT_NORM):
            dims = [d]
        elif tid in (F.T_TOKEN_EMBD, F.T_OUTPUT):
            dims = [d, shape.vocab_size]
        else:
            dims = list(synth.tensor_dims(shape, tid))
        out.append((tensor_name(layer, tid), dims, fmt, np.ascontiguousarray(data).tobytes()))
    return out


def write_synthetic_model(path: str, shape: synth.Shape, seed: int, tied: bool = False,
                          context_length: int = 32768):
    """A seeded random-init Q4_K_M model of `shape` as a GGUF file."""
    tensors = gguf_tensors(shape, synth.model_tensors(shape, seed), tied=tied)
    write_gguf(path, mistral3_metadata(shape, context_length), tensors)


def load_model(backend, path: str, kv_context: int, prefill_rows: int = 0, flags: int = 0):
    """A HipModel built from a GGUF file: configuration from its mistral3 metadata, every
    tensor uploaded by gh_gguf_load_model (checked before the first upload)."""
    from .backend import HipModel
    with GgufFile(path) as g:
        cfg = g.model_config(kv_context, prefill_rows, flags)
        g.check_model(cfg)
        model = HipModel(backend, cfg)
        try:
            g.load_model(model, cfg)
        except Exception:
            model.close()
            raise
    return model
