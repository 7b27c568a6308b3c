"""Python mirror of the engine's `trait Backend` (backend/contract.rs:20-319) over the C ABI.

Each method forwards to the matching `gh_*` entry point with the same argument order; errors
raise `GhError` carrying the bounded status code and the backend's last error text. Host data
crosses as numpy arrays. This layer is plumbing for tests, the smoke check and the benchmark;
the numerics all run in the gfx950 kernels behind libgh_hip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _ffi as F
from ._ffi import GhBuf, GhKv, GhModelConfig, GhSampling, GhYarn


class GhError(RuntimeError):
    def __init__(self, code: int, what: str, detail: str = ""):
        self.code = code
        super().__init__(f"{what}: {F.STATUS.get(code, code)} {detail}".strip())


@dataclass
class Yarn:
    """backend/rope.rs:11-21."""
    rope_dim: int
    original_context: int
    freq_base: float
    factor: float
    beta_fast: float
    beta_slow: float
    log_multiplier: float
    q_temperature_scale: float

    def c(self) -> GhYarn:
        return GhYarn(self.rope_dim, self.original_context, self.freq_base, self.factor,
                      self.beta_fast, self.beta_slow, self.log_multiplier,
                      self.q_temperature_scale)


def _ptr(a: np.ndarray) -> C.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


class HipBackend:
    """One gfx950 device, one stream. Methods follow the trait's names and argument order."""

    def __init__(self, device: int = 0, code_objects: str | None = None):
        """code_objects: directory of the gh_*_gfx950.co files (default: next to the library)."""
        self.lib = F.lib()
        h = C.c_void_p()
        path = code_objects.encode() if code_objects else None
        rc = self.lib.gh_create(C.byref(F.GhConfig(device, path)), C.byref(h))
        if rc != F.GH_OK:
            raise GhError(rc, "gh_create", "(no gfx950 device, or code objects missing)")
        self.h = h
        self.enc = None

    def close(self):
        if self.h:
            self.lib.gh_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _ok(self, rc: int, what: str):
        if rc != F.GH_OK:
            raise GhError(rc, what, self.lib.gh_last_error(self.h).decode(errors="replace"))

    # ---- buffers ----
    def alloc_buffer(self, nbytes: int) -> GhBuf:
        b = GhBuf()
        self._ok(self.lib.gh_alloc_buffer(self.h, nbytes, C.byref(b)), "alloc_buffer")
        return b

    def free_buffer(self, buf: GhBuf):
        self._ok(self.lib.gh_free_buffer(self.h, C.byref(buf)), "free_buffer")

    def view(self, buf: GhBuf, offset: int, length: int) -> GhBuf:
        v = GhBuf()
        self._ok(self.lib.gh_view(self.h, C.byref(buf), offset, length, C.byref(v)), "view")
        return v

    def min_buffer_offset_alignment(self) -> int:
        return self.lib.gh_min_buffer_offset_alignment(self.h)

    def upload(self, buf: GhBuf, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        self._ok(self.lib.gh_upload(self.h, C.byref(buf), offset, _ptr(arr), arr.nbytes), "upload")

    def download(self, buf: GhBuf, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        self._ok(self.lib.gh_download(self.h, C.byref(buf), offset, _ptr(out), out.nbytes),
                 "download")
        return out

    def from_host(self, arr: np.ndarray) -> GhBuf:
        arr = np.ascontiguousarray(arr)
        b = self.alloc_buffer(max(arr.nbytes, 4))
        self.upload(b, arr)
        return b

    def load_weight(self, fmt: int, data: np.ndarray, in_dim: int, out_dim: int) -> GhBuf:
        data = np.ascontiguousarray(data)
        b = GhBuf()
        self._ok(self.lib.gh_load_weight(self.h, fmt, _ptr(data), data.nbytes, in_dim, out_dim,
                                         C.byref(b)), "load_weight")
        return b

    # ---- encoder ----
    def begin(self):
        e = C.c_void_p()
        self._ok(self.lib.gh_begin(self.h, C.byref(e)), "begin")
        self.enc = e
        return e

    def submit(self):
        e, self.enc = self.enc, None
        self._ok(self.lib.gh_submit(self.h, e), "submit")

    def no_barrier(self):
        self.lib.gh_no_barrier(self.h)

    def _run(self, name, *args):
        own = self.enc is None
        if own:
            self.begin()
        rc = getattr(self.lib, name)(self.h, self.enc, *args)
        if own:
            e, self.enc = self.enc, None
            rs = self.lib.gh_submit(self.h, e)
            rc = rc if rc != F.GH_OK else rs
        self._ok(rc, name)

    # ---- numeric ops (contract.rs order) ----
    def dequant_rows(self, out, w, row0, rows):
        self._run("gh_dequant_rows", C.byref(out), C.byref(w), row0, rows)

    def kv_write(self, kv: GhKv, k, v, k_off, v_off, vectors, k_meta=0, v_meta=0):
        self._run("gh_kv_write", C.byref(kv), C.byref(k), C.byref(v), k_off, v_off, k_meta,
                  v_meta, vectors)

    def embed(self, x, token_embd, token, embd):
        self._run("gh_embed", C.byref(x), C.byref(token_embd), token, embd)

    def matmul(self, out, a, w, in_dim, out_dim):
        self._run("gh_matmul", C.byref(out), C.byref(a), C.byref(w), in_dim, out_dim)

    def matmul_batched(self, out, a, w, in_dim, out_dim, n):
        self._run("gh_matmul_batched", C.byref(out), C.byref(a), C.byref(w), in_dim, out_dim, n)

    def logits(self, out, x, w, in_dim, out_dim):
        self._run("gh_logits", C.byref(out), C.byref(x), C.byref(w), in_dim, out_dim)

    def rmsnorm_x(self, out, x, w, dim, eps, rows):
        self._run("gh_rmsnorm_x", C.byref(out), C.byref(x), C.byref(w), dim, eps, rows)

    def rope_yarn(self, x, heads, head_dim, pos, yarn: Yarn, role):
        self._run("gh_rope_yarn", C.byref(x), heads, head_dim, pos, C.byref(yarn.c()), role)

    def rope_yarn_batched(self, q, k, q_heads, kv_heads, head_dim, base, rows, yarn: Yarn):
        self._run("gh_rope_yarn_batched", C.byref(q), C.byref(k), q_heads, kv_heads, head_dim,
                  base, rows, C.byref(yarn.c()))

    def silu_mul(self, out, gate, up, n):
        self._run("gh_silu_mul", C.byref(out), C.byref(gate), C.byref(up), n)

    def residual_add(self, x, y, n):
        self._run("gh_residual_add", C.byref(x), C.byref(y), n)

    def attention_decode(self, out, q, kv: GhKv, q_heads, pos, layer):
        self._run("gh_attention_decode", C.byref(out), C.byref(q), C.byref(kv), q_heads, pos,
                  layer)

    def attention_prefill(self, out, q, kv: GhKv, q_heads, base, n, layer):
        self._run("gh_attention_prefill", C.byref(out), C.byref(q), C.byref(kv), q_heads, base,
                  n, layer)

    # ---- read-back ----
    def read_logits(self, logits, vocab) -> np.ndarray:
        out = np.empty(vocab, dtype=np.float32)
        self._ok(self.lib.gh_read_logits(self.h, C.byref(logits), vocab, _ptr(out)), "read_logits")
        return out

    def read_argmax(self, logits, vocab) -> int:
        r = C.c_uint32()
        self._ok(self.lib.gh_read_argmax(self.h, C.byref(logits), vocab, C.byref(r)), "read_argmax")
        return r.value

    def read_topk(self, logits, vocab, k):
        idx = np.zeros(max(k, 1), dtype=np.uint32)
        val = np.zeros(max(k, 1), dtype=np.float32)
        cnt = C.c_uint64()
        self._ok(self.lib.gh_read_topk(self.h, C.byref(logits), vocab, k, _ptr(idx), _ptr(val),
                                       C.byref(cnt)), "read_topk")
        return [(int(i), v) for i, v in zip(idx[:cnt.value], val[:cnt.value])]  # np.float32: raw bits

    # ---- measurement ----
    def timer_start(self):
        self._ok(self.lib.gh_timer_start(self.h), "timer_start")

    def timer_stop(self) -> float:
        ms = C.c_float()
        self._ok(self.lib.gh_timer_stop(self.h, C.byref(ms)), "timer_stop")
        return ms.value

    def synchronize(self):
        self._ok(self.lib.gh_synchronize(self.h), "synchronize")

    def scratch_info(self):
        """(workspace bytes, attention-merge counter slots, generation) of the backend."""
        ws, cs, gen = C.c_uint64(), C.c_uint64(), C.c_uint64()
        self._ok(self.lib.gh_scratch_info(self.h, C.byref(ws), C.byref(cs), C.byref(gen)),
                 "scratch_info")
        return ws.value, cs.value, gen.value

    def set_attention_splits(self, splits: int):
        """Decode attention workgroups per (row, kv head); 0 = the backend's policy."""
        self._ok(self.lib.gh_set_attention_splits(self.h, splits), "set_attention_splits")

    def set_attention_xcd_merge(self, enable: bool):
        """Decode attention's split merge through one XCD's L2 (True, the default where the
        start-up probe confirmed the dispatch rule) or through device memory (False)."""
        self._ok(self.lib.gh_set_attention_xcd_merge(self.h, int(bool(enable))), "set_attention_xcd_merge")

    @property
    def xcd_count(self) -> int:
        """XCDs confirmed by the start-up dispatch probe (0: not confirmed)."""
        return int(self.lib.gh_xcd_count(self.h))


class HipModel:
    """The C++ graph driver (gh_model_*): MistralGraph's decode and prefill over the backend."""

    def __init__(self, backend: HipBackend, cfg: GhModelConfig):
        self.b = backend
        self.cfg = cfg
        h = C.c_void_p()
        backend._ok(backend.lib.gh_model_create(backend.h, C.byref(cfg), C.byref(h)), "model_create")
        self.h = h

    def close(self):
        if self.h:
            self.b.lib.gh_model_destroy(self.h)
            self.h = None

    def load_tensor(self, layer: int, tensor: int, fmt: int, data: np.ndarray):
        data = np.ascontiguousarray(data)
        self.b._ok(self.b.lib.gh_model_load_tensor(self.h, layer, tensor, fmt, _ptr(data),
                                                   data.nbytes), "model_load_tensor")

    def token(self, token: int, pos: int):
        self.b._ok(self.b.lib.gh_model_token(self.h, token, pos), "model_token")

    def prefill(self, tokens, base: int):
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        self.b._ok(self.b.lib.gh_model_prefill(self.h, _ptr(t), len(t), base), "model_prefill")

    def read_logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab_size, dtype=np.float32)
        self.b._ok(self.b.lib.gh_model_read_logits(self.h, _ptr(out)), "model_read_logits")
        return out

    def read_argmax(self) -> int:
        r = C.c_uint32()
        self.b._ok(self.b.lib.gh_model_read_argmax(self.h, C.byref(r)), "model_read_argmax")
        return r.value

    def decode_greedy(self, token: int, pos: int, steps: int) -> np.ndarray:
        out = np.zeros(max(steps, 1), dtype=np.uint32)
        self.b._ok(self.b.lib.gh_model_decode_greedy(self.h, token, pos, steps, _ptr(out)),
                   "model_decode_greedy")
        return out[:steps]

    def read_topk(self, k: int):
        idx = np.zeros(max(k, 1), dtype=np.uint32)
        val = np.zeros(max(k, 1), dtype=np.float32)
        cnt = C.c_uint64()
        self.b._ok(self.b.lib.gh_model_read_topk(self.h, k, _ptr(idx), _ptr(val), C.byref(cnt)),
                   "model_read_topk")
        return [(int(i), v) for i, v in zip(idx[:cnt.value], val[:cnt.value])]

    def generate(self, prompt, sampling: "GhSampling", max_tokens: int, eos: int = 0xFFFFFFFF):
        """generation::drive: prefill `prompt` at 0.., then up to max_tokens sampled tokens."""
        t = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        n = C.c_uint32()
        self.b._ok(self.b.lib.gh_model_generate(self.h, _ptr(t), len(t), C.byref(sampling),
                                                max_tokens, eos, _ptr(out), C.byref(n)),
                   "model_generate")
        return out[:n.value]

    def kv(self) -> GhKv:
        kv = GhKv()
        self.b._ok(self.b.lib.gh_model_kv(self.h, C.byref(kv)), "model_kv")
        return kv

    def read_x(self) -> np.ndarray:
        out = np.empty(self.cfg.embedding_length, dtype=np.float32)
        self.b._ok(self.b.lib.gh_model_read_x(self.h, _ptr(out)), "model_read_x")
        return out
