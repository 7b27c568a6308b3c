"""forward::token and prefill::prefill restated in Python over the C ABI, op by op (test helper).

This is the engine's own structure — the graph recorders generic over `Backend`
(family/mistral/graph/forward.rs:68-83, block.rs:17-107, mlp.rs:12-61, tail.rs:22-59) —
driving the gh_* entry points one trait method at a time. The fused driver (gh_model_*) must
produce the same bits: its epilogues apply the same ops to the same FP16-rounded values.
"""
from __future__ import annotations

import numpy as np

from graph_horizon_amd import Yarn, synth
from graph_horizon_amd import _ffi as F

_LAYER_NAMES = {F.T_ATTN_NORM: "attn_norm", F.T_ATTN_Q: "q", F.T_ATTN_K: "k", F.T_ATTN_V: "v",
                F.T_ATTN_OUTPUT: "attn_out", F.T_FFN_NORM: "ffn_norm", F.T_FFN_GATE: "gate",
                F.T_FFN_UP: "up", F.T_FFN_DOWN: "down"}
_GLOBAL_NAMES = {F.T_TOKEN_EMBD: "token_embd", F.T_OUTPUT_NORM: "output_norm", F.T_OUTPUT: "output"}


class _Recorder:
    """The backend seen through the reference's shape recorder (graph/shape.rs:120-360): every
    op call is forwarded and logged under the name of the weight it was handed (looked up by
    device address), or under its op name when it takes none."""

    def __init__(self, hip, names):
        self.hip, self.names, self.trace = hip, names, []

    def _name(self, buf):
        return self.names.get(buf.addr, "?")

    def __getattr__(self, op):
        fn = getattr(self.hip, op)

        def call(*args):
            if op in ("matmul", "matmul_batched", "rmsnorm_x"):
                self.trace.append(self._name(args[2]))
            elif op == "logits":
                self.trace.append("logits:" + self._name(args[2]))
            elif op == "rope_yarn":
                self.trace.append("rope_q" if args[5] == F.ROPE_QUERY else "rope_k")
            elif op in ("begin", "submit", "embed", "kv_write", "silu_mul"):
                self.trace.append(op)
            elif op == "residual_add":
                self.trace.append("residual")
            elif op == "attention_decode":
                self.trace.append("attention")
            elif op in ("attention_prefill", "rope_yarn_batched"):
                self.trace.append(op)
            return fn(*args)
        return call


class AbiGraph:
    def __init__(self, hip, shape, seed, kv_context, tied=False, tensors=None):
        """`tensors`: (layer, tensor id, format, data) tuples (synth.model_tensors(shape, seed)
        when None); tied drops the output matrix, so the logits read token_embd
        (tail.rs:43-58)."""
        self.hip, self.shape = hip, shape
        self.w = {}
        names = {}
        for layer, tid, fmt, data in (tensors if tensors is not None else synth.model_tensors(shape, seed)):
            if tied and layer == F.NO_LAYER and tid == F.T_OUTPUT:
                continue
            if fmt == F.FMT_F32:
                self.w[(layer, tid)] = hip.load_weight(F.FMT_F32, data, data.size, 1)
            else:
                ind, outd = ((shape.embedding_length, shape.vocab_size) if layer == F.NO_LAYER
                             else synth.tensor_dims(shape, tid))
                self.w[(layer, tid)] = hip.load_weight(fmt, data, ind, outd)
            names[self.w[(layer, tid)].addr] = (_GLOBAL_NAMES[tid] if layer == F.NO_LAYER
                                                else f"l{layer}.{_LAYER_NAMES[tid]}")
        self.out_key = (F.NO_LAYER, F.T_OUTPUT if (F.NO_LAYER, F.T_OUTPUT) in self.w else F.T_TOKEN_EMBD)
        self.rec = _Recorder(hip, names)
        d, ffn = shape.embedding_length, shape.feed_forward_length
        qw, kw = shape.head_count * shape.head_dim, shape.kv_head_count * shape.head_dim
        a = hip.alloc_buffer
        self.x, self.normed = a(d * 4), a(d * 2)
        self.q, self.k, self.v, self.attn = a(qw * 2), a(kw * 2), a(kw * 2), a(qw * 2)
        self.proj, self.gate, self.up, self.act = a(d * 2), a(ffn * 2), a(ffn * 2), a(ffn * 2)
        self.ffn_out, self.logits = a(d * 2), a(shape.vocab_size * 4)
        n = shape.block_count * kv_context * kw
        self.kv = F.GhKv(a(n * 2), a(n * 2), F.KV_F16, shape.block_count, kv_context,
                         shape.kv_head_count, shape.head_dim, shape.head_dim)
        self.kv_context = kv_context
        self.yarn = Yarn(**synth.yarn_params(shape))

    def token(self, tok, pos, trace=None):
        """One decode token op by op; `trace` (a list) receives the recorded op names."""
        h, s = (self.rec, self.shape) if trace is not None else (self.hip, self.shape)
        self.rec.trace = trace if trace is not None else []
        d, ffn = s.embedding_length, s.feed_forward_length
        qw, kw = s.head_count * s.head_dim, s.kv_head_count * s.head_dim
        eps = 1e-5
        h.begin()
        h.embed(self.x, self.w[(F.NO_LAYER, F.T_TOKEN_EMBD)], tok, d)
        for li in range(s.block_count):
            w = lambda t: self.w[(li, t)]  # noqa: E731
            h.rmsnorm_x(self.normed, self.x, w(F.T_ATTN_NORM), d, eps, 1)
            h.matmul(self.q, self.normed, w(F.T_ATTN_Q), d, qw)
            h.matmul(self.k, self.normed, w(F.T_ATTN_K), d, kw)
            h.matmul(self.v, self.normed, w(F.T_ATTN_V), d, kw)
            h.rope_yarn(self.q, s.head_count, s.head_dim, pos, self.yarn, F.ROPE_QUERY)
            h.rope_yarn(self.k, s.kv_head_count, s.head_dim, pos, self.yarn, F.ROPE_KEY)
            off = ((li * self.kv_context + pos) * kw) * 2
            h.kv_write(self.kv, self.k, self.v, off, off, s.kv_head_count)
            h.attention_decode(self.attn, self.q, self.kv, s.head_count, pos, li)
            h.matmul(self.proj, self.attn, w(F.T_ATTN_OUTPUT), qw, d)
            h.residual_add(self.x, self.proj, d)
            h.rmsnorm_x(self.normed, self.x, w(F.T_FFN_NORM), d, eps, 1)
            h.matmul(self.gate, self.normed, w(F.T_FFN_GATE), d, ffn)
            h.matmul(self.up, self.normed, w(F.T_FFN_UP), d, ffn)
            h.silu_mul(self.act, self.gate, self.up, ffn)
            h.matmul(self.ffn_out, self.act, w(F.T_FFN_DOWN), ffn, d)
            h.residual_add(self.x, self.ffn_out, d)
        h.rmsnorm_x(self.normed, self.x, self.w[(F.NO_LAYER, F.T_OUTPUT_NORM)], d, eps, 1)
        h.logits(self.logits, self.normed, self.w[self.out_key], d, s.vocab_size)
        h.submit()
        return self.hip.read_logits(self.logits, s.vocab_size)

    def prefill(self, toks, base):
        """prefill::record_batch (graph/prefill/encode.rs:43-106, layer.rs:18-122) for one batch
        of rows at positions base..: every trait op batched over the rows, the tail on the
        last row. Returns the last row's logits."""
        h, s = self.hip, self.shape
        n = len(toks)
        d, ffn = s.embedding_length, s.feed_forward_length
        qw, kw = s.head_count * s.head_dim, s.kv_head_count * s.head_dim
        eps = 1e-5
        a = h.alloc_buffer
        x, normed = a(n * d * 4), a(n * d * 2)
        q, k, v, attn = a(n * qw * 2), a(n * kw * 2), a(n * kw * 2), a(n * qw * 2)
        proj, gate, up, act, ffn_out = a(n * d * 2), a(n * ffn * 2), a(n * ffn * 2), a(n * ffn * 2), a(n * d * 2)
        h.begin()
        for r, tok in enumerate(toks):
            h.embed(h.view(x, r * d * 4, d * 4), self.w[(F.NO_LAYER, F.T_TOKEN_EMBD)], int(tok), d)
        for li in range(s.block_count):
            w = lambda t: self.w[(li, t)]  # noqa: E731
            h.rmsnorm_x(normed, x, w(F.T_ATTN_NORM), d, eps, n)
            h.matmul_batched(q, normed, w(F.T_ATTN_Q), d, qw, n)
            h.matmul_batched(k, normed, w(F.T_ATTN_K), d, kw, n)
            h.matmul_batched(v, normed, w(F.T_ATTN_V), d, kw, n)
            h.rope_yarn_batched(q, k, s.head_count, s.kv_head_count, s.head_dim, base, n, self.yarn)
            off = ((li * self.kv_context + base) * kw) * 2
            h.kv_write(self.kv, k, v, off, off, n * s.kv_head_count)
            h.attention_prefill(attn, q, self.kv, s.head_count, base, n, li)
            h.matmul_batched(proj, attn, w(F.T_ATTN_OUTPUT), qw, d, n)
            h.residual_add(x, proj, n * d)
            h.rmsnorm_x(normed, x, w(F.T_FFN_NORM), d, eps, n)
            h.matmul_batched(gate, normed, w(F.T_FFN_GATE), d, ffn, n)
            h.matmul_batched(up, normed, w(F.T_FFN_UP), d, ffn, n)
            h.silu_mul(act, gate, up, n * ffn)
            h.matmul_batched(ffn_out, act, w(F.T_FFN_DOWN), ffn, d, n)
            h.residual_add(x, ffn_out, n * d)
        last = h.view(x, (n - 1) * d * 4, d * 4)
        h.rmsnorm_x(self.normed, last, self.w[(F.NO_LAYER, F.T_OUTPUT_NORM)], d, eps, 1)
        h.logits(self.logits, self.normed, self.w[self.out_key], d, s.vocab_size)
        h.submit()
        self.prefill_x = h.download(x, np.float32, n * d)
        for b in (x, normed, q, k, v, attn, proj, gate, up, act, ffn_out):
            h.free_buffer(b)
        return h.read_logits(self.logits, s.vocab_size)

    def read_x(self):
        return self.hip.download(self.x, np.float32, self.shape.embedding_length)
