"""A model loaded from a GGUF file (gh_gguf_load_model) against the same tensors uploaded one by
one (gh_model_load_tensor): identical device weights, so prefill logits and greedy tokens must
match bit for bit — for a dedicated output matrix and for the tied case (no output.weight: the
token table doubles as the output matrix, cpu/weights.rs:80-95)."""
import numpy as np
import pytest

from graph_horizon_amd import HipModel, gguf, synth
from graph_horizon_amd import _ffi as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tied", [False, True])
def test_gguf_model_matches_direct_upload(hip, tmp_path, tied):
    shape, seed, ctx = synth.SHAPES["tiny"], 21, 96
    path = str(tmp_path / "m.gguf")
    gguf.write_synthetic_model(path, shape, seed, tied=tied)
    a = gguf.load_model(hip, path, ctx, prefill_rows=64)
    b = HipModel(hip, synth.model_config(shape, ctx, prefill_rows=64))
    embd = None
    for layer, tid, fmt, data in synth.model_tensors(shape, seed):
        if tid == F.T_TOKEN_EMBD:
            embd = (fmt, data)
        if tied and tid == F.T_OUTPUT:
            fmt, data = embd
        b.load_tensor(layer, tid, fmt, data)
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, shape.vocab_size, 37)]
    a.prefill(prompt, 0)
    b.prefill(prompt, 0)
    la, lb = a.read_logits(), b.read_logits()
    assert np.isfinite(la).all()
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    first = int(np.argmax(la))
    ta = a.decode_greedy(first, len(prompt), 12)
    tb = b.decode_greedy(first, len(prompt), 12)
    assert np.array_equal(ta, tb)
    a.close()
    b.close()
