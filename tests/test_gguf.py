"""GGUF reader (gh_gguf_* in libgh_hip.so) on the CPU: the reference loader's own cases
(gguf/loader/mod.rs:213-290, loader/cursor.rs:129-139), the mistral3 configuration contract
(family/mistral/config.rs:43-160) and tensor contract (family/mistral/tensors.rs:40-180), over
files written by graph_horizon_amd.gguf.write_gguf. No GPU is touched.
"""
import os
import struct

import numpy as np
import pytest

from graph_horizon_amd import _ffi as F
from graph_horizon_amd import gguf, synth
from graph_horizon_amd.gguf import GgufError, GgufFile


def _open(path):
    return GgufFile(str(path))


def _one_tensor(tmp_path, dims, gtype, offset, data_bytes, name="w", tag="t"):
    """Minimal v3 file with one tensor and no metadata (loader/mod.rs:196-231 builder)."""
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 1, 0)
    b += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims))
    b += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", gtype, offset)
    b += b"\0" * ((-len(b)) % 32) + b"\0" * data_bytes
    p = tmp_path / f"{tag}.gguf"
    p.write_bytes(bytes(b))
    return p


def _tensors_file(tmp_path, tensors, data_bytes, tag="m"):
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, len(tensors), 0)
    for name, dims, gtype, offset in tensors:
        b += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims))
        b += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", gtype, offset)
    b += b"\0" * ((-len(b)) % 32) + b"\0" * data_bytes
    p = tmp_path / f"{tag}.gguf"
    p.write_bytes(bytes(b))
    return p


def _err(path):
    with pytest.raises(GgufError) as e:
        _open(path)
    return e.value


# ---- loader/mod.rs tests ----

def test_well_formed_tensor_opens(tmp_path):
    with _open(_one_tensor(tmp_path, [256], 0, 0, 1024)) as g:
        assert g.tensor_count == 1 and g.data_offset % 32 == 0
        t = g.tensor(0)
        assert t["name"] == "w" and t["dims"] == [256] and t["nbytes"] == 1024


def test_tensor_offset_plus_len_beyond_file_is_rejected(tmp_path):
    e = _err(_one_tensor(tmp_path, [256], 0, 0, 0))
    assert "beyond end of file" in e.message


def test_incoherent_byte_len_is_rejected(tmp_path):
    e = _err(_one_tensor(tmp_path, [100], 12, 0, 4096))  # Q4_K [100]: 100 % 256 != 0
    assert "cannot size tensor" in e.message


def test_overlapping_tensor_ranges_are_rejected(tmp_path):
    e = _err(_tensors_file(tmp_path, [("a", [256], 0, 0), ("b", [256], 0, 512)], 2048))
    assert "overlaps tensor" in e.message


def test_tensor_offset_overflow_is_rejected(tmp_path):
    e = _err(_one_tensor(tmp_path, [256], 0, 2**64 - 1, 1024))
    assert "tensor offset overflow" in e.message


def test_known_bf16_tensor_layout_is_indexed(tmp_path):
    with _open(_one_tensor(tmp_path, [256], 30, 0, 512)) as g:
        t = g.tensor(0)
        assert t["type"] == 30 and t["nbytes"] == 512


def test_unknown_tensor_type_cannot_be_sized(tmp_path):
    e = _err(_one_tensor(tmp_path, [256], 99, 0, 4096))
    assert "cannot size tensor" in e.message


# ---- header / cursor ----

def test_bad_magic_and_version(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + struct.pack("<IQQ", 3, 0, 0))
    assert "bad magic" in _err(p).message
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    e = _err(p)
    assert e.status == -8 and "unsupported GGUF version 1" in e.message
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 2, 0, 0))
    assert "data section beyond end of file" in _err(p).message  # 24 bytes, aligned start 32
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 2, 0, 0) + bytes(8))
    with _open(p) as g:
        assert g.version == 2 and g.tensor_count == 0


def test_too_many_dims_rejected(tmp_path):
    e = _err(_one_tensor(tmp_path, [1, 1, 1, 1, 256], 0, 0, 1024))
    assert "too many dimensions" in e.message


def _meta_file(tmp_path, meta, tag="meta"):
    p = tmp_path / f"{tag}.gguf"
    gguf.write_gguf(str(p), meta, [])
    return p


def test_metadata_value_types_round_trip(tmp_path):
    meta = [("u8", gguf.U8, 7), ("i8", gguf.I8, -3), ("u16", gguf.U16, 65535),
            ("i16", gguf.I16, 1234), ("u32", gguf.U32, 2**32 - 1), ("i32", gguf.I32, -5),
            ("f32", gguf.F32, 0.25), ("b", gguf.BOOL, 1), ("s", gguf.STRING, "héllo"),
            ("u64", gguf.U64, 2**63), ("i64", gguf.I64, 42), ("f64", gguf.F64, -1.5),
            ("arr", gguf.ARRAY, (gguf.U32, [1, 2, 3])), ("sarr", gguf.ARRAY, (gguf.STRING, ["a", "bc"]))]
    with _open(_meta_file(tmp_path, meta)) as g:
        assert g.kv_count == len(meta)
        assert g.meta_u64("u8") == 7 and g.meta_u64("u16") == 65535 and g.meta_u64("u32") == 2**32 - 1
        assert g.meta_u64("u64") == 2**63 and g.meta_u64("i64") == 42 and g.meta_u64("i16") == 1234
        with pytest.raises(GgufError):
            g.meta_u64("i8")  # negative: not an unsigned value (GgufValue::as_u64)
        assert g.meta_f64("f32") == 0.25 and g.meta_f64("f64") == -1.5
        assert g.meta_str("s") == "héllo" and g.meta_str("u8") is None
        assert g.meta_array_len("arr") == 3 and g.meta_array_len("sarr") == 2


def test_invalid_utf8_rejected(tmp_path):
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2) + b"\xc3\x28"
    b += struct.pack("<I", 4) + struct.pack("<I", 1)
    p = tmp_path / "utf.gguf"
    p.write_bytes(bytes(b))
    assert "invalid utf-8" in _err(p).message


def test_duplicate_keys_last_wins(tmp_path):
    with _open(_meta_file(tmp_path, [("k", gguf.U32, 1), ("k", gguf.U32, 2)])) as g:
        assert g.meta_u64("k") == 2


def test_nested_arrays_and_unknown_value_types_rejected(tmp_path):
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 0, 1)
    b += struct.pack("<Q", 1) + b"k" + struct.pack("<I", 9) + struct.pack("<IQ", 9, 0)
    p = tmp_path / "nested.gguf"
    p.write_bytes(bytes(b))
    assert "nested arrays" in _err(p).message
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k"
    b += struct.pack("<I", 13)
    p.write_bytes(bytes(b))
    assert "unknown metadata value type 13" in _err(p).message


def test_alignment_metadata_sets_the_data_section(tmp_path):
    p = tmp_path / "al.gguf"
    gguf.write_gguf(str(p), [("general.alignment", gguf.U32, 256)],
                    [("w", [256], 0, bytes(1024))], alignment=256)
    with _open(p) as g:
        assert g.data_offset % 256 == 0 and g.data_offset > 0
        assert gguf.GgufFile.tensor_bytes(g, "w") == bytes(1024)


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "tiny.gguf"
    gguf.write_synthetic_model(str(p), synth.SHAPES["tiny"], 11)
    return p


def test_truncated_files_fail_cleanly(tmp_path, tiny_file):
    data = tiny_file.read_bytes()
    with _open(tiny_file) as g:
        header_end = g.data_offset
    cuts = sorted(set([0, 3, 4, 8, 16, 24, 30, 100, header_end // 2, header_end - 1,
                       header_end + 10, len(data) - 1]))
    for cut in cuts:
        p = tmp_path / f"cut{cut}.gguf"
        p.write_bytes(data[:cut])
        with pytest.raises(GgufError):
            _open(p)


def test_mutated_headers_never_crash(tmp_path, tiny_file):
    """Random byte flips inside the header: the reader either opens the file or returns an
    error — every read is bounds-checked, so nothing crashes."""
    data = bytearray(tiny_file.read_bytes())
    with _open(tiny_file) as g:
        header_end = g.data_offset
    rng = np.random.default_rng(5)
    outcomes = {"ok": 0, "err": 0}
    for i in range(150):
        m = bytearray(data[:header_end])
        for _ in range(int(rng.integers(1, 4))):
            m[int(rng.integers(0, header_end))] = int(rng.integers(0, 256))
        p = tmp_path / "mut.gguf"
        p.write_bytes(bytes(m) + bytes(data[header_end:]))
        try:
            with _open(p) as g:
                for k in range(min(g.tensor_count, 64)):
                    g.tensor(k)
            outcomes["ok"] += 1
        except GgufError:
            outcomes["err"] += 1
    assert outcomes["ok"] + outcomes["err"] == 150 and outcomes["err"] > 0


# ---- a whole synthetic model ----

def test_synthetic_model_round_trip(tiny_file):
    shape = synth.SHAPES["tiny"]
    want = {gguf.tensor_name(l, t): (f, np.ascontiguousarray(d).tobytes())
            for l, t, f, d in synth.model_tensors(shape, 11)}
    with _open(tiny_file) as g:
        assert g.version == 3 and g.tensor_count == len(want)
        assert g.meta_str("general.architecture") == "mistral3"
        for t in g.tensors():
            fmt, data = want[t["name"]]
            assert t["type"] == fmt and t["nbytes"] == len(data) and t["offset"] % 32 == 0
            assert g.tensor_bytes(t["name"]) == data
        cfg = g.model_config(256, 64)
        ref = synth.model_config(shape, 256, prefill_rows=64)
        for f, _ in F.GhModelConfig._fields_:
            if f == "yarn":
                for y, _ in F.GhYarn._fields_:
                    assert getattr(cfg.yarn, y) == pytest.approx(getattr(ref.yarn, y), rel=1e-7), y
            elif f != "context_length":
                assert getattr(cfg, f) == pytest.approx(getattr(ref, f), rel=1e-7), f
        assert cfg.context_length == 32768
        g.check_model(cfg)
        with pytest.raises(GgufError) as e:
            g.model_config(40000, 64)  # beyond mistral3.context_length
        assert e.value.status == -5


def _model_meta_without(shape, drop=None, replace=None):
    meta = []
    for k, t, v in gguf.mistral3_metadata(shape):
        if k == drop:
            continue
        if replace and k in replace:
            t, v = replace[k]
        meta.append((k, t, v))
    return meta


REQUIRED = ["mistral3.block_count", "mistral3.context_length", "mistral3.embedding_length",
            "mistral3.feed_forward_length", "mistral3.vocab_size", "mistral3.attention.head_count",
            "mistral3.attention.head_count_kv", "mistral3.attention.key_length",
            "mistral3.attention.value_length", "mistral3.rope.dimension_count",
            "mistral3.rope.freq_base", "mistral3.attention.layer_norm_rms_epsilon",
            "mistral3.rope.scaling.factor", "mistral3.rope.scaling.yarn_beta_fast",
            "mistral3.rope.scaling.yarn_beta_slow", "mistral3.rope.scaling.yarn_log_multiplier",
            "mistral3.rope.scaling.original_context_length",
            "mistral3.attention.temperature_scale", "mistral3.rope.scaling.type"]


@pytest.mark.parametrize("key", REQUIRED)
def test_each_required_key_is_enforced(tmp_path, key):
    shape = synth.SHAPES["tiny"]
    p = _meta_file(tmp_path, _model_meta_without(shape, drop=key), tag="cfg")
    with _open(p) as g, pytest.raises(GgufError) as e:
        g.model_config(128, 64)
    assert e.value.message == f"E06 missing or invalid GGUF metadata '{key}'"


@pytest.mark.parametrize("replace,key", [
    ({"mistral3.rope.scaling.type": (gguf.STRING, "linear")}, "mistral3.rope.scaling.type"),
    ({"mistral3.block_count": (gguf.U32, 0)}, "mistral3.block_count"),
    ({"mistral3.block_count": (gguf.I32, 2)}, "mistral3.block_count"),       # signed: rejected
    ({"mistral3.rope.freq_base": (gguf.F64, 1e6)}, "mistral3.rope.freq_base"),  # F64: rejected
    ({"mistral3.rope.freq_base": (gguf.F32, float("inf"))}, "mistral3.rope.freq_base"),
    ({"mistral3.rope.scaling.factor": (gguf.F32, -1.0)}, "mistral3.rope.scaling.factor"),
    ({"mistral3.vocab_size": (gguf.U32, 2047)}, "mistral3.vocab_size"),      # != token table
    ({"mistral3.attention.head_count_kv": (gguf.U32, 3)}, "mistral3.attention.head_count"),
    ({"mistral3.attention.head_count_kv": (gguf.U32, 16)}, "mistral3.attention.head_count"),
    ({"mistral3.embedding_length": (gguf.U32, 516)}, "mistral3.attention.head_count"),
    ({"mistral3.rope.dimension_count": (gguf.U32, 127)}, "mistral3.rope.dimension_count"),
    ({"mistral3.rope.dimension_count": (gguf.U32, 256)}, "mistral3.rope.dimension_count"),
])
def test_invalid_metadata_values(tmp_path, replace, key):
    shape = synth.SHAPES["tiny"]
    p = _meta_file(tmp_path, _model_meta_without(shape, replace=replace), tag="bad")
    with _open(p) as g, pytest.raises(GgufError) as e:
        g.model_config(128, 64)
    assert e.value.message == f"E06 missing or invalid GGUF metadata '{key}'"


def _model_file(tmp_path, shape, mutate, tag):
    tensors = gguf.gguf_tensors(shape, synth.model_tensors(shape, 3))
    tensors = mutate(tensors)
    p = tmp_path / f"{tag}.gguf"
    gguf.write_gguf(str(p), gguf.mistral3_metadata(shape), tensors)
    return p


def _check_model_error(p, cfg_rows=128):
    with _open(p) as g:
        cfg = g.model_config(cfg_rows, 64)
        with pytest.raises(GgufError) as e:
            g.check_model(cfg)
    return e.value


def test_tensor_contract(tmp_path):
    shape = synth.SHAPES["tiny"]
    # missing tensor -> E07
    p = _model_file(tmp_path, shape, lambda ts: [t for t in ts if t[0] != "blk.1.attn_v.weight"], "miss")
    assert _check_model_error(p).message == "E07 missing or invalid tensor 'blk.1.attn_v.weight'"
    # transposed dims -> E07
    def transpose(ts):
        return [(n, dims[::-1] if n == "blk.0.attn_q.weight" else dims, f, b) for n, dims, f, b in ts]
    p = _model_file(tmp_path, shape, transpose, "dims")
    assert _check_model_error(p).message == "E07 missing or invalid tensor 'blk.0.attn_q.weight'"
    # Q8_0 matrix -> E08 (same byte count per element row is irrelevant: the type is refused)
    def q8(ts):
        out = []
        for n, dims, f, b in ts:
            if n == "blk.0.ffn_up.weight":
                b = bytes(gguf.tensor_nbytes(dims, 8))
                f = 8
            out.append((n, dims, f, b))
        return out
    p = _model_file(tmp_path, shape, q8, "q8")
    e = _check_model_error(p)
    assert e.message == "E08 unsupported tensor type 'Q8_0'" and e.status == -8
    # F16 norm -> E08 (norms are F32 in the file, tensors.rs:135-146)
    def f16norm(ts):
        return [(n, dims, 1, bytes(len(b) // 2)) if n == "blk.1.ffn_norm.weight" else (n, dims, f, b)
                for n, dims, f, b in ts]
    p = _model_file(tmp_path, shape, f16norm, "f16n")
    assert _check_model_error(p).message == "E08 unsupported tensor type 'F16'"


def test_tied_output_is_accepted(tmp_path):
    shape = synth.SHAPES["tiny"]
    p = tmp_path / "tied.gguf"
    gguf.write_synthetic_model(str(p), shape, 4, tied=True)
    with _open(p) as g:
        with pytest.raises(GgufError):
            g.tensor("output.weight")
        g.check_model(g.model_config(128, 64))
