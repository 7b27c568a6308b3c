"""ctypes declarations of the C ABI in include/gh_backend.h (the drop-in boundary).

Loads graph_horizon_amd/lib/libgh_hip.so (built in-tree). There is no fallback: if the
library or its gfx950 code objects are missing, loading fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libgh_hip.so")

GH_OK = 0
STATUS = {
    0: "GH_OK",
    -1: "GH_E_INVALID",
    -2: "GH_E_NO_DEVICE",
    -3: "GH_E_HIP",
    -4: "GH_E_OOM",
    -5: "GH_E_RANGE",
    -6: "GH_E_MODULE",
    -7: "GH_E_STATE",
    -8: "GH_E_UNSUPPORTED",
}
FMT_F32, FMT_F16, FMT_Q4_K, FMT_Q6_K = 0, 1, 12, 14
BUF_ALLOC, BUF_VIEW, BUF_WEIGHT = 1, 2, 3
ROPE_QUERY, ROPE_KEY = 0, 1
KV_F16 = 0
NO_LAYER = 0xFFFFFFFF
(T_ATTN_NORM, T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_OUTPUT, T_FFN_NORM, T_FFN_GATE, T_FFN_UP,
 T_FFN_DOWN) = range(9)
T_TOKEN_EMBD, T_OUTPUT_NORM, T_OUTPUT = 16, 17, 18


class GhBuf(C.Structure):
    _fields_ = [("addr", C.c_uint64), ("bytes", C.c_uint64), ("format", C.c_uint32),
                ("kind", C.c_uint32), ("rows", C.c_uint32), ("cols", C.c_uint32)]


class GhConfig(C.Structure):
    _fields_ = [("device", C.c_int32), ("code_object_path", C.c_char_p)]


class GhYarn(C.Structure):
    _fields_ = [("rope_dim", C.c_uint32), ("original_context", C.c_uint32),
                ("freq_base", C.c_float), ("factor", C.c_float), ("beta_fast", C.c_float),
                ("beta_slow", C.c_float), ("log_multiplier", C.c_float),
                ("q_temperature_scale", C.c_float)]


class GhKv(C.Structure):
    _fields_ = [("k", GhBuf), ("v", GhBuf), ("scheme", C.c_uint32), ("block_count", C.c_uint32),
                ("context", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("value_dim", C.c_uint32)]


class GhSampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("min_p", C.c_float), ("repeat_penalty", C.c_float), ("seed", C.c_uint64)]


SAMPLE_GREEDY, SAMPLE_TOPK, SAMPLE_FALLBACK = 0, 1, 2


class GhModelConfig(C.Structure):
    _fields_ = [("block_count", C.c_uint32), ("context_length", C.c_uint32),
                ("embedding_length", C.c_uint32), ("feed_forward_length", C.c_uint32),
                ("head_count", C.c_uint32), ("kv_head_count", C.c_uint32),
                ("key_length", C.c_uint32), ("value_length", C.c_uint32),
                ("vocab_size", C.c_uint32), ("rms_epsilon", C.c_float), ("yarn", GhYarn),
                ("kv_context", C.c_uint32), ("prefill_rows", C.c_uint32),
                ("flags", C.c_uint32)]


MODEL_NO_GRAPH = 1
MODEL_NO_F16_WEIGHTS = 2


class GhGgufTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("type", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("data", C.c_void_p)]


P = C.c_void_p
BUFP = C.POINTER(GhBuf)
U32, U64, F32, I32 = C.c_uint32, C.c_uint64, C.c_float, C.c_int

# name -> (restype, argtypes); every entry point declared in include/gh_backend.h
SIGNATURES = {
    "gh_create": (I32, [C.POINTER(GhConfig), C.POINTER(P)]),
    "gh_destroy": (None, [P]),
    "gh_last_error": (C.c_char_p, [P]),
    "gh_alloc_buffer": (I32, [P, U64, BUFP]),
    "gh_free_buffer": (I32, [P, BUFP]),
    "gh_view": (I32, [P, BUFP, U64, U64, BUFP]),
    "gh_min_buffer_offset_alignment": (U64, [P]),
    "gh_upload": (I32, [P, BUFP, U64, P, U64]),
    "gh_download": (I32, [P, BUFP, U64, P, U64]),
    "gh_load_weight": (I32, [P, U32, P, U64, U32, U32, BUFP]),
    "gh_dequant_rows": (I32, [P, P, BUFP, BUFP, U32, U32]),
    "gh_begin": (I32, [P, C.POINTER(P)]),
    "gh_submit": (I32, [P, P]),
    "gh_no_barrier": (None, [P]),
    "gh_kv_write": (I32, [P, P, C.POINTER(GhKv), BUFP, BUFP, U64, U64, U64, U64, U32]),
    "gh_embed": (I32, [P, P, BUFP, BUFP, U32, U32]),
    "gh_matmul": (I32, [P, P, BUFP, BUFP, BUFP, U32, U32]),
    "gh_matmul_batched": (I32, [P, P, BUFP, BUFP, BUFP, U32, U32, U32]),
    "gh_logits": (I32, [P, P, BUFP, BUFP, BUFP, U32, U32]),
    "gh_rmsnorm_x": (I32, [P, P, BUFP, BUFP, BUFP, U32, F32, U32]),
    "gh_rope_yarn": (I32, [P, P, BUFP, U32, U32, U32, C.POINTER(GhYarn), U32]),
    "gh_rope_yarn_batched": (I32, [P, P, BUFP, BUFP, U32, U32, U32, U32, U32, C.POINTER(GhYarn)]),
    "gh_silu_mul": (I32, [P, P, BUFP, BUFP, BUFP, U32]),
    "gh_residual_add": (I32, [P, P, BUFP, BUFP, U32]),
    "gh_attention_decode": (I32, [P, P, BUFP, BUFP, C.POINTER(GhKv), U32, U32, U32]),
    "gh_attention_decode_noalloc": (I32, [P, P, BUFP, BUFP, C.POINTER(GhKv), U32, U32, U32]),
    "gh_attention_prefill": (I32, [P, P, BUFP, BUFP, C.POINTER(GhKv), U32, U32, U32, U32]),
    "gh_read_logits": (I32, [P, BUFP, U64, P]),
    "gh_read_argmax": (I32, [P, BUFP, U64, C.POINTER(U32)]),
    "gh_read_topk": (I32, [P, BUFP, U64, U64, P, P, C.POINTER(U64)]),
    "gh_timer_start": (I32, [P]),
    "gh_timer_stop": (I32, [P, C.POINTER(F32)]),
    "gh_synchronize": (I32, [P]),
    "gh_set_attention_splits": (I32, [P, U32]),
    "gh_set_attention_xcd_merge": (I32, [P, I32]),
    "gh_xcd_count": (U32, [P]),
    "gh_stream_probe": (I32, [P, P, BUFP, U64, U64, BUFP, U32]),
    "gh_scratch_info": (I32, [P, C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
    "gh_model_create": (I32, [P, C.POINTER(GhModelConfig), C.POINTER(P)]),
    "gh_model_destroy": (None, [P]),
    "gh_model_load_tensor": (I32, [P, U32, U32, U32, P, U64]),
    "gh_model_token": (I32, [P, U32, U32]),
    "gh_model_prefill": (I32, [P, P, U32, U32]),
    "gh_model_read_logits": (I32, [P, P]),
    "gh_model_read_argmax": (I32, [P, C.POINTER(U32)]),
    "gh_model_decode_greedy": (I32, [P, U32, U32, U32, P]),
    "gh_model_kv": (I32, [P, C.POINTER(GhKv)]),
    "gh_model_read_x": (I32, [P, P]),
    "gh_model_weight": (I32, [P, U32, U32, BUFP]),
    "gh_model_read_topk": (I32, [P, U64, P, P, C.POINTER(U64)]),
    "gh_prefill_rows": (U32, [P, U32, U32]),
    "gh_model_generate": (I32, [P, P, U32, C.POINTER(GhSampling), U32, U32, P, C.POINTER(U32)]),
    "gh_sampling_plan": (I32, [C.POINTER(GhSampling), C.POINTER(U32)]),
    "gh_rng_seed": (U64, [U64]),
    "gh_rng_next_f32": (C.c_float, [C.POINTER(U64)]),
    "gh_sample": (I32, [P, U64, C.POINTER(GhSampling), P, U64, C.POINTER(U64), C.POINTER(U32)]),
    "gh_sample_from_candidates": (I32, [P, P, U64, C.POINTER(GhSampling), C.POINTER(U64),
                                        C.POINTER(U32)]),
    "gh_gguf_last_error": (C.c_char_p, []),
    "gh_gguf_open": (I32, [C.c_char_p, C.POINTER(P)]),
    "gh_gguf_close": (None, [P]),
    "gh_gguf_info": (I32, [P, C.POINTER(U32), C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
    "gh_gguf_tensor": (I32, [P, U64, C.POINTER(GhGgufTensorInfo)]),
    "gh_gguf_find": (I32, [P, C.c_char_p, C.POINTER(U64)]),
    "gh_gguf_meta_u64": (I32, [P, C.c_char_p, C.POINTER(U64)]),
    "gh_gguf_meta_f64": (I32, [P, C.c_char_p, C.POINTER(C.c_double)]),
    "gh_gguf_meta_str": (C.c_char_p, [P, C.c_char_p]),
    "gh_gguf_meta_array_len": (I32, [P, C.c_char_p, C.POINTER(U64)]),
    "gh_gguf_model_config": (I32, [P, U32, U32, C.POINTER(GhModelConfig)]),
    "gh_gguf_check_model": (I32, [P, C.POINTER(GhModelConfig)]),
    "gh_gguf_load_model": (I32, [P, C.POINTER(GhModelConfig), P]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded libgh_hip.so with every C-ABI signature declared."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the gfx950 backend first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib
