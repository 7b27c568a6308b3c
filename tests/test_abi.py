"""The C-ABI library loads and exports every entry point include/gh_backend.h declares (no GPU)."""
import ctypes as C
import os
import re
import subprocess

from graph_horizon_amd import _ffi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gh_backend.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_trait_surface():
    names = set(declared_functions())
    # contract.rs:20-319: one entry point per trait method
    trait = {"gh_alloc_buffer", "gh_free_buffer", "gh_view", "gh_min_buffer_offset_alignment",
             "gh_kv_write", "gh_begin", "gh_submit", "gh_no_barrier", "gh_embed", "gh_matmul",
             "gh_matmul_batched", "gh_logits", "gh_rmsnorm_x", "gh_rope_yarn",
             "gh_rope_yarn_batched", "gh_silu_mul", "gh_residual_add", "gh_attention_decode",
             "gh_attention_prefill", "gh_read_logits", "gh_read_argmax", "gh_read_topk"}
    assert trait <= names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_ffi.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", _ffi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (gh_\w+)", out))
    assert set(declared_functions()) <= exported


def test_python_binding_covers_the_header():
    assert set(declared_functions()) == set(_ffi.SIGNATURES)


def test_code_objects_present_and_gfx950():
    for m in ("gh_quant", "gh_gemv", "gh_glue", "gh_attention"):
        path = os.path.join(_ffi.LIB_DIR, f"{m}_gfx950.co")
        data = open(path, "rb").read()
        assert data[:4] == b"\x7fELF"
        assert b"gfx950" in data


def test_no_device_is_a_bounded_error():
    """Without a gfx950 device gh_create fails with GH_E_NO_DEVICE instead of crashing. Run in a
    child process that hides every GPU, so the check holds on a GPU host too."""
    code = ("import ctypes as C, sys; sys.path.insert(0, %r); from graph_horizon_amd import _ffi;"
            "h = C.c_void_p(); rc = _ffi.lib().gh_create(None, C.byref(h)); print(rc)") % ROOT
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = subprocess.run(["python", "-c", code], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    assert int(r.stdout.strip().splitlines()[-1]) == -2


def test_prefill_rows_policy():
    """gh_prefill_rows (host-only): 2048-row chunks, capped by the context."""
    lib = C.CDLL(_ffi.LIB_PATH)
    lib.gh_prefill_rows.restype = C.c_uint32
    lib.gh_prefill_rows.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    assert lib.gh_prefill_rows(None, 34, 8192) == 2048
    assert lib.gh_prefill_rows(None, 40, 600) == 600
    assert lib.gh_prefill_rows(None, 1, 131072) == 2048
