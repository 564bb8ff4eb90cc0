"""The C-ABI library loads and exports every symbol include/*.h declares
(CPU only: no compute calls)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(mslim_attn_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_symbols()
    for required in ("mslim_attn_last_error", "mslim_attn_ctx_new", "mslim_attn_decode_dense",
                     "mslim_attn_decode_paged", "mslim_attn_prefill_causal", "mslim_attn_rmsnorm",
                     "mslim_attn_rope", "mslim_attn_swiglu", "mslim_attn_logical_kv_sha256"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import mslim_attn

    if not os.path.exists(mslim_attn.LIB_PATH):
        pytest.fail("libmslim_attn.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(mslim_attn.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares exactly the header's entry points
    assert sorted(mslim_attn.EXPORTS) == declared_symbols()
    mslim_attn.library()


def test_library_is_gfx950_only():
    # the code object embedded in the library targets gfx950 and nothing else
    import mslim_attn

    blob = open(mslim_attn.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100", b"gfx1103", b"sm_"):
        assert b"amdgcn-amd-amdhsa--" + other not in blob


def test_error_before_context_is_reported():
    import mslim_attn

    lib = mslim_attn.library()
    assert lib.mslim_attn_decode_dense(None, None, None, None, None, 1, None, 0, 1, 1, 8, 1.0, 0) == -1
    assert b"null context" in lib.mslim_attn_last_error()


def test_split_auto_policy_is_layout_independent():
    # the split choice is a function of lengths and kv heads only, so the dense
    # and paged entry points pick the same partition
    from mslim_attn import split_count
    assert split_count(1024, 64) == 16
    assert split_count(1, 64) == 1
    assert split_count(65, 64) == 2


def test_host_library_exports_the_model_runner():
    # include/mslim_model.h is the runner's boundary, exported by libmslim_host
    from mslim_attn import model

    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "mslim_model.h")).read(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(mslim_model_[a-z0-9_]+)\s*\(", text)))
    assert declared == sorted(model.MODEL_EXPORTS)
    if not os.path.exists(model.HOST_LIB_PATH):
        pytest.fail("libmslim_host.so is not built: run __graft_entry__.build()")
    model.host_library()
    lib = ctypes.CDLL(model.HOST_LIB_PATH)
    assert [n for n in declared if not hasattr(lib, n)] == []
