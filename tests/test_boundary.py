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


def _one_per_cu_split(lens, kv_heads):
    per = -(-sum(lens) * kv_heads // 256)
    return min(16384, max(256, -(-per // 256) * 256))


def test_auto_split_choices():
    # host-only policy of split_tokens = 0 (mslim_attn_decode_auto_split)
    import numpy as np
    from mslim_attn import auto_split
    # equal lengths keep about one workgroup per CU: cfg4 (256 workgroups), cfg5
    assert auto_split([32768] * 4, 8) == 4096
    assert auto_split([4224] * 8, 8) == 1280
    # ragged lengths take the split that evens out the busiest CU when the
    # last partitions launch after the full ones, longest first; both were
    # measured faster on MI355X than the one-per-CU split (116.7 vs 154 us and
    # 101.6 vs 149 us)
    cfg3 = np.random.default_rng(20261203).integers(512, 8193, size=32).tolist()
    assert auto_split(cfg3, 8) == 2304 and _one_per_cu_split(cfg3, 8) == 4608
    skew = np.random.default_rng(17).integers(1024, 32769, size=8).tolist()
    assert auto_split(skew, 8) == 2304
    # batches too small to give each CU 256 tokens take 128-token splits:
    # cfg1 (B = 1, T = 1,024, 8 kv heads) and short decode contexts
    assert auto_split([1024], 8) == 128
    assert auto_split([300, 17, 3000], 8) == 128
    assert auto_split([4096, 4096], 8) == 256


def test_auto_split_invariants():
    import numpy as np
    from mslim_attn import auto_split, split_count
    for seed in range(40):
        rng = np.random.default_rng(seed)
        lens = rng.integers(1, 65537, size=int(rng.integers(1, 65))).tolist()
        kvh = int(rng.choice([1, 2, 4, 8, 16]))
        s, s1 = auto_split(lens, kvh), _one_per_cu_split(lens, kvh)
        if sum(lens) * kvh <= 128 * 256:
            assert s == 128
            continue
        assert s % 256 == 0 and 256 <= s <= s1 and s >= s1 // 4 - 255
        if s != s1:
            assert sum(split_count(t, s) for t in lens) * kvh <= 2048
        if len(set(lens)) == 1:
            assert s == s1
        assert auto_split(list(reversed(lens)), kvh) % 256 == 0
    assert auto_split([1] * 64, 1) == 128


def test_auto_split_rejects_bad_batches():
    from mslim_attn import MslimAttnError, auto_split
    for lens, kvh in (([], 8), ([0], 8), ([5] * 4097, 8), ([5], 0)):
        with pytest.raises(MslimAttnError, match="code=-1"):
            auto_split(lens, kvh)


def test_prefill_split_choices():
    # host-only plan of mslim_attn_prefill_causal: chunk length in key tiles,
    # 0 when the launch keeps every CU busy without splitting
    from mslim_attn import MslimAttnError, prefill_split_tiles
    assert prefill_split_tiles(8192, 0, 64, 8, 128) == 0     # cfg4: 2,048 workgroups
    assert prefill_split_tiles(2048, 0, 32, 8, 128) == 20    # cfg2: 256 workgroups of 1..32 tiles
    assert prefill_split_tiles(512, 3584, 32, 8, 128) == 16  # a decoder prompt chunk after 3,584 tokens
    assert prefill_split_tiles(512, 512, 32, 8, 128) == 8
    assert prefill_split_tiles(1000, 777, 32, 8, 128) == 14
    # 32-row blocks (64/8 heads) after 777 tokens, and a first 512-token chunk:
    # measured no slower unsplit, so not split
    assert prefill_split_tiles(1000, 777, 64, 8, 128) == 0
    assert prefill_split_tiles(512, 0, 32, 8, 128) == 0
    assert prefill_split_tiles(100, 0, 32, 8, 128) == 0
    assert prefill_split_tiles(300, 0, 4, 2, 80) == 0        # generic kernel: never split
    for args in ((0, 0, 32, 8, 128), (5, -1, 32, 8, 128), (5, 0, 32, 3, 128)):
        with pytest.raises(MslimAttnError):
            prefill_split_tiles(*args)


def test_prefill_pool_choices():
    # host-only plan of mslim_attn_prefill_causal: row blocks per XCD handed
    # out at run time; a quarter of each XCD's slice up to 64, only for
    # unsplit launches with at least two row blocks per CU (64 per XCD)
    from mslim_attn import MslimAttnError, prefill_pool_items
    assert prefill_pool_items(8192, 0, 64, 8, 128) == 64     # cfg4: 256 row blocks per XCD
    assert prefill_pool_items(16384, 0, 64, 8, 128) == 64    # 512 per XCD: capped
    assert prefill_pool_items(4096, 0, 64, 8, 128) == 32     # 128 per XCD
    assert prefill_pool_items(8192, 0, 32, 8, 128) == 32     # 64-row blocks of 4 heads
    assert prefill_pool_items(2048, 0, 64, 8, 128) == 16     # 64 per XCD
    assert prefill_pool_items(1024, 0, 64, 8, 128) == 0      # 32 per XCD: one per CU
    assert prefill_pool_items(2048, 0, 32, 8, 128) == 0      # cfg2 is split
    assert prefill_pool_items(4096, 0, 4, 2, 80) == 0        # generic kernel: static
    for args in ((0, 0, 32, 8, 128), (5, -1, 32, 8, 128), (5, 0, 32, 3, 128)):
        with pytest.raises(MslimAttnError):
            prefill_pool_items(*args)
