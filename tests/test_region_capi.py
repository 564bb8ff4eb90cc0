"""The region store's C ABI (include/mslim_region.h, libmslim_host) on the
CPU: the reference's GpuRegionStore API (gpu_region_store.rs:118-928) as the
native CPU runtime drives it (native_cpu_adapter.rs:337, :458-484) --
single-token and batched appends, partial reads, reopen of a persisted
store, and the logical K/V digest checked against the oracle's restatement
(gpu_region_store.rs:341-371)."""
import os
import re

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
QH, KVH, D, LAYERS = 8, 2, 64, 3


def rows(rng, n):
    return oracle.write_bf16(rng.standard_normal(n * KVH * D, dtype=np.float32)).reshape(n, KVH * D)


def test_header_declares_the_binding_and_library_exports_it():
    import ctypes

    from mslim_attn import model, region

    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "mslim_region.h")).read(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(mslim_region_[a-z0-9_]+)\s*\(", text)))
    assert declared == sorted(region.REGION_EXPORTS)
    lib = ctypes.CDLL(model.HOST_LIB_PATH)
    assert all(hasattr(lib, name) for name in declared)


def test_append_read_digest_and_reopen(tmp_path):
    from mslim_attn.region import RegionStore

    rng = np.random.default_rng(20261204)
    directory = str(tmp_path)
    keys = [rows(rng, 37) for _ in range(LAYERS)]
    values = [rows(rng, 37) for _ in range(LAYERS)]
    with RegionStore(QH, KVH, D, LAYERS, directory) as store:
        for layer in range(LAYERS):
            # a 21-token prompt batch in 16-token pages, then single-token steps
            store.append(layer, 0, keys[layer][:21], values[layer][:21], page_tokens=16)
            for t in range(21, 37):
                store.append(layer, t, keys[layer][t:t + 1], values[layer][t:t + 1])
            assert store.layer_tokens(layer) == 37
        for layer in range(LAYERS):
            assert np.array_equal(store.read(layer, "k", range(37)), keys[layer])
            assert np.array_equal(store.read(layer, "v", range(37)), values[layer])
            pick = [0, 15, 16, 17, 20, 36]  # across page and record boundaries
            assert np.array_equal(store.read(layer, "v", pick), values[layer][pick])
            from mslim_attn import MslimAttnError
            with pytest.raises(MslimAttnError, match="sorted and unique"):
                store.read(layer, "k", [3, 2])
        digest = store.logical_kv_sha256()
        assert digest == oracle.logical_kv_sha256(keys, values, 37, KVH, D * 2)
    # the persisted store reopens with every record verified, same catalogue
    with RegionStore(QH, KVH, D, LAYERS, directory) as again:
        assert [again.layer_tokens(l) for l in range(LAYERS)] == [37] * LAYERS
        assert again.logical_kv_sha256() == digest
        from mslim_attn import MslimAttnError
        with pytest.raises(MslimAttnError, match="exclusive writer"):
            RegionStore(QH, KVH, D, LAYERS, directory)


def test_rejections_match_the_reference_messages():
    from mslim_attn import MslimAttnError
    from mslim_attn.region import RegionStore

    rng = np.random.default_rng(7)
    with RegionStore(QH, KVH, D, 2) as store:
        k, v = rows(rng, 4), rows(rng, 4)
        bad = v.copy()
        bad[2, 5] = 0x7FC0  # NaN
        with pytest.raises(MslimAttnError, match="GPU ColdStore V nonfinite"):
            store.append(1, 0, k, bad, page_tokens=4)
        assert store.layer_tokens(1) == 0  # nothing committed
        store.append(1, 0, k, v, page_tokens=4)
        with pytest.raises(MslimAttnError, match="GPU LOD append needs sequential tokens"):
            store.append(1, 7, k[:1], v[:1])
        with pytest.raises(MslimAttnError, match="layer out of range"):
            store.layer_tokens(2)
    with pytest.raises(MslimAttnError, match="must be"):
        RegionStore(QH, KVH, D, 2, stage_tokens=4096)
