"""GPU parity of the ColdStore record frames (csrc/coldstore.hip).

Every record assembled from a device frame and its pool payloads must equal,
byte for byte, the oracle's restatement of ColdStore::prepare_page
(cold_store.rs:269-349), which is pinned by the reference's committed_bytes
known answer, FNV-1a and FIPS 180-4 vectors and the committed fixtures.
"""
import numpy as np
import pytest
import torch

import mslim_attn
import oracle

pytestmark = pytest.mark.gpu

HDR, FTR = mslim_attn.RECORD_HEADER_BYTES, mslim_attn.RECORD_FOOTER_BYTES


def make_pool(rng, pool_pages, kv_heads, page_tokens, head_dim):
    shape = (pool_pages, kv_heads, page_tokens, head_dim)
    k = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
    v = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
    return k, v


def device(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).to("cuda")


def records_array(descs):
    arr = (mslim_attn.PageRecord * max(1, len(descs)))()
    for i, (page_id, token_start, layer, tokens, pool_page) in enumerate(descs):
        arr[i] = mslim_attn.PageRecord(page_id, token_start, layer, tokens, pool_page, 0)
    raw = np.frombuffer(bytes(arr), np.uint8)[: 32 * len(descs)]
    return device(raw) if len(descs) else torch.zeros(32, dtype=torch.uint8, device="cuda")


def run_frames(ctx, k, v, page_tokens, tile, descs):
    pool_pages, kv_heads, _, head_dim = k.shape
    slot = mslim_attn.Context.record_frame_bytes(page_tokens)
    frames = torch.full((max(1, len(descs)) * slot,), 0xAB, dtype=torch.uint8, device="cuda")
    ctx.record_frames(device(k), device(v), pool_pages, page_tokens, kv_heads, head_dim, tile,
                      records_array(descs), len(descs), frames)
    torch.cuda.synchronize()
    return frames.cpu().numpy(), slot


def file_bytes(frame: np.ndarray, k, v, pool_page, tokens):
    """Record bytes as the host writes them: frame prefix | K | V | footer."""
    kp = np.ascontiguousarray(k[pool_page, :, :tokens, :]).view(np.uint8).reshape(-1)
    vp = np.ascontiguousarray(v[pool_page, :, :tokens, :]).view(np.uint8).reshape(-1)
    return bytes(frame[: HDR + 16 * tokens]) + kp.tobytes() + vp.tobytes() + bytes(frame[-FTR:])


def oracle_record(k, v, page_id, token_start, layer, tokens, pool_page, tile):
    kv_heads, head_dim = k.shape[1], k.shape[3]
    kp = np.ascontiguousarray(k[pool_page, :, :tokens, :]).view(np.uint8).tobytes()
    vp = np.ascontiguousarray(v[pool_page, :, :tokens, :]).view(np.uint8).tobytes()
    return oracle.coldstore_record(page_id, layer, token_start, tokens, kv_heads, head_dim, tile, kp, vp)


def test_frame_slot_size():
    assert mslim_attn.Context.record_frame_bytes(16) == 104 + 16 * 16 + 56
    assert mslim_attn.Context.record_frame_bytes(1) == 176


@pytest.mark.parametrize("kv_heads,head_dim,page_tokens", [
    (8, 128, 16),   # the pool geometry of the attention path
    (8, 128, 64),   # prefill seal pages (prefill.rs:22)
    (2, 8, 1),      # single-token decode pages (gpu_region_store.rs:376-384)
    (4, 64, 32),
    (3, 80, 16),
])
def test_frames_equal_oracle_records(ctx, kv_heads, head_dim, page_tokens):
    rng = np.random.default_rng(kv_heads * 1000 + head_dim + page_tokens)
    pool_pages = 11
    k, v = make_pool(rng, pool_pages, kv_heads, page_tokens, head_dim)
    tile = 16 if head_dim % 16 == 0 else 1
    descs = []
    for i in range(9):
        tokens = page_tokens if i % 3 else int(rng.integers(1, page_tokens + 1))
        descs.append((int(rng.integers(0, 1 << 40)), int(rng.integers(0, 1 << 33)), int(rng.integers(0, 80)),
                      tokens, int(rng.integers(0, pool_pages))))
    frames, slot = run_frames(ctx, k, v, page_tokens, tile, descs)
    for i, (page_id, token_start, layer, tokens, pool_page) in enumerate(descs):
        frame = frames[i * slot:(i + 1) * slot]
        got = file_bytes(frame, k, v, pool_page, tokens)
        want = oracle_record(k, v, page_id, token_start, layer, tokens, pool_page, tile)
        assert got == want, f"record {i} (tokens {tokens}) differs"
        assert not frame[HDR + 16 * tokens: slot - FTR].any(), "padding between tables and footer"


def test_invalid_descriptors_get_zero_slots(ctx):
    rng = np.random.default_rng(5)
    k, v = make_pool(rng, 4, 8, 16, 128)
    descs = [(0, 0, 0, 16, 1), (1, 16, 0, 0, 1), (2, 32, 0, 17, 1), (3, 48, 0, 16, 4),
             (4, 64, 0, 16, -1), (5, 80, 0, 5, 3)]
    frames, slot = run_frames(ctx, k, v, 16, 16, descs)
    for i in (1, 2, 3, 4):
        assert not frames[i * slot:(i + 1) * slot].any()
    for i in (0, 5):
        page_id, token_start, layer, tokens, pool_page = descs[i]
        got = file_bytes(frames[i * slot:(i + 1) * slot], k, v, pool_page, tokens)
        assert got == oracle_record(k, v, page_id, token_start, layer, tokens, pool_page, 16)


def test_zero_records_is_a_no_op(ctx):
    rng = np.random.default_rng(6)
    k, v = make_pool(rng, 2, 8, 16, 128)
    frames, _ = run_frames(ctx, k, v, 16, 16, [])
    assert (frames == 0xAB).all()


def test_rejects_bad_arguments(ctx):
    kp = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    rec = records_array([(0, 0, 0, 1, 0)])
    out = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="tile"):
        ctx.record_frames(kp, kp, 1, 1, 2, 8, 3, rec, 1, out)
    with pytest.raises(mslim_attn.MslimAttnError, match="power of two"):
        ctx.record_frames(kp, kp, 1, 3, 2, 8, 8, rec, 1, out)
    with pytest.raises(mslim_attn.MslimAttnError, match="multiple of 8"):
        ctx.record_frames(kp, kp, 1, 1, 2, 4, 4, rec, 1, out)


def test_cfg4_layer_seal_properties(ctx):
    """cfg4 scale: 4 x 32,768 tokens = 8,192 pool pages of 16 tokens, every
    record framed in one call.  Size-independent checks on all of them (magic,
    lengths, token-hash table checksum fields), full byte parity on a sample."""
    kv_heads, head_dim, page_tokens, pool_pages = 8, 128, 16, 8192
    g = torch.Generator(device="cuda").manual_seed(44)
    k_pool = torch.randint(-32768, 32767, (pool_pages * kv_heads * page_tokens * head_dim,),
                           generator=g, device="cuda", dtype=torch.int16)
    v_pool = torch.randint(-32768, 32767, k_pool.shape, generator=g, device="cuda", dtype=torch.int16)
    perm = np.random.default_rng(7).permutation(pool_pages)
    descs = [(i, (i % 2048) * 16, 0, 16, int(perm[i])) for i in range(pool_pages)]
    slot = mslim_attn.Context.record_frame_bytes(page_tokens)
    frames = torch.empty((pool_pages * slot,), dtype=torch.uint8, device="cuda")
    ctx.record_frames(k_pool, v_pool, pool_pages, page_tokens, kv_heads, head_dim, 16,
                      records_array(descs), len(descs), frames)
    torch.cuda.synchronize()
    f = frames.cpu().numpy().reshape(pool_pages, slot)
    payload = kv_heads * 16 * head_dim * 2
    assert (f[:, :8] == np.frombuffer(b"TSKVPG04", np.uint8)).all()
    assert (f[:, -FTR:-FTR + 8] == np.frombuffer(b"TSKVCMIT", np.uint8)).all()
    rec_len = f[:, -FTR + 16:-FTR + 24].copy().view(np.uint64).reshape(-1)
    assert (rec_len == HDR + 16 * 16 + 2 * payload + FTR).all()
    page_ids = f[:, 16:24].copy().view(np.uint64).reshape(-1)
    assert (page_ids == np.arange(pool_pages)).all()
    k_host = k_pool.view(torch.int16).cpu().numpy().view(np.uint16).reshape(pool_pages, kv_heads, 16, head_dim)
    v_host = v_pool.view(torch.int16).cpu().numpy().view(np.uint16).reshape(pool_pages, kv_heads, 16, head_dim)
    for i in np.random.default_rng(8).choice(pool_pages, 6, replace=False):
        page_id, token_start, layer, tokens, pool_page = descs[i]
        got = file_bytes(f[i], k_host, v_host, pool_page, tokens)
        assert got == oracle_record(k_host, v_host, page_id, token_start, layer, tokens, pool_page, 16)
