"""mslim_attn_decode_paged_noalloc against mslim_attn_decode_paged.

The allocation-free entry point keeps its split partials in the library's
fixed 16 MiB device array and merges them in a second launch; it must give
the same bits as the allocating entry point with the same split_tokens, on
two calls in a row (the second smaller, so the array holds the first call's
partials when it starts), and refuse a shape whose partials exceed the array.
"""
import numpy as np
import pytest
import torch

import mslim_attn
from _data import from_torch

pytestmark = pytest.mark.gpu


def _pool(lens, qh, kvh, d, page_tokens, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    batch = len(lens)
    pps = max(-(-t // page_tokens) for t in lens)
    needed = [-(-t // page_tokens) for t in lens]
    total = sum(needed)
    perm = np.random.default_rng(seed).permutation(total).astype(np.int32)
    table = np.zeros((batch, pps), np.int32)
    cursor = 0
    for b, n in enumerate(needed):
        table[b, :n] = perm[cursor:cursor + n]
        cursor += n
    k_pool = torch.randn((total, kvh, page_tokens, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v_pool = torch.randn((total, kvh, page_tokens, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn((batch, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    return q, k_pool, v_pool, torch.from_numpy(table).cuda(), pps


def _both(ctx, q, k_pool, v_pool, lens, table, pps, pt, qh, kvh, d, split):
    want = torch.empty_like(q)
    got = torch.empty_like(q)
    ctx.decode_paged(q, k_pool, v_pool, want, lens, table, pps, pt, qh, kvh, d, split_tokens=split)
    ctx.decode_paged_noalloc(q, k_pool, v_pool, got, lens, table, pps, pt, qh, kvh, d, split_tokens=split)
    torch.cuda.synchronize()
    return from_torch(got), from_torch(want)


def test_noalloc_decode_equals_decode_paged_two_calls(ctx):
    print("noalloc: cfg3-shaped call then a smaller call", flush=True)
    qh, kvh, d, pt = 32, 8, 128, 16
    # call 1: BASELINE cfg3 shape (32 sessions, lengths U[512, 8192]), automatic split
    lens1 = [int(x) for x in np.random.default_rng(3).integers(512, 8193, size=32)]
    q, kp, vp, table, pps = _pool(lens1, qh, kvh, d, pt, seed=11)
    got, want = _both(ctx, q, kp, vp, lens1, table, pps, pt, qh, kvh, d, 0)
    assert np.array_equal(got, want)
    # call 2: smaller, more splits per token, right after call 1
    lens2 = [300, 1, 77, 1024]
    q, kp, vp, table, pps = _pool(lens2, 16, 4, d, pt, seed=12)
    got2, want2 = _both(ctx, q, kp, vp, lens2, table, pps, pt, 16, 4, d, 64)
    assert np.array_equal(got2, want2)
    # both calls again in the other order of sizes: the array holds call 2's partials
    q, kp, vp, table, pps = _pool(lens1, qh, kvh, d, pt, seed=13)
    got3, want3 = _both(ctx, q, kp, vp, lens1, table, pps, pt, qh, kvh, d, 512)
    assert np.array_equal(got3, want3)


def test_noalloc_decode_on_a_fresh_context_allocates_nothing(ctx):
    """The first call on a new context leaves the device's free memory
    unchanged (no hipMalloc, no context buffer grown), then matches the
    allocating entry point, which grows the context's workspace."""
    qh, kvh, d, pt = 32, 8, 128, 16
    lens = [int(x) for x in np.random.default_rng(5).integers(512, 8193, size=32)]
    q, kp, vp, table, pps = _pool(lens, qh, kvh, d, pt, seed=21)
    got, want = torch.empty_like(q), torch.empty_like(q)
    torch.cuda.synchronize()
    fresh = mslim_attn.Context()
    fresh.use_torch_stream()
    try:
        before, _ = torch.cuda.mem_get_info()
        fresh.decode_paged_noalloc(q, kp, vp, got, lens, table, pps, pt, qh, kvh, d)
        torch.cuda.synchronize()
        after, _ = torch.cuda.mem_get_info()
        assert after == before, (before, after)
        fresh.decode_paged(q, kp, vp, want, lens, table, pps, pt, qh, kvh, d)
        torch.cuda.synchronize()
        assert np.array_equal(from_torch(got), from_torch(want))
    finally:
        fresh.close()


def test_noalloc_decode_rejects_partials_above_the_fixed_array(ctx):
    # 64 sequences x 32,768 tokens at 64-token splits: 32,768 partitions x
    # 8 kv heads x 8 heads x 130 floats = 1.09 GB of partials > 16 MiB.  The
    # host check refuses it before any launch.
    qh, kvh, d, pt = 64, 8, 128, 16
    lens = [32768] * 64
    pps = 32768 // pt
    q = torch.zeros((64, qh, d), dtype=torch.int16, device="cuda")
    out = torch.empty_like(q)
    pool = torch.zeros((1, kvh, pt, d), dtype=torch.int16, device="cuda")
    table = torch.zeros((64, pps), dtype=torch.int32, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="16777216-byte scratch"):
        ctx.decode_paged_noalloc(q, pool, pool, out, lens, table, pps, pt, qh, kvh, d, split_tokens=64)


def test_noalloc_decode_rejects_more_sequences_than_the_kernel_arguments_hold(ctx):
    # Above 64 sequences the launch tables need a device copy, which the
    # allocation-free entry point does not make; the host check refuses it.
    qh, kvh, d, pt = 8, 8, 128, 16
    q, k_pool, v_pool, table, pps = _pool([16] * 65, qh, kvh, d, pt, seed=65)
    out = torch.empty_like(q)
    with pytest.raises(mslim_attn.MslimAttnError, match="at most 64 sequences"):
        ctx.decode_paged_noalloc(q, k_pool, v_pool, out, [16] * 65, table, pps, pt, qh, kvh, d, split_tokens=64)
