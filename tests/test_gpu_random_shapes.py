"""Seeded randomized parity sweep of decode and prefill over geometries,
ragged lengths, page sizes and splits that the fixed-shape tests do not name.

Every case is drawn from a PCG64 stream seeded by its index, so a failure
names a reproducible case.  The bar is the fixed-shape tests': max abs
<= 2e-2 against the CPU reference attention (dense_attention_bf16 for decode,
native_cpu_adapter.rs:253-307; prefill_causal_cpu for causal chunks), paged
decode equal to dense decode bit for bit, both decode merge modes equal bit
for bit, and a split prefill equal to itself on a repeat.
"""
import numpy as np
import pytest
import torch

import mslim_attn
import oracle
from _data import check_bf16, from_torch, normal_bf16, to_torch

pytestmark = pytest.mark.gpu

TOL = 2e-2

# head_dim: any multiple of 8 up to 256 is accepted by the C ABI.  Half of
# the draws take the MFMA kernels' geometries (head_dim 64 or 128, a group of
# 1, 2, 4, 8 or 16 query heads per kv head), the others any geometry, which
# mostly lands on the generic kernels.
HEAD_DIMS = (40, 64, 72, 80, 96, 128, 136, 192, 256)
GROUPS = (1, 2, 3, 4, 5, 8, 16)
FAST_DIMS = (64, 128)
FAST_GROUPS = (1, 2, 4, 8, 16)


def _geometry(rng, max_kv_heads):
    fast = rng.random() < 0.5
    d = int(rng.choice(FAST_DIMS if fast else HEAD_DIMS))
    g = int(rng.choice(FAST_GROUPS if fast else GROUPS))
    kvh = int(rng.integers(1, max_kv_heads + 1))
    return g * kvh, kvh, d
DECODE_CASES = 24
PREFILL_CASES = 16


def _decode_case(seed):
    rng = np.random.default_rng(1000 + seed)
    qh, kvh, d = _geometry(rng, 8)
    batch = int(rng.integers(1, 7))
    # ragged: a mix of tiny, page-boundary and long histories
    pool = [1, 2, 15, 16, 17, 63, 64, 65, 255, 256, 257]
    lens = [int(rng.choice(pool)) if rng.random() < 0.4 else int(rng.integers(1, 3001))
            for _ in range(batch)]
    page = int(rng.choice((16, 32, 64)))
    split = int(rng.choice((0, 64, 128, 256, 1024)))
    return rng, qh, kvh, d, lens, page, split


@pytest.mark.parametrize("seed", range(DECODE_CASES))
def test_random_decode_dense_paged_and_merge_modes(ctx, seed):
    rng, qh, kvh, d, lens, page, split = _decode_case(seed)
    case = dict(seed=seed, qh=qh, kvh=kvh, d=d, lens=lens, page=page, split=split)
    print("case", case, flush=True)
    b = len(lens)
    stride = max(lens)
    qb = normal_bf16(rng, (b, qh, d))
    kb = normal_bf16(rng, (b, stride, kvh, d))
    vb = normal_bf16(rng, (b, stride, kvh, d))
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)

    outs = []
    try:
        for separate in (False, True):
            ctx.set_decode_merge(separate)
            out = torch.empty_like(q)
            ctx.decode_dense(q, k, v, out, lens, qh, kvh, d, seq_stride_tokens=stride,
                             split_tokens=split)
            torch.cuda.synchronize()
            outs.append(from_torch(out))
    finally:
        ctx.set_decode_merge(False)
    dense, separate_merge = outs
    assert np.array_equal(dense, separate_merge), case
    dense = dense.reshape(b, -1)
    for i, t in enumerate(lens):
        ref = oracle.dense_attention_bf16(oracle.read_bf16(qb[i]), kb[i, :t], vb[i, :t], qh, kvh, d)
        check_bf16(dense[i], ref, TOL, "test_random_decode_dense_paged_and_merge_modes")

    # scatter into a seeded random page pool with the product's page writer
    needed = [(t + page - 1) // page for t in lens]
    pps = max(needed)
    perm = rng.permutation(sum(needed)).astype(np.int32)
    table = np.zeros((b, pps), np.int32)
    cursor = 0
    for i, n in enumerate(needed):
        table[i, :n] = perm[cursor:cursor + n]
        cursor += n
    table_t = torch.from_numpy(table).cuda()
    k_pool = torch.zeros((sum(needed), kvh, page, d), dtype=torch.int16, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    for i, t in enumerate(lens):
        ctx.pages_write(k_pool, v_pool, table_t[i], page, kvh, d, 0, t,
                        k[i, :t].contiguous(), v[i, :t].contiguous())
    paged = torch.empty_like(q)
    ctx.decode_paged(q, k_pool, v_pool, paged, lens, table_t, pps, page, qh, kvh, d,
                     split_tokens=split)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(paged).reshape(b, -1), dense), case


def _prefill_case(seed):
    rng = np.random.default_rng(2000 + seed)
    qh, kvh, d = _geometry(rng, 4)
    queries = int(rng.choice((1, 2, 7, 63, 64, 65, 127, 128, 129))) if rng.random() < 0.4 \
        else int(rng.integers(1, 400))
    prior = 0 if rng.random() < 0.3 else int(rng.integers(0, 1500))
    return rng, qh, kvh, d, queries, prior


@pytest.mark.parametrize("seed", range(PREFILL_CASES))
def test_random_prefill_against_oracle(ctx, seed):
    rng, qh, kvh, d, queries, prior = _prefill_case(seed)
    split_tiles = mslim_attn.prefill_split_tiles(queries, prior, qh, kvh, d)
    case = dict(seed=seed, qh=qh, kvh=kvh, d=d, queries=queries, prior=prior, split_tiles=split_tiles)
    print("case", case, flush=True)
    hist = prior + queries
    qb = normal_bf16(rng, (queries, qh, d))
    kb = normal_bf16(rng, (hist, kvh, d))
    vb = normal_bf16(rng, (hist, kvh, d))
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)
    out = torch.empty_like(q)
    again = torch.empty_like(q)
    ctx.prefill_causal(q, k, v, out, queries, prior, qh, kvh, d)
    ctx.prefill_causal(q, k, v, again, queries, prior, qh, kvh, d)
    torch.cuda.synchronize()
    assert torch.equal(out, again), case
    ref = oracle.prefill_causal_cpu(oracle.read_bf16(qb), kb, vb, qh, kvh, d, queries, prior)
    check_bf16(from_torch(out), ref, TOL, "test_random_prefill_against_oracle")
    if split_tiles:
        whole = torch.empty_like(q)
        try:
            ctx.set_prefill_split(False)
            ctx.prefill_causal(q, k, v, whole, queries, prior, qh, kvh, d)
        finally:
            ctx.set_prefill_split(True)
        torch.cuda.synchronize()
        check_bf16(from_torch(whole), ref, TOL, "test_random_prefill_against_oracle (unsplit)")


def test_random_sweep_reaches_both_prefill_launch_forms():
    # The sweep is only as wide as its draws: at least one case each of the
    # split and the whole-chunk prefill launch, and of every decode page size.
    split = []
    for s in range(PREFILL_CASES):
        _, qh, kvh, d, queries, prior = _prefill_case(s)
        split.append(mslim_attn.prefill_split_tiles(queries, prior, qh, kvh, d) > 0)
    assert any(split) and not all(split)
    assert {_decode_case(s)[5] for s in range(DECODE_CASES)} == {16, 32, 64}
