"""GPU parity of single-token decode (dense and ColdStore-paged) against the
CPU oracle, through the C ABI.

Tolerance (north star): max abs <= 2e-2 on BF16 outputs against the
reference CPU attention (`dense_attention_bf16`, native_cpu_adapter.rs:253-307)
and against the f64 CpuReferenceBackend (portable.rs:575-646).  The paged
path must equal the dense path bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from _data import check_bf16, from_torch, normal_bf16, tiled_input, to_torch

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _decode(ctx, qb, kb, vb, lens, qh, kvh, d, split=0, stride=0):
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)
    out = torch.empty_like(q)
    ctx.decode_dense(q, k, v, out, lens, qh, kvh, d, seq_stride_tokens=stride, split_tokens=split)
    torch.cuda.synchronize()
    return from_torch(out)


def _oracle_decode(qb, kb, vb, qh, kvh, d):
    return oracle.dense_attention_bf16(oracle.read_bf16(qb), kb, vb, qh, kvh, d)


def test_decode_cfg1_parity_repeatability_and_inputs_untouched(ctx):
    # B=1, T=1024, 32/8/128, N(0,1) seeded -> BF16.
    rng = np.random.default_rng(20261201)
    qh, kvh, d, t = 32, 8, 128, 1024
    qb = normal_bf16(rng, (1, qh, d))
    kb = normal_bf16(rng, (t, kvh, d))
    vb = normal_bf16(rng, (t, kvh, d))
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)
    out = torch.empty_like(q)
    ctx.decode_dense(q, k, v, out, [t], qh, kvh, d)
    torch.cuda.synchronize()
    got = from_torch(out)
    ref = _oracle_decode(qb, kb, vb, qh, kvh, d)
    check_bf16(got, ref, TOL, "test_decode_cfg1_parity_repeatability_and_inputs_untouched")
    rc, f64 = oracle.cpu_reference_decode(oracle.read_bf16(qb), kb, vb, 1, qh, kvh, d)
    assert rc == 0
    check_bf16(got, f64, TOL, "decode cfg1 vs f64 CpuReferenceBackend")
    # repeat: bit-identical (tiled_attention.rs:380-387); K/V unmodified (:388-397)
    out2 = torch.empty_like(q)
    ctx.decode_dense(q, k, v, out2, [t], qh, kvh, d)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(out2), got)
    assert np.array_equal(from_torch(k), kb) and np.array_equal(from_torch(v), vb)


# The reference's tiled-attention geometries (tiled_attention.rs:412-419:
# (64, 4/4), (128, 8/2), (128, 4/1), (80, 4/2), (256, 4/1)) and the shapes of
# the BASELINE configs.
GEOMS = [(32, 8, 128), (64, 8, 128), (8, 8, 128), (16, 8, 128), (8, 2, 64), (32, 4, 64),
         (4, 2, 80), (4, 1, 256), (12, 4, 128), (4, 4, 64), (8, 2, 128), (4, 1, 128)]
# tiled_attention.rs:430 histories and the fused-vs-three-kernel lengths of
# gpu_llm/mod.rs:4311-4415.
HISTORIES = [1, 2, 15, 31, 32, 33, 63, 65, 127, 129, 375, 512, 1024, 2048, 2049, 4097]
# tiled_attention.rs:374-378: an online (flash) kernel against the reference
# GPU three-kernel arithmetic on these synthetic vectors.
ONLINE_TOL = 0.0078125


@pytest.mark.parametrize("qh,kvh,d", GEOMS)
def test_decode_histories_and_geometries(ctx, qh, kvh, d):
    # The reference's deterministic synthetic inputs (tiled_attention.rs:305-312).
    for t in HISTORIES:
        qb = tiled_input(qh * d, 3).reshape(1, qh, d)
        kb = tiled_input(t * kvh * d, 7).reshape(t, kvh, d)
        vb = tiled_input(t * kvh * d, 11).reshape(t, kvh, d)
        ref = _oracle_decode(qb, kb, vb, qh, kvh, d)
        gpu_ref = oracle.gpu_reference_attention(qb, kb, vb, qh, kvh, d, 1, t - 1)
        for split in (0, 64):
            got = _decode(ctx, qb, kb, vb, [t], qh, kvh, d, split=split)
            check_bf16(got, ref, TOL, "test_decode_histories_and_geometries")
            check_bf16(got, oracle.read_bf16(gpu_ref), ONLINE_TOL, "decode vs reference GPU arithmetic")


def test_decode_ragged_batch_dense(ctx):
    rng = np.random.default_rng(7)
    qh, kvh, d, stride = 32, 8, 128, 1100
    lens = [1, 100, 1000, 64, 513, 1100, 2]
    qb = normal_bf16(rng, (len(lens), qh, d))
    kb = normal_bf16(rng, (len(lens), stride, kvh, d))
    vb = normal_bf16(rng, (len(lens), stride, kvh, d))
    got = _decode(ctx, qb, kb, vb, lens, qh, kvh, d, stride=stride).reshape(len(lens), -1)
    for b, t in enumerate(lens):
        ref = _oracle_decode(qb[b], kb[b, :t], vb[b, :t], qh, kvh, d)
        check_bf16(got[b], ref, TOL, "test_decode_ragged_batch_dense")


def test_decode_ragged_partition_order(ctx):
    # The kernel launches every sequence's full partitions first and the last
    # partitions after them, longest first; partials are stored by logical
    # partition index.  Sequences of one partition, of a 1-token last
    # partition and of many partitions, in an order unrelated to their
    # lengths: dense against the oracle, paged == dense bit for bit, for a
    # fixed split and the automatic one.
    rng = np.random.default_rng(11)
    qh, kvh, d, stride = 32, 8, 128, 5000
    lens = [1, 256, 257, 5000, 100, 3000, 511, 2048, 4097]
    qb = normal_bf16(rng, (len(lens), qh, d))
    kb = normal_bf16(rng, (len(lens), stride, kvh, d))
    vb = normal_bf16(rng, (len(lens), stride, kvh, d))
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)
    k_pool, v_pool, table_t, pps, _ = _paged_pool(ctx, k, v, lens, stride, 16, seed=5)
    for split in (256, 0):
        got = _decode(ctx, qb, kb, vb, lens, qh, kvh, d, split=split, stride=stride).reshape(len(lens), -1)
        for b, t in enumerate(lens):
            ref = _oracle_decode(qb[b], kb[b, :t], vb[b, :t], qh, kvh, d)
            check_bf16(got[b], ref, TOL, "test_decode_ragged_partition_order")
        paged = torch.empty_like(q)
        ctx.decode_paged(q, k_pool, v_pool, paged, lens, table_t, pps, 16, qh, kvh, d, split_tokens=split)
        torch.cuda.synchronize()
        assert np.array_equal(from_torch(paged).reshape(len(lens), -1), got), split


def _paged_pool(ctx, k, v, lens, stride, page_tokens, seed):
    """Scatter dense [B][stride][KVH][D] K/V into a randomly permuted page pool
    with the product's page writer; returns (k_pool, v_pool, table, pages_per_seq)."""
    b_count = len(lens)
    kvh, d = k.shape[2], k.shape[3]
    pages_per_seq = (max(lens) + page_tokens - 1) // page_tokens
    needed = [(t + page_tokens - 1) // page_tokens for t in lens]
    total = sum(needed)
    perm = np.random.default_rng(seed).permutation(total).astype(np.int32)
    table = np.zeros((b_count, pages_per_seq), np.int32)
    cursor = 0
    for b, n in enumerate(needed):
        table[b, :n] = perm[cursor:cursor + n]
        cursor += n
    table_t = torch.from_numpy(table).cuda()
    k_pool = torch.zeros((total, kvh, page_tokens, d), dtype=torch.int16, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    for b, t in enumerate(lens):
        ctx.pages_write(k_pool, v_pool, table_t[b], page_tokens, kvh, d, 0, t,
                        k[b, :t].contiguous(), v[b, :t].contiguous())
    torch.cuda.synchronize()
    return k_pool, v_pool, table_t, pages_per_seq, table


def test_paged_equals_dense_bitwise_cfg3(ctx):
    # 32 sessions, T ~ U[512, 8192] seeded, 16-token pages,
    # seeded random page table, epsilon = 0, 32/8/128.
    rng = np.random.default_rng(3)
    qh, kvh, d, pt = 32, 8, 128, 16
    lens = [int(x) for x in rng.integers(512, 8193, size=32)]
    stride = max(lens)
    gen = torch.Generator(device="cuda").manual_seed(1234)
    k = torch.randn((32, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((32, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn((32, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k_pool, v_pool, table_t, pps, table = _paged_pool(ctx, k, v, lens, stride, pt, seed=99)
    for split in (0, 64, 512):
        dense = torch.empty_like(q)
        paged = torch.empty_like(q)
        ctx.decode_dense(q, k, v, dense, lens, qh, kvh, d, seq_stride_tokens=stride, split_tokens=split)
        ctx.decode_paged(q, k_pool, v_pool, paged, lens, table_t, pps, pt, qh, kvh, d, split_tokens=split)
        torch.cuda.synchronize()
        assert torch.equal(dense, paged), split
    # parity of a few sessions against the CPU oracle
    dn = from_torch(dense).reshape(32, -1)
    for b in (0, int(np.argmax(lens)), int(np.argmin(lens)), 17):
        t = lens[b]
        kb = from_torch(k[b, :t])
        vb = from_torch(v[b, :t])
        qb = from_torch(q[b])
        check_bf16(dn[b], _oracle_decode(qb, kb, vb, qh, kvh, d), TOL, "test_paged_equals_dense_bitwise_cfg3")
    # the pool holds the dense bytes exactly: gather each session back
    for b in (0, 5, 31):
        t = lens[b]
        rows = torch.empty((t, kvh, d), dtype=torch.int16, device="cuda")
        ctx.pages_gather(k_pool, table_t[b], pt, kvh, d, 0, t, rows)
        torch.cuda.synchronize()
        assert torch.equal(rows, k[b, :t])


def test_paged_parity_small_pages_and_tails(ctx):
    rng = np.random.default_rng(21)
    qh, kvh, d = 16, 4, 128
    lens = [1, 15, 16, 17, 33, 300, 1023]
    stride = 1024
    for pt in (16, 32, 64):
        kb = normal_bf16(rng, (len(lens), stride, kvh, d))
        vb = normal_bf16(rng, (len(lens), stride, kvh, d))
        qb = normal_bf16(rng, (len(lens), qh, d))
        k, v, q = to_torch(kb), to_torch(vb), to_torch(qb)
        k_pool, v_pool, table_t, pps, _ = _paged_pool(ctx, k, v, lens, stride, pt, seed=pt)
        paged = torch.empty_like(q)
        dense = torch.empty_like(q)
        ctx.decode_paged(q, k_pool, v_pool, paged, lens, table_t, pps, pt, qh, kvh, d, split_tokens=64)
        ctx.decode_dense(q, k, v, dense, lens, qh, kvh, d, seq_stride_tokens=stride, split_tokens=64)
        torch.cuda.synchronize()
        assert torch.equal(paged, dense), pt
        got = from_torch(paged).reshape(len(lens), -1)
        for b, t in enumerate(lens):
            ref = _oracle_decode(qb[b], kb[b, :t], vb[b, :t], qh, kvh, d)
            check_bf16(got[b], ref, TOL, "test_paged_parity_small_pages_and_tails")


def test_decode_cfg4_shape_parity(ctx):
    # BASELINE config 4 decode shape: B=4, T=32768, 64/8/128.  Two sequences
    # are checked in full against the CPU oracle.
    qh, kvh, d, t, batch = 64, 8, 128, 32768, 4
    gen = torch.Generator(device="cuda").manual_seed(4)
    k = torch.randn((batch, t, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((batch, t, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn((batch, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty_like(q)
    ctx.decode_dense(q, k, v, out, [t] * batch, qh, kvh, d, seq_stride_tokens=t)
    torch.cuda.synchronize()
    got = from_torch(out).reshape(batch, -1)
    for b in (0, 3):
        ref = _oracle_decode(from_torch(q[b]), from_torch(k[b]), from_torch(v[b]), qh, kvh, d)
        check_bf16(got[b], ref, TOL, "test_decode_cfg4_shape_parity")


def test_extreme_scores_are_stable(ctx):
    # portable.rs:712-726 analogue: one dominant key -> its V exactly.
    qh, kvh, d, t = 8, 8, 128, 70
    qb = oracle.write_bf16(np.full((1, qh, d), 8.0, np.float32))
    k = np.zeros((t, kvh, d), np.float32)
    k[37] = 8.0
    k[5] = -8.0
    v = np.tile(np.arange(t, dtype=np.float32)[:, None, None], (1, kvh, d))
    got = oracle.read_bf16(_decode(ctx, qb, oracle.write_bf16(k), oracle.write_bf16(v), [t], qh, kvh, d))
    assert np.all(got == 37.0)


def test_decode_rejects_bad_arguments(ctx):
    import mslim_attn
    q = torch.zeros((1, 8, 128), dtype=torch.int16, device="cuda")
    k = torch.zeros((64, 8, 128), dtype=torch.int16, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="alias"):
        ctx.decode_dense(q, k, k, q, [64], 8, 8, 128)
    out = torch.empty_like(q)
    for kwargs, msg in [(dict(split_tokens=65), "split_tokens"), (dict(split_tokens=-64), "split_tokens")]:
        with pytest.raises(mslim_attn.MslimAttnError, match=msg):
            ctx.decode_dense(q, k, k, out, [64], 8, 8, 128, **kwargs)
    with pytest.raises(mslim_attn.MslimAttnError, match="seq_lens"):
        ctx.decode_dense(q, k, k, out, [0], 8, 8, 128)
    with pytest.raises(mslim_attn.MslimAttnError, match="1..4096"):
        ctx.decode_dense(q, k, k, out, [1] * 4097, 8, 8, 128, seq_stride_tokens=64)
    with pytest.raises(mslim_attn.MslimAttnError, match="geometry"):
        ctx.decode_dense(q, k, k, out, [64], 8, 3, 128)
    table = torch.zeros((1, 4), dtype=torch.int32, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="page_tokens"):
        ctx.decode_paged(q, k, k, out, [64], table, 4, 24, 8, 8, 128)
    with pytest.raises(mslim_attn.MslimAttnError, match="shorter"):
        ctx.decode_paged(q, k, k, out, [65], table, 4, 16, 8, 8, 128)


def _merge_modes(ctx, fn):
    """fn() under the fused last-workgroup merge and under the separate merge
    launch; returns both outputs (host bits) and restores the default."""
    outs = []
    try:
        for separate in (False, True):
            ctx.set_decode_merge(separate)
            outs.append(fn())
    finally:
        ctx.set_decode_merge(False)
    return outs


def test_decode_merge_modes_bitwise_ragged(ctx):
    # The fused merge (the last workgroup of each (sequence, kv head) to
    # count its split merges, partials published by agent-scope stores that
    # complete before the counter atomic) and the two-launch merge read the
    # same partials in the same fixed order.
    rng = np.random.default_rng(31)
    qh, kvh, d, stride = 32, 8, 128, 6000
    lens = [1, 300, 6000, 257, 4096, 1023, 2, 5555]
    qb = normal_bf16(rng, (len(lens), qh, d))
    kb = normal_bf16(rng, (len(lens), stride, kvh, d))
    vb = normal_bf16(rng, (len(lens), stride, kvh, d))
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)
    k_pool, v_pool, table_t, pps, _ = _paged_pool(ctx, k, v, lens, stride, 16, seed=8)
    for split in (64, 256, 0):
        def dense():
            out = torch.empty_like(q)
            ctx.decode_dense(q, k, v, out, lens, qh, kvh, d, seq_stride_tokens=stride, split_tokens=split)
            torch.cuda.synchronize()
            return from_torch(out)

        def paged():
            out = torch.empty_like(q)
            ctx.decode_paged(q, k_pool, v_pool, out, lens, table_t, pps, 16, qh, kvh, d, split_tokens=split)
            torch.cuda.synchronize()
            return from_torch(out)

        fused_d, separate_d = _merge_modes(ctx, dense)
        fused_p, separate_p = _merge_modes(ctx, paged)
        assert np.array_equal(fused_d, separate_d), split
        assert np.array_equal(fused_p, separate_p), split
        assert np.array_equal(fused_d, fused_p), split
        got = fused_d.reshape(len(lens), -1)
        for b in (0, 2, 7):
            t = lens[b]
            check_bf16(got[b], _oracle_decode(qb[b], kb[b, :t], vb[b, :t], qh, kvh, d), TOL, "test_decode_merge_modes_bitwise_ragged")


# Launches with more partitions than two per CU (512) and at most 896 run the
# partitions as 512 host-packed lists (fused merge only); the separate merge
# launch keeps one partition per workgroup.  Same partitions, same fixed merge
# order: the bits must agree.  cfg3's batch (640 partitions at the automatic
# split), a D = 64 / group-8 geometry and a batch whose 896 partitions fill
# the lists.
LIST_CASES = [(32, 512, 8193, 20261203, 32, 8, 128, 0), (24, 300, 6001, 5, 16, 2, 64, 0),
              (40, 2000, 6001, 6, 32, 8, 128, 1856)]


@pytest.mark.parametrize("batch,lo,hi,seed,qh,kvh,d,split", LIST_CASES)
def test_decode_list_mode_matches_one_partition_per_workgroup(ctx, batch, lo, hi, seed, qh, kvh, d, split):
    import mslim_attn
    lens = np.random.default_rng(seed).integers(lo, hi, size=batch).tolist()
    s = split or mslim_attn.auto_split(lens, kvh)
    parts = sum(-(-t // s) for t in lens) * kvh
    assert 512 < parts <= 896, parts
    stride = max(lens)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((batch, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k = torch.randn((batch, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((batch, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k_pool, v_pool, table_t, pps, _ = _paged_pool(ctx, k, v, lens, stride, 16, seed=seed)

    def dense():
        out = torch.empty_like(q)
        ctx.decode_dense(q, k, v, out, lens, qh, kvh, d, seq_stride_tokens=stride, split_tokens=split)
        torch.cuda.synchronize()
        return from_torch(out)

    def paged():
        out = torch.empty_like(q)
        ctx.decode_paged(q, k_pool, v_pool, out, lens, table_t, pps, 16, qh, kvh, d, split_tokens=split)
        torch.cuda.synchronize()
        return from_torch(out)

    listed_d, static_d = _merge_modes(ctx, dense)
    listed_p, static_p = _merge_modes(ctx, paged)
    again = paged()
    assert np.array_equal(listed_d, static_d)
    assert np.array_equal(listed_p, static_p)
    assert np.array_equal(listed_d, listed_p)
    assert np.array_equal(listed_p, again)
    got = listed_p.reshape(batch, -1)
    qb = from_torch(q)
    for b in (0, int(np.argmax(lens)), int(np.argmin(lens)), batch - 1):
        t = lens[b]
        kb, vb = from_torch(k[b, :t].contiguous()), from_torch(v[b, :t].contiguous())
        check_bf16(got[b], _oracle_decode(qb[b], kb, vb, qh, kvh, d), TOL, "test_decode_list_mode_matches_one_partition_per_workgroup")


def _cfg4_hot_cold_pool(k, v, lens, hot_window, page_tokens, seed, ctx):
    """cfg4's layout: per sequence the cold pages are a seeded random
    permutation of pool slots and the most recent `hot_window` tokens one
    contiguous run of slots after them."""
    batch, t_max, kvh, d = k.shape
    pages = t_max // page_tokens
    hot = hot_window // page_tokens
    cold = pages - hot
    rng = np.random.default_rng(seed)
    cold_slots = rng.permutation(batch * cold).astype(np.int32)
    table = np.zeros((batch, pages), np.int32)
    for b in range(batch):
        table[b, :cold] = cold_slots[b * cold:(b + 1) * cold]
        table[b, cold:] = batch * cold + b * hot + np.arange(hot, dtype=np.int32)
    table_t = torch.from_numpy(table).cuda()
    k_pool = torch.empty((batch * pages, kvh, page_tokens, d), dtype=torch.int16, device="cuda")
    v_pool = torch.empty_like(k_pool)
    for b in range(batch):
        ctx.pages_write(k_pool, v_pool, table_t[b], page_tokens, kvh, d, 0, lens[b], k[b, :lens[b]].contiguous(),
                        v[b, :lens[b]].contiguous())
    torch.cuda.synchronize()
    return k_pool, v_pool, table_t, pages


def test_decode_cfg4_hot_window_cold_pages_against_oracle(ctx):
    # BASELINE config 4 as configured: B=4, T=32,768, 64/8/128, a 4,096-token
    # contiguous hot window plus cold 16-token pages in a seeded random
    # permutation.  paged == dense bit for bit under both merge modes; two
    # sequences in full against the CPU oracle.
    qh, kvh, d, t, batch = 64, 8, 128, 32768, 4
    gen = torch.Generator(device="cuda").manual_seed(44)
    k = torch.randn((batch, t, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((batch, t, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn((batch, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    lens = [t] * batch
    k_pool, v_pool, table_t, pps = _cfg4_hot_cold_pool(k, v, lens, 4096, 16, 20261201, ctx)

    def paged():
        out = torch.empty_like(q)
        ctx.decode_paged(q, k_pool, v_pool, out, lens, table_t, pps, 16, qh, kvh, d)
        torch.cuda.synchronize()
        return from_torch(out)

    dense = torch.empty_like(q)
    ctx.decode_dense(q, k, v, dense, lens, qh, kvh, d, seq_stride_tokens=t)
    torch.cuda.synchronize()
    fused, separate = _merge_modes(ctx, paged)
    assert np.array_equal(fused, from_torch(dense))
    assert np.array_equal(fused, separate)
    got = fused.reshape(batch, -1)
    for b in (1, 2):
        ref = _oracle_decode(from_torch(q[b]), from_torch(k[b]), from_torch(v[b]), qh, kvh, d)
        check_bf16(got[b], ref, TOL, "test_decode_cfg4_hot_window_cold_pages_against_oracle")


def test_decode_stream_switch_between_ragged_split_decodes(ctx):
    # One context's split workspace and counters serve one stream at a time:
    # a ragged split decode queued on stream A, then a switch to stream B and
    # a second ragged split decode there.  The switch waits for A, so both
    # outputs equal the same calls made on one stream.
    rng = np.random.default_rng(41)
    qh, kvh, d, stride = 32, 8, 128, 8192
    lens_a = [8192, 700, 5000, 3]
    lens_b = [2048, 8000, 1]
    qa, qb = normal_bf16(rng, (len(lens_a), qh, d)), normal_bf16(rng, (len(lens_b), qh, d))
    ka = to_torch(normal_bf16(rng, (len(lens_a), stride, kvh, d)))
    va = to_torch(normal_bf16(rng, (len(lens_a), stride, kvh, d)))
    kb = ka[:len(lens_b)].flip(0).contiguous()
    vb = va[:len(lens_b)].flip(0).contiguous()
    qa_t, qb_t = to_torch(qa), to_torch(qb)
    want_a, want_b = torch.empty_like(qa_t), torch.empty_like(qb_t)
    ctx.decode_dense(qa_t, ka, va, want_a, lens_a, qh, kvh, d, seq_stride_tokens=stride, split_tokens=256)
    ctx.decode_dense(qb_t, kb, vb, want_b, lens_b, qh, kvh, d, seq_stride_tokens=stride, split_tokens=256)
    torch.cuda.synchronize()
    s_a, s_b = torch.cuda.Stream(), torch.cuda.Stream()
    out_a, out_b = torch.empty_like(qa_t), torch.empty_like(qb_t)
    try:
        ctx.set_stream(s_a.cuda_stream)
        ctx.decode_dense(qa_t, ka, va, out_a, lens_a, qh, kvh, d, seq_stride_tokens=stride, split_tokens=256)
        ctx.set_stream(s_b.cuda_stream)
        ctx.decode_dense(qb_t, kb, vb, out_b, lens_b, qh, kvh, d, seq_stride_tokens=stride, split_tokens=256)
        ctx.synchronize()
    finally:
        ctx.use_torch_stream()
    torch.cuda.synchronize()
    assert torch.equal(out_a, want_a)
    assert torch.equal(out_b, want_b)


def test_decode_option_rejects_unknown_values(ctx):
    import mslim_attn
    with pytest.raises(mslim_attn.MslimAttnError, match="merge mode"):
        ctx.set_option(mslim_attn.OPT_DECODE_MERGE, 2)
    with pytest.raises(mslim_attn.MslimAttnError, match="unknown context option"):
        ctx.set_option(99, 0)


def _chunked(fn, batch, step):
    """fn(lo, hi) for consecutive sequence ranges of at most `step`."""
    for lo in range(0, batch, step):
        fn(lo, min(batch, lo + step))


def test_decode_batches_past_the_kernel_argument_tables(ctx):
    # Launches of more than 64 sequences read their launch tables from a
    # device copy made on the stream before the kernel.  Partitions are fixed
    # by logical token index, so a sequence's output does not depend on the
    # batch it rides in: 300 sequences in one launch equal the same sequences
    # in launches of at most 64, bit for bit, dense and paged, under the fused
    # and the separate merge; 100 single-partition sequences (800 partitions
    # over 8 kv heads) take the list mode with the tables on the device.
    # Six large launches are queued back to back, more than the context's
    # ring of table buffers, before anything is read back.
    gen = torch.Generator(device="cuda").manual_seed(4096)
    rng = np.random.default_rng(4096)
    qh, kvh, d, pt, split = 32, 8, 128, 16, 256
    batch = 300
    lens = [int(x) for x in rng.integers(1, 700, size=batch)]
    lens[:100] = [int(x) for x in rng.integers(1, split + 1, size=100)]
    stride = max(lens)
    k = torch.randn((batch, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((batch, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn((batch, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k_pool, v_pool, table_t, pps, _ = _paged_pool(ctx, k, v, lens, stride, pt, seed=77)

    def dense(lo, hi, out):
        ctx.decode_dense(q[lo:hi], k[lo:hi], v[lo:hi], out[lo:hi], lens[lo:hi], qh, kvh, d,
                         seq_stride_tokens=stride, split_tokens=split)

    def paged(lo, hi, out):
        ctx.decode_paged(q[lo:hi], k_pool, v_pool, out[lo:hi], lens[lo:hi], table_t[lo:hi], pps, pt,
                         qh, kvh, d, split_tokens=split)

    def run():
        outs = [torch.full_like(q, -1) for _ in range(6)]
        dense(0, batch, outs[0])
        paged(0, batch, outs[1])
        dense(0, 100, outs[2])   # list mode, tables on the device
        paged(0, 100, outs[3])
        dense(64, batch, outs[4])
        paged(64, batch, outs[5])
        torch.cuda.synchronize()
        return [from_torch(o).reshape(batch, -1) for o in outs]

    fused, separate = _merge_modes(ctx, run)
    small = [torch.full_like(q, -1) for _ in range(2)]
    _chunked(lambda lo, hi: dense(lo, hi, small[0]), batch, 64)
    _chunked(lambda lo, hi: paged(lo, hi, small[1]), batch, 50)
    torch.cuda.synchronize()
    want = from_torch(small[0]).reshape(batch, -1)
    assert np.array_equal(from_torch(small[1]).reshape(batch, -1), want)
    for outs in (fused, separate):
        assert np.array_equal(outs[0], want) and np.array_equal(outs[1], want)
        assert np.array_equal(outs[2][:100], want[:100]) and np.array_equal(outs[3][:100], want[:100])
        assert np.array_equal(outs[4][64:], want[64:]) and np.array_equal(outs[5][64:], want[64:])
    for b in (0, 99, 100, int(np.argmax(lens)), batch - 1):
        t = lens[b]
        ref = _oracle_decode(from_torch(q[b]), from_torch(k[b, :t]), from_torch(v[b, :t]), qh, kvh, d)
        check_bf16(want[b], ref, TOL, "test_decode_batches_past_the_kernel_argument_tables")
    # the library's own split for the whole batch: paged == dense, and parity
    auto_d, auto_p = torch.empty_like(q), torch.empty_like(q)
    ctx.decode_dense(q, k, v, auto_d, lens, qh, kvh, d, seq_stride_tokens=stride)
    ctx.decode_paged(q, k_pool, v_pool, auto_p, lens, table_t, pps, pt, qh, kvh, d)
    torch.cuda.synchronize()
    assert torch.equal(auto_d, auto_p)
    got = from_torch(auto_d).reshape(batch, -1)
    for b in (3, int(np.argmax(lens))):
        t = lens[b]
        ref = _oracle_decode(from_torch(q[b]), from_torch(k[b, :t]), from_torch(v[b, :t]), qh, kvh, d)
        check_bf16(got[b], ref, TOL, "decode of 300 sequences, automatic split")


def test_decode_at_the_batch_limit(ctx):
    # MSLIM_ATTN_MAX_BATCH (4,096) sequences of 1 to 40 tokens: dense ==
    # paged, both equal to the same sequences in launches of 64, and sampled
    # sequences against the oracle; one more sequence is refused.
    import mslim_attn
    batch, qh, kvh, d, pt, split = mslim_attn.MAX_BATCH, 8, 4, 64, 16, 64
    gen = torch.Generator(device="cuda").manual_seed(4096)
    rng = np.random.default_rng(4097)
    lens = [int(x) for x in rng.integers(1, 41, size=batch)]
    stride = max(lens)
    k = torch.randn((batch, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((batch, stride, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn((batch, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k_pool, v_pool, table_t, pps, _ = _paged_pool(ctx, k, v, lens, stride, pt, seed=41)
    dense, paged, small = (torch.full_like(q, -1) for _ in range(3))
    ctx.decode_dense(q, k, v, dense, lens, qh, kvh, d, seq_stride_tokens=stride, split_tokens=split)
    ctx.decode_paged(q, k_pool, v_pool, paged, lens, table_t, pps, pt, qh, kvh, d, split_tokens=split)
    _chunked(lambda lo, hi: ctx.decode_dense(q[lo:hi], k[lo:hi], v[lo:hi], small[lo:hi], lens[lo:hi], qh, kvh, d,
                                             seq_stride_tokens=stride, split_tokens=split), batch, 64)
    torch.cuda.synchronize()
    assert torch.equal(dense, paged) and torch.equal(dense, small)
    got = from_torch(dense).reshape(batch, -1)
    for b in (0, 1, 2047, int(np.argmax(lens)), batch - 1):
        t = lens[b]
        ref = _oracle_decode(from_torch(q[b]), from_torch(k[b, :t]), from_torch(v[b, :t]), qh, kvh, d)
        check_bf16(got[b], ref, TOL, "test_decode_at_the_batch_limit")
    over = torch.empty((batch + 1, qh, d), dtype=torch.int16, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="1..4096"):
        ctx.decode_dense(over, k, k, over.clone(), [1] * (batch + 1), qh, kvh, d, seq_stride_tokens=stride)
