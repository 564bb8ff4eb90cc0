"""GPU parity of causal prefill attention against the CPU oracle.

Row i of a chunk attends keys 0..prior+i (llm_prefill_qk/softmax/pv,
gpu_llm.cl:462-541; the CPU decoder processes prompts token by token,
native_cpu_adapter.rs:486-534).  Tolerance: max abs <= 2e-2 on BF16 outputs.
"""
import numpy as np
import pytest
import torch

import oracle
from _data import check_bf16, from_torch, max_abs_bf16, normal_bf16, tiled_input, to_torch

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _prefill(ctx, qb, kb, vb, queries, prior, qh, kvh, d):
    q, k, v = to_torch(qb), to_torch(kb), to_torch(vb)
    out = torch.empty_like(q)
    ctx.prefill_causal(q, k, v, out, queries, prior, qh, kvh, d)
    torch.cuda.synchronize()
    return from_torch(out)


@pytest.mark.parametrize("qh,kvh,d", [(32, 8, 128), (64, 8, 128), (8, 8, 128), (16, 8, 128),
                                      (8, 2, 64), (4, 4, 64), (4, 2, 80), (12, 4, 128)])
def test_prefill_small_shapes(ctx, qh, kvh, d):
    rng = np.random.default_rng(qh * 7 + d)
    for queries, prior in [(1, 0), (5, 0), (33, 7), (100, 0), (130, 60), (64, 64)]:
        hist = prior + queries
        qb = normal_bf16(rng, (queries, qh, d))
        kb = normal_bf16(rng, (hist, kvh, d))
        vb = normal_bf16(rng, (hist, kvh, d))
        got = _prefill(ctx, qb, kb, vb, queries, prior, qh, kvh, d)
        ref = oracle.prefill_causal_cpu(oracle.read_bf16(qb), kb, vb, qh, kvh, d, queries, prior)
        check_bf16(got, ref, TOL, "test_prefill_small_shapes")
        gref = oracle.gpu_reference_attention(qb, kb, vb, qh, kvh, d, queries, prior)
        check_bf16(got, oracle.read_bf16(gref), TOL, "prefill vs reference GPU arithmetic")


def test_prefill_reference_inputs_multi_query(ctx):
    # tiled_attention.rs:345-362: queries in {1, min(n,5)} at histories n.
    qh, kvh, d = 8, 2, 128
    for n in [1, 2, 31, 33, 63, 65, 129, 375]:
        for queries in sorted({1, min(n, 5)}):
            prior = n - queries
            qb = tiled_input(queries * qh * d, 3).reshape(queries, qh, d)
            kb = tiled_input(n * kvh * d, 7).reshape(n, kvh, d)
            vb = tiled_input(n * kvh * d, 11).reshape(n, kvh, d)
            got = _prefill(ctx, qb, kb, vb, queries, prior, qh, kvh, d)
            ref = oracle.prefill_causal_cpu(oracle.read_bf16(qb), kb, vb, qh, kvh, d, queries, prior)
            check_bf16(got, ref, TOL, "test_prefill_reference_inputs_multi_query")


@pytest.mark.parametrize("qh,kvh,d", [(16, 2, 128), (8, 2, 64)])
def test_prefill_moving_reference_recomputes_tiles(ctx, qh, kvh, d):
    """Scores that climb by about 6.5 log2 units per 64-key tile, so every
    tile's row sums under the previous reference exceed 2^8 and the kernel
    must move the reference and recompute that tile's P; and one late key
    whose score is ~280 log2 units above the reference, so p overflows to
    inf before the recompute.  Q = 1, K[t] = 0.4 t / 64 (D = 128 scaling)
    except K[450] = 20; V random.  Checked against the oracle."""
    rng = np.random.default_rng(20261202 + d)
    queries, prior = 512, 0
    scale = (128.0 / d) ** 0.5  # the same log2 growth per tile at D = 64
    q = np.ones((queries, qh, d), np.float32)
    kvals = 0.4 * scale * np.arange(queries, dtype=np.float32) / 64.0
    kvals[450] = 20.0 * scale
    k = np.repeat(kvals[:, None, None], kvh, axis=1).repeat(d, axis=2)
    qb = oracle.write_bf16(q).reshape(q.shape)
    kb = oracle.write_bf16(k).reshape(k.shape)
    vb = normal_bf16(rng, (queries, kvh, d))
    got = _prefill(ctx, qb, kb, vb, queries, prior, qh, kvh, d)
    ref = oracle.prefill_causal_cpu(oracle.read_bf16(qb), kb, vb, qh, kvh, d, queries, prior)
    assert np.isfinite(oracle.read_bf16(got)).all()
    check_bf16(got, ref, TOL, "test_prefill_moving_reference_recomputes_tiles")


def _rows_reference(q_bits, k_bits, v_bits, rows, prior, qh, kvh, d):
    out = {}
    for r in rows:
        n = prior + r + 1
        out[r] = oracle.dense_attention_bf16(oracle.read_bf16(q_bits[r].reshape(-1)), k_bits[:n],
                                             v_bits[:n], qh, kvh, d)
    return out


def test_prefill_cfg2_with_rope(ctx):
    # S=2048, 32/8/128, RoPE theta=5e5 rotate-half applied
    # to Q and K by the product's RoPE kernel, causal, fp32 accumulate.
    s, qh, kvh, d = 2048, 32, 8, 128
    rng = np.random.default_rng(2)
    qb = normal_bf16(rng, (s, qh, d))
    kb = normal_bf16(rng, (s, kvh, d))
    vb = normal_bf16(rng, (s, kvh, d))
    q_raw, k_raw, v = to_torch(qb), to_torch(kb), to_torch(vb)
    q = torch.empty_like(q_raw)
    k = torch.empty_like(k_raw)
    ctx.rope(q_raw, q, s, qh, d, 0, 500000.0)
    ctx.rope(k_raw, k, s, kvh, d, 0, 500000.0)
    out = torch.empty_like(q)
    ctx.prefill_causal(q, k, v, out, s, 0, qh, kvh, d)
    torch.cuda.synchronize()
    # the RoPE outputs are bit-exact against the oracle's restatement
    q_rot = oracle.rope_gpu(qb, s, qh, d, 0, 500000.0).reshape(s, qh, d)
    k_rot = oracle.rope_gpu(kb, s, kvh, d, 0, 500000.0).reshape(s, kvh, d)
    assert np.array_equal(from_torch(q), q_rot)
    assert np.array_equal(from_torch(k), k_rot)
    got = from_torch(out)
    rows = [0, 1, 31, 32, 63, 64, 127, 1000, 1023, 1024, 2046, 2047] + \
        [int(x) for x in rng.integers(0, s, size=12)]
    ref = _rows_reference(q_rot, k_rot, vb, rows, 0, qh, kvh, d)
    for r in rows:
        check_bf16(got[r], ref[r], TOL, "test_prefill_cfg2_with_rope")
    # repeat is bit-identical and inputs are unmodified
    out2 = torch.empty_like(q)
    ctx.prefill_causal(q, k, v, out2, s, 0, qh, kvh, d)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert np.array_equal(from_torch(v), vb)


def test_prefill_cfg4_shape_rows(ctx):
    # BASELINE config 4 prefill shape: S=8192, 64/8/128.  Sampled rows.
    s, qh, kvh, d = 8192, 64, 8, 128
    gen = torch.Generator(device="cuda").manual_seed(8)
    q = torch.randn((s, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k = torch.randn((s, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((s, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty_like(q)
    ctx.prefill_causal(q, k, v, out, s, 0, qh, kvh, d)
    torch.cuda.synchronize()
    got = from_torch(out)
    qb, kb, vb = from_torch(q), from_torch(k), from_torch(v)
    rows = [0, 8191, 4095, 4096, 127, 128, 5000, 7777]
    ref = _rows_reference(qb, kb, vb, rows, 0, qh, kvh, d)
    for r in rows:
        check_bf16(got[r], ref[r], TOL, "test_prefill_cfg4_shape_rows")


def test_prefill_chunk_after_prior_matches_single_pass(ctx):
    # a prompt processed as two chunks (prefill.rs chunking) equals one pass
    qh, kvh, d, s = 16, 4, 128, 300
    rng = np.random.default_rng(12)
    qb = normal_bf16(rng, (s, qh, d))
    kb = normal_bf16(rng, (s, kvh, d))
    vb = normal_bf16(rng, (s, kvh, d))
    whole = _prefill(ctx, qb, kb, vb, s, 0, qh, kvh, d)
    second = _prefill(ctx, qb[200:], kb, vb, 100, 200, qh, kvh, d)
    ref = oracle.prefill_causal_cpu(oracle.read_bf16(qb[200:]), kb, vb, qh, kvh, d, 100, 200)
    check_bf16(second, ref, TOL, "test_prefill_chunk_after_prior_matches_single_pass")
    assert max_abs_bf16(whole[200:], oracle.read_bf16(second)) <= TOL


def test_prefill_rejects_bad_arguments(ctx):
    import mslim_attn
    q = torch.zeros((4, 8, 128), dtype=torch.int16, device="cuda")
    k = torch.zeros((4, 8, 128), dtype=torch.int16, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="alias"):
        ctx.prefill_causal(q, k, k, k, 4, 0, 8, 8, 128)
    out = torch.empty_like(q)
    with pytest.raises(mslim_attn.MslimAttnError):
        ctx.prefill_causal(q, k, k, out, 0, 0, 8, 8, 128)
    with pytest.raises(mslim_attn.MslimAttnError):
        ctx.prefill_causal(q, k, k, out, 4, -1, 8, 8, 128)


# Launches too small to fill the CUs split long row blocks into chunks of key
# tiles (merged in fixed chunk order): cfg2, the decoder's 512-token prompt
# chunks after a long prior, ragged query counts, D = 64 and a group of 2.
SPLIT_SHAPES = [(2048, 0, 32, 8, 128), (512, 3584, 32, 8, 128), (1000, 777, 32, 8, 128),
                (1500, 0, 16, 2, 64), (2048, 0, 16, 8, 128), (512, 512, 32, 8, 128),
                (512, 512, 64, 8, 128), (2048, 0, 32, 8, 64)]


@pytest.mark.parametrize("queries,prior,qh,kvh,d", SPLIT_SHAPES)
def test_prefill_split_launches(ctx, queries, prior, qh, kvh, d):
    import mslim_attn
    assert mslim_attn.prefill_split_tiles(queries, prior, qh, kvh, d) > 0
    hist = prior + queries
    gen = torch.Generator(device="cuda").manual_seed(queries + prior + qh)
    q = torch.randn((queries, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    k = torch.randn((hist, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    v = torch.randn((hist, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    out, again, whole = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    ctx.prefill_causal(q, k, v, out, queries, prior, qh, kvh, d)
    ctx.prefill_causal(q, k, v, again, queries, prior, qh, kvh, d)
    try:
        ctx.set_prefill_split(False)
        ctx.prefill_causal(q, k, v, whole, queries, prior, qh, kvh, d)
    finally:
        ctx.set_prefill_split(True)
    torch.cuda.synchronize()
    # deterministic: the merge order does not depend on which chunk ends last
    assert torch.equal(out, again)
    got, unsplit = from_torch(out), from_torch(whole)
    qb, kb, vb = from_torch(q), from_torch(k), from_torch(v)
    rng = np.random.default_rng(queries)
    rows = sorted({0, 1, 63, 64, queries // 2, queries - 2, queries - 1} |
                  {int(x) for x in rng.integers(0, queries, size=10)})
    ref = _rows_reference(qb, kb, vb, rows, prior, qh, kvh, d)
    for r in rows:
        check_bf16(got[r], ref[r], TOL, "test_prefill_split_launches")
        check_bf16(unsplit[r], ref[r], TOL, "test_prefill_split_launches")
    # split and unsplit launches differ in rounding only
    diff = np.abs(oracle.read_bf16(got).astype(np.float64) - oracle.read_bf16(unsplit).astype(np.float64))
    assert float(diff.max()) <= TOL


def test_prefill_split_random_shapes_match_unsplit(ctx):
    # The chunk length comes from a model of the dispatch and varies with the
    # shape; every chunking must equal the unsplit launch up to rounding and
    # repeat bit for bit.  Seeded shapes of every head layout the fast kernel
    # takes, with and without a prior (195 such shapes passed the same check
    # when the model was introduced; these are a fixed sample).
    import mslim_attn
    rng = np.random.default_rng(20261202)
    layouts = [(32, 8), (64, 8), (16, 2), (8, 8), (32, 4), (28, 4), (16, 16), (24, 8)]
    checked = 0
    while checked < 24:
        qh, kvh = layouts[int(rng.integers(len(layouts)))]
        d = int(rng.choice([64, 128]))
        queries = int(rng.integers(1, 4097))
        prior = int(rng.choice([0, 0, int(rng.integers(0, 8193))]))
        chunk = mslim_attn.prefill_split_tiles(queries, prior, qh, kvh, d)
        if chunk <= 0:
            continue
        checked += 1
        print(f"split shape {queries} after {prior}, {qh}/{kvh} heads, d {d}: chunks of {chunk} tiles", flush=True)
        gen = torch.Generator(device="cuda").manual_seed(checked)
        q = torch.randn((queries, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
        k = torch.randn((prior + queries, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
        v = torch.randn((prior + queries, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
        out, again, whole = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
        ctx.prefill_causal(q, k, v, out, queries, prior, qh, kvh, d)
        ctx.prefill_causal(q, k, v, again, queries, prior, qh, kvh, d)
        try:
            ctx.set_prefill_split(False)
            ctx.prefill_causal(q, k, v, whole, queries, prior, qh, kvh, d)
        finally:
            ctx.set_prefill_split(True)
        torch.cuda.synchronize()
        assert torch.equal(out, again)
        got = out.view(torch.bfloat16).float()
        assert bool(torch.isfinite(got).all())
        assert (got - whole.view(torch.bfloat16).float()).abs().max().item() <= TOL


def test_prefill_split_plan_is_shape_only(ctx):
    import mslim_attn
    # cfg4's 8,192-token prefill has 2,048 workgroups: never split
    assert mslim_attn.prefill_split_tiles(8192, 0, 64, 8, 128) == 0
    # tiny launches have nothing to split
    assert mslim_attn.prefill_split_tiles(100, 0, 32, 8, 128) == 0
    assert mslim_attn.prefill_split_tiles(2048, 0, 32, 8, 128) == 20
    with pytest.raises(mslim_attn.MslimAttnError):
        mslim_attn.prefill_split_tiles(0, 0, 32, 8, 128)


# Launches with at least two row blocks per CU hand their shortest row blocks
# out at run time (an atomic counter in the context): cfg4-like 8 heads per
# workgroup, 4 heads (64-row blocks), D = 64, and kv_heads = 4 with a work
# list that does not fill the last XCD's slice (pool entries past the end).
POOL_SHAPES = [(4096, 0, 64, 8, 128), (8192, 0, 32, 8, 128), (8192, 0, 16, 2, 64),
               (4250, 100, 32, 4, 128), (3000, 500, 64, 8, 128)]


def test_prefill_pool_matches_static_mapping(ctx):
    import mslim_attn
    sentinel = -0x40  # 0xFFC0: a BF16 NaN, so a row block left unwritten shows
    for queries, prior, qh, kvh, d in POOL_SHAPES:
        assert mslim_attn.prefill_pool_items(queries, prior, qh, kvh, d) > 0
        hist = prior + queries
        gen = torch.Generator(device="cuda").manual_seed(queries * 3 + qh)
        q = torch.randn((queries, qh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
        k = torch.randn((hist, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
        v = torch.randn((hist, kvh, d), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
        pooled = [torch.full_like(q, sentinel) for _ in range(2)]
        static = torch.full_like(q, sentinel)
        # two pooled launches back to back: the first must leave its counter at zero
        for out in pooled:
            ctx.prefill_causal(q, k, v, out, queries, prior, qh, kvh, d)
        try:
            ctx.set_prefill_pool(False)
            ctx.prefill_causal(q, k, v, static, queries, prior, qh, kvh, d)
        finally:
            ctx.set_prefill_pool(True)
        torch.cuda.synchronize()
        shape = (queries, prior, qh, kvh, d)
        assert not bool((static == sentinel).any()), shape
        # each row block is computed the same way whichever workgroup takes it
        assert torch.equal(pooled[0], static), shape
        assert torch.equal(pooled[1], static), shape
        got = from_torch(pooled[0])
        qb, kb, vb = from_torch(q), from_torch(k), from_torch(v)
        rows = [0, 31, 32, queries // 2, queries - 33, queries - 1]
        ref = _rows_reference(qb, kb, vb, rows, prior, qh, kvh, d)
        for r in rows:
            check_bf16(got[r], ref[r], TOL, "test_prefill_pool_matches_static_mapping")


def test_prefill_pool_option_rejects_bad_values(ctx):
    import mslim_attn
    with pytest.raises(mslim_attn.MslimAttnError):
        ctx.set_option(mslim_attn.OPT_PREFILL_POOL, 2)
