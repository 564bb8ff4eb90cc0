"""GPU parity of the feeder kernels (bit-exact against the oracle's
restatement of gpu_llm.cl) and of the ColdStore-exact page pool (byte-exact
gather, logical K/V SHA-256 equal across dense, paged and the oracle)."""
import numpy as np
import pytest
import torch

import oracle
from _data import from_torch, normal_bf16, to_torch

pytestmark = pytest.mark.gpu


# 4096 and 8192 take the LDS-staged kernel; 4104, 100, 130 and 14336 the direct one
@pytest.mark.parametrize("tokens,hidden", [(1, 4096), (3, 4096), (8, 4096), (2, 8192), (5, 4104), (2, 100),
                                           (4, 130), (1, 14336)])
def test_rmsnorm_bit_exact(ctx, tokens, hidden):
    rng = np.random.default_rng(hidden + tokens)
    xb = normal_bf16(rng, (tokens, hidden), 3.0)
    wb = normal_bf16(rng, (hidden,), 0.02)
    out = torch.empty((tokens, hidden), dtype=torch.int16, device="cuda")
    ctx.rmsnorm(to_torch(xb), to_torch(wb), out, tokens, hidden, 1e-5)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(out).reshape(-1), oracle.rmsnorm_gpu(xb, wb, tokens, hidden, 1e-5))


def test_bf16_encoder_matches_the_rule_on_every_encoding(ctx):
    # the conversion instruction every kernel writes with, against the
    # reference's integer rule (gpu_llm.cl:10-21), over all 2^32 f32 inputs
    assert ctx.check_bf16_encoding() == 0


@pytest.mark.parametrize("llama3", [False, True])
@pytest.mark.parametrize("start", [0, 1, 4090, 32760])
def test_rope_bit_exact(ctx, llama3, start):
    rng = np.random.default_rng(start + 17)
    tokens, heads, d = 9, 32, 128
    xb = normal_bf16(rng, (tokens, heads, d))
    params = (8.0, 1.0, 4.0, 8192.0) if llama3 else (1.0, 1.0, 2.0, 1.0)
    out = torch.empty((tokens, heads, d), dtype=torch.int16, device="cuda")
    ctx.rope(to_torch(xb), out, tokens, heads, d, start, 500000.0, llama3, *params)
    torch.cuda.synchronize()
    ref = oracle.rope_gpu(xb, tokens, heads, d, start, 500000.0, int(llama3), *params)
    assert np.array_equal(from_torch(out).reshape(-1), ref)


@pytest.mark.parametrize("tokens,qh,kvh,d,start,llama3", [
    (2048, 32, 8, 128, 0, False),     # cfg2's prompt: three rows per workgroup
    (13, 32, 8, 128, 4090, True),     # a ragged last workgroup
    (9, 64, 8, 128, 7, False),        # one row per workgroup
    (7, 4, 2, 64, 123, False),
    (3, 2, 1, 512, 32760, True),      # the whole 256-pair table
    (4, 8, 8, 256, 1, False),
    (5, 4, 4, 72, 9, False),          # head_dim % 16 != 0: two separate launches
    (3, 96, 32, 128, 40, False),      # 16,384 elements per row: the most one launch takes
    (3, 160, 32, 128, 40, True),      # 24,576: two separate launches
    (2, 224, 32, 128, 5, False),      # 32,768
])
def test_rope_qk_bit_exact(ctx, tokens, qh, kvh, d, start, llama3):
    # one launch for Q and K gives mslim_attn_rope's bits on each
    rng = np.random.default_rng(tokens * 7 + d)
    qb, kb = normal_bf16(rng, (tokens, qh, d)), normal_bf16(rng, (tokens, kvh, d), 2.0)
    params = (8.0, 1.0, 4.0, 8192.0) if llama3 else (1.0, 1.0, 2.0, 1.0)
    qo = torch.empty((tokens, qh, d), dtype=torch.int16, device="cuda")
    ko = torch.empty((tokens, kvh, d), dtype=torch.int16, device="cuda")
    ctx.rope_qk(to_torch(qb), qo, to_torch(kb), ko, tokens, qh, kvh, d, start, 500000.0, llama3, *params)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(qo).reshape(-1), oracle.rope_gpu(qb, tokens, qh, d, start, 500000.0,
                                                                      int(llama3), *params))
    assert np.array_equal(from_torch(ko).reshape(-1), oracle.rope_gpu(kb, tokens, kvh, d, start, 500000.0,
                                                                      int(llama3), *params))


@pytest.mark.parametrize("heads", [128, 129, 256])
def test_rope_many_heads_bit_exact(ctx, heads):
    # mslim_attn_rope on rows of up to 128 heads x 128 runs the Q + K kernel
    # with no K rows; wider rows the per-token kernel; both give the oracle's
    # bits
    tokens, d, start = 3, 128, 1000
    rng = np.random.default_rng(heads)
    xb = normal_bf16(rng, (tokens, heads, d))
    out = torch.empty((tokens, heads, d), dtype=torch.int16, device="cuda")
    ctx.rope(to_torch(xb), out, tokens, heads, d, start, 500000.0)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(out).reshape(-1), oracle.rope_gpu(xb, tokens, heads, d, start, 500000.0))


@pytest.mark.parametrize("llama3", [False, True])
def test_rope_table_equals_the_oracle_at_every_position(ctx, llama3):
    # Rows of ones in the first half of a head and zeros in the second make
    # RoPE output c (first half) and s (second half) of every pair, so one
    # call over positions 0 .. 36,863 reads back the whole c/s table the
    # context builds for them, through the per-token and the fused Q + K
    # kernels; each must equal the oracle's c and s at every position.
    d, tokens = 128, 36864
    row = np.concatenate([np.full(d // 2, 0x3F80, np.uint16), np.zeros(d // 2, np.uint16)])
    xb = np.tile(row, (tokens, 1))
    params = (8.0, 1.0, 4.0, 8192.0) if llama3 else (1.0, 1.0, 2.0, 1.0)
    want = oracle.rope_gpu(xb, tokens, 1, d, 0, 500000.0, int(llama3), *params)
    out = torch.empty((tokens, 1, d), dtype=torch.int16, device="cuda")
    ctx.rope(to_torch(xb), out, tokens, 1, d, 0, 500000.0, llama3, *params)
    qo, ko = torch.empty_like(out), torch.empty_like(out)
    ctx.rope_qk(to_torch(xb), qo, to_torch(xb), ko, tokens, 1, 1, d, 0, 500000.0, llama3, *params)
    torch.cuda.synchronize()
    for got in (out, qo, ko):
        bad = np.nonzero(from_torch(got).reshape(-1) != want)[0]
        assert bad.size == 0, f"{bad.size} values differ, first at position {bad[0] // d}, pair {bad[0] % d}"


def test_rope_cossin_table_limit_and_configurations(ctx):
    # The context keeps a table of c and s by position (at most 32 MiB:
    # 131,072 positions at head_dim 128).  Rows inside it read the table,
    # rows past it (and workgroups that straddle it) compute c and s
    # themselves, and a new configuration rebuilds it; every case gives the
    # oracle's bits.
    rng = np.random.default_rng(11)
    qh, kvh, d = 4, 2, 128
    for theta in (500000.0, 10000.0, 500000.0):
        for start, tokens in ((131060, 20), (200000, 3), (5, 9)):
            qb, kb = normal_bf16(rng, (tokens, qh, d)), normal_bf16(rng, (tokens, kvh, d))
            qo = torch.empty((tokens, qh, d), dtype=torch.int16, device="cuda")
            ko = torch.empty((tokens, kvh, d), dtype=torch.int16, device="cuda")
            ro = torch.empty((tokens, qh, d), dtype=torch.int16, device="cuda")
            ctx.rope_qk(to_torch(qb), qo, to_torch(kb), ko, tokens, qh, kvh, d, start, theta)
            ctx.rope(to_torch(qb), ro, tokens, qh, d, start, theta)
            torch.cuda.synchronize()
            want_q = oracle.rope_gpu(qb, tokens, qh, d, start, theta)
            assert np.array_equal(from_torch(qo).reshape(-1), want_q), (theta, start)
            assert np.array_equal(from_torch(ro).reshape(-1), want_q), (theta, start)
            assert np.array_equal(from_torch(ko).reshape(-1), oracle.rope_gpu(kb, tokens, kvh, d, start, theta))


def test_rope_other_head_dims(ctx):
    # 64, 80, 256, 512: 16-byte chunks (512: the whole 256-pair frequency
    # table); 72 (half not a multiple of 8): one element per lane; 1024: the
    # per-element kernel (head_dim > 512)
    rng = np.random.default_rng(1)
    for d in (64, 72, 80, 256, 512, 1024):
        xb = normal_bf16(rng, (5, 4, d))
        out = torch.empty((5, 4, d), dtype=torch.int16, device="cuda")
        ctx.rope(to_torch(xb), out, 5, 4, d, 123, 10000.0)
        torch.cuda.synchronize()
        assert np.array_equal(from_torch(out).reshape(-1), oracle.rope_gpu(xb, 5, 4, d, 123, 10000.0))


def test_rope_unaligned_rows_take_the_element_path(ctx):
    # an output one element past a 16-byte boundary cannot take 16-byte chunks
    rng = np.random.default_rng(2)
    tokens, heads, d = 3, 8, 128
    xb = normal_bf16(rng, (tokens, heads, d))
    buf = torch.empty(tokens * heads * d + 1, dtype=torch.int16, device="cuda")
    out = buf[1:]
    ctx.rope(to_torch(xb), out, tokens, heads, d, 77, 500000.0)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(out).reshape(-1), oracle.rope_gpu(xb, tokens, heads, d, 77, 500000.0))


def test_swiglu_bit_exact(ctx):
    rng = np.random.default_rng(5)
    n = 14336 * 3
    gb = normal_bf16(rng, (n,), 4.0)
    ub = normal_bf16(rng, (n,))
    special = oracle.write_bf16(np.array([0.0, -0.0, 88.0, -88.0, 1e30, -1e30, np.inf, -np.inf], np.float32))
    gb[:special.size] = special
    out = torch.empty((n,), dtype=torch.int16, device="cuda")
    ctx.swiglu(to_torch(gb), to_torch(ub), out, n)
    torch.cuda.synchronize()
    got = from_torch(out)
    ref = oracle.swiglu(gb, ub)
    finite = np.isfinite(oracle.read_bf16(ref))
    assert np.array_equal(got[finite], ref[finite])
    # non-finite results: same class (inf/nan) and sign
    assert np.array_equal(np.isnan(oracle.read_bf16(got)), np.isnan(oracle.read_bf16(ref)))


def _table(pages, seed):
    return np.random.default_rng(seed).permutation(pages).astype(np.int32)


@pytest.mark.parametrize("page_tokens", [16, 64])
def test_pages_write_gather_and_oracle_gather(ctx, page_tokens):
    rng = np.random.default_rng(page_tokens)
    kvh, d, t = 8, 128, 1000
    kb = normal_bf16(rng, (t, kvh, d))
    vb = normal_bf16(rng, (t, kvh, d))
    pages = (t + page_tokens - 1) // page_tokens
    table = _table(pages, 5)
    tt = torch.from_numpy(table).cuda()
    k_pool = torch.zeros((pages, kvh, page_tokens, d), dtype=torch.int16, device="cuda")
    v_pool = torch.zeros_like(k_pool)
    # append in two uneven batches, as decode appends after prefill
    ctx.pages_write(k_pool, v_pool, tt, page_tokens, kvh, d, 0, 700,
                    to_torch(kb[:700]), to_torch(vb[:700]))
    ctx.pages_write(k_pool, v_pool, tt, page_tokens, kvh, d, 700, 300,
                    to_torch(kb[700:]), to_torch(vb[700:]))
    torch.cuda.synchronize()
    # every page is the head-major ColdStore payload of its tokens
    kp = from_torch(k_pool)
    for i in (0, 3, pages - 1):
        n = min(page_tokens, t - i * page_tokens)
        payload = oracle.token_to_head_major(kb[i * page_tokens:i * page_tokens + n], n, kvh, d * 2)
        page = kp[table[i]].reshape(kvh, page_tokens, d)[:, :n, :]
        assert page.tobytes() == payload.tobytes()
    # device gather == source rows == oracle gather through the same table
    rows = torch.empty((t, kvh, d), dtype=torch.int16, device="cuda")
    ctx.pages_gather(v_pool, tt, page_tokens, kvh, d, 0, t, rows)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(rows), vb)
    positions = np.array([0, 1, 15, 16, 17, 500, 999], np.uint32)
    page_of = table[np.arange(t) // page_tokens].astype(np.uint32)
    offset_of = (np.arange(t) % page_tokens).astype(np.uint32)
    sparse = oracle.gather_token_major(from_torch(v_pool), page_tokens, kvh, d * 2, page_of,
                                       offset_of, positions)
    assert sparse.tobytes() == vb[positions].tobytes()
    part = torch.empty((200, kvh, d), dtype=torch.int16, device="cuda")
    ctx.pages_gather(k_pool, tt, page_tokens, kvh, d, 650, 200, part)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(part), kb[650:850])


def test_logical_kv_sha256_dense_paged_oracle(ctx):
    rng = np.random.default_rng(42)
    layers, kvh, d, t, pt = 3, 8, 128, 777, 16
    ks = [normal_bf16(rng, (t, kvh, d)) for _ in range(layers)]
    vs = [normal_bf16(rng, (t, kvh, d)) for _ in range(layers)]
    expected = oracle.logical_kv_sha256(ks, vs, t, kvh, d * 2)
    kd = [to_torch(k) for k in ks]
    vd = [to_torch(v) for v in vs]
    assert ctx.logical_kv_sha256(kd, vd, t, kvh, d) == expected
    pages = (t + pt - 1) // pt
    kps, vps, tables = [], [], []
    for layer in range(layers):
        tt = torch.from_numpy(_table(pages, layer)).cuda()
        kp = torch.zeros((pages, kvh, pt, d), dtype=torch.int16, device="cuda")
        vp = torch.zeros_like(kp)
        ctx.pages_write(kp, vp, tt, pt, kvh, d, 0, t, kd[layer], vd[layer])
        kps.append(kp); vps.append(vp); tables.append(tt)
    torch.cuda.synchronize()
    assert ctx.logical_kv_sha256(kps, vps, t, kvh, d, page_tables=tables, page_tokens=pt) == expected
    # a single flipped bit changes the digest
    vd[1][5, 3, 7] ^= 1
    assert ctx.logical_kv_sha256(kd, vd, t, kvh, d) != expected
