"""GPU parity of the projection GEMM (mslim_attn_matrix_multiply, the
tv_hip_matrix_multiply replacement, and its device form) against the oracle's
restatement of the reference product (hipblaslt_bridge.cpp:203-233).  Both
accumulate in fp32, in different orders, so both are held to the same bound
against the exact (f64) product: one BF16 ulp of the exact value (the final
rounding) plus 1e-5 * sum_i |w_i x_i| (fp32 accumulation).  Near-cancelling
outputs are thereby judged in absolute terms, as their terms demand."""
import numpy as np
import pytest
import torch

import mslim_attn
import oracle

pytestmark = pytest.mark.gpu


def bf16(rng, n, scale=1.0):
    return oracle.write_bf16(rng.standard_normal(n, dtype=np.float32) * np.float32(scale))


def within_bound(got_bits, w_bits, x_bits, inner, rows, tokens):
    w = oracle.read_bf16(w_bits).astype(np.float64).reshape(rows, inner)
    x = oracle.read_bf16(x_bits[: tokens * inner]).astype(np.float64).reshape(tokens, inner)
    exact = (x @ w.T).reshape(-1)
    scale = (np.abs(x) @ np.abs(w).T).reshape(-1)
    got = oracle.read_bf16(got_bits[: tokens * rows]).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
    return bool(np.all(np.abs(got - exact) <= ulp + 1e-5 * scale))


def upload(ctx, bits):
    return ctx.buf_upload(np.ascontiguousarray(bits, np.uint16).tobytes())


@pytest.mark.parametrize("inner,rows,tokens", [
    (4096, 6144, 1),    # fused QKV of the cfg5 shape, decode
    (4096, 4096, 8),    # O projection, B = 8
    (14336, 4096, 8),   # down projection
    (4096, 28672, 2),   # gate + up
    (128, 96, 3),
    (4096, 6144, 512),  # prefill chunk, first rows checked
    (14336, 4096, 40),  # down projection of a prompt chunk: the k range split in two, merged
    (8192, 200, 33),    # split with ragged row and token tiles
])
def test_matrix_multiply_matches_oracle(ctx, inner, rows, tokens):
    rng = np.random.default_rng(inner + rows + tokens)
    w = bf16(rng, rows * inner, 0.02)
    x = bf16(rng, tokens * inner)
    wd = upload(ctx, w)
    try:
        got = ctx.matrix_multiply(wd, x, inner, rows, tokens)
        check = min(tokens, 4)
        assert within_bound(got, w, x, inner, rows, check)
        # the oracle's restatement meets the same bound
        want = oracle.matmul_bf16(w, x[: check * inner], inner, rows, check)
        assert within_bound(want, w, x, inner, rows, check)
        # the device form gives the same bits
        xin = torch.from_numpy(x.view(np.int16).copy()).cuda()
        out = torch.empty(tokens * rows, dtype=torch.int16, device="cuda")
        ctx.gemm_bf16(wd, xin, out, inner, rows, tokens)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), got)
    finally:
        ctx.buf_free(wd)


def test_identity_weight_is_exact(ctx):
    n = 256
    rng = np.random.default_rng(3)
    x = bf16(rng, 5 * n)
    eye = oracle.write_bf16(np.eye(n, dtype=np.float32).reshape(-1))
    wd = upload(ctx, eye)
    try:
        assert np.array_equal(ctx.matrix_multiply(wd, x, n, n, 5), x)
    finally:
        ctx.buf_free(wd)


def test_matrix_multiply_rejects_bad_arguments(ctx):
    wd = upload(ctx, np.zeros(64, np.uint16))
    try:
        x = np.zeros(8 * 513, np.uint16)
        with pytest.raises(mslim_attn.MslimAttnError, match="code=-1"):
            ctx.matrix_multiply(wd, x, 8, 8, 513)
        with pytest.raises(mslim_attn.MslimAttnError, match="code=-1"):
            ctx.matrix_multiply(wd, x, 0, 8, 1)
    finally:
        ctx.buf_free(wd)


def dev_bits(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16).copy()).cuda()


def host_bits(t):
    return t.cpu().numpy().view(np.uint16).reshape(-1)


@pytest.mark.parametrize("tokens", [1, 2, 7, 8, 15, 16, 17])
@pytest.mark.parametrize("inner,rows", [(4096, 1000), (14336, 72), (64, 17)])
def test_decode_batch_product_within_bound(ctx, inner, rows, tokens):
    # tokens <= 16 with inner % 32 == 0 run the MFMA decode kernel (ragged row
    # tiles, padded token columns); 17 takes hipBLASLt; same bound for both
    rng = np.random.default_rng(inner * 31 + rows + tokens)
    w, x = bf16(rng, rows * inner, 0.02), bf16(rng, tokens * inner)
    out = torch.empty(tokens * rows, dtype=torch.int16, device="cuda")
    ctx.gemm_bf16(dev_bits(w), dev_bits(x), out, inner, rows, tokens)
    torch.cuda.synchronize()
    assert within_bound(host_bits(out), w, x, inner, rows, tokens)


@pytest.mark.parametrize("inner", [4096, 8192, 14336, 4128])
def test_decode_product_does_not_depend_on_the_batch(ctx, inner):
    # A token's output is the same whichever batch it rides in: 8 tokens
    # (token rows staged in LDS up to 4096 inputs) against the first 8 of 9
    # (token rows read from L2 every k-step) and a 1-token call, bit for bit,
    # plain and with the residual add
    rng = np.random.default_rng(inner)
    rows = 208
    w, x = bf16(rng, rows * inner, 0.02), bf16(rng, 9 * inner)
    resid = bf16(rng, 9 * rows, 2.0)
    wd = dev_bits(w)
    outs = {}
    for t in (9, 8, 1):
        out = torch.empty(t * rows, dtype=torch.int16, device="cuda")
        add = torch.empty(t * rows, dtype=torch.int16, device="cuda")
        ctx.gemm_bf16(wd, dev_bits(x[: t * inner]), out, inner, rows, t)
        ctx.gemm_bf16_add(wd, dev_bits(x[: t * inner]), dev_bits(resid[: t * rows]), add, inner, rows, t)
        outs[t] = (out, add)
    torch.cuda.synchronize()
    for i in range(2):
        nine = host_bits(outs[9][i])
        assert np.array_equal(host_bits(outs[8][i]), nine[: 8 * rows])
        assert np.array_equal(host_bits(outs[1][i]), nine[:rows])
    assert within_bound(host_bits(outs[9][0]), w, x, inner, rows, 9)


def test_unaligned_inner_uses_library_path(ctx):
    rng = np.random.default_rng(9)
    inner, rows, tokens = 4104, 300, 4
    w, x = bf16(rng, rows * inner, 0.02), bf16(rng, tokens * inner)
    out = torch.empty(tokens * rows, dtype=torch.int16, device="cuda")
    ctx.gemm_bf16(dev_bits(w), dev_bits(x), out, inner, rows, tokens)
    torch.cuda.synchronize()
    assert within_bound(host_bits(out), w, x, inner, rows, tokens)


@pytest.mark.parametrize("tokens,inner", [(1, 512), (8, 512), (16, 512), (17, 512), (40, 512), (300, 512), (8, 4096), (4, 14336),
                                          (40, 8192)])
def test_fused_projections_equal_unfused(ctx, tokens, inner):
    # the fused entries are the unfused product followed by the elementwise
    # kernel, bit for bit, on both sides of the decode-kernel token limit, for
    # both tile shapes of the prompt-chunk kernel (300 tokens) and with the
    # split k range of long inner dimensions (8192)
    rng = np.random.default_rng(tokens + inner)
    qr, kvr, inter = 256, 64, 704
    x = dev_bits(bf16(rng, tokens * inner))
    wq, wk, wv = (dev_bits(bf16(rng, r * inner, 0.05)) for r in (qr, kvr, kvr))
    wg, wu = dev_bits(bf16(rng, inter * inner, 0.05)), dev_bits(bf16(rng, inter * inner, 0.05))
    wo = dev_bits(bf16(rng, inner * qr, 0.05))
    empty = lambda n: torch.empty(tokens * n, dtype=torch.int16, device="cuda")  # noqa: E731
    q, k, v = empty(qr), empty(kvr), empty(kvr)
    ctx.gemm_qkv(wq, wk, wv, x, q, k, v, inner, qr, kvr, tokens)
    q2, k2, v2 = empty(qr), empty(kvr), empty(kvr)
    ctx.gemm_bf16(wq, x, q2, inner, qr, tokens)
    ctx.gemm_bf16(wk, x, k2, inner, kvr, tokens)
    ctx.gemm_bf16(wv, x, v2, inner, kvr, tokens)
    act, g, u, act2 = empty(inter), empty(inter), empty(inter), empty(inter)
    ctx.gemm_swiglu(wg, wu, x, act, inner, inter, tokens)
    ctx.gemm_bf16(wg, x, g, inner, inter, tokens)
    ctx.gemm_bf16(wu, x, u, inner, inter, tokens)
    ctx.swiglu(g, u, act2, tokens * inter)
    # O projection with the residual, in place and out of place
    resid = dev_bits(bf16(rng, tokens * inner, 2.0))
    in_place, added, prod, added2 = resid.clone(), empty(inner), empty(inner), empty(inner)
    ctx.gemm_bf16_add(wo, q, resid, added, qr, inner, tokens)
    ctx.gemm_bf16_add(wo, q, in_place, in_place, qr, inner, tokens)
    ctx.gemm_bf16(wo, q, prod, qr, inner, tokens)
    ctx.add(resid, prod, added2, tokens * inner)
    # a down-like product over the full inner dimension (split when long)
    wd = dev_bits(bf16(rng, qr * inner, 0.05))
    resid_d = dev_bits(bf16(rng, tokens * qr, 2.0))
    down, down_prod, down2 = empty(qr), empty(qr), empty(qr)
    ctx.gemm_bf16_add(wd, x, resid_d, down, inner, qr, tokens)
    ctx.gemm_bf16(wd, x, down_prod, inner, qr, tokens)
    ctx.add(resid_d, down_prod, down2, tokens * qr)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    assert torch.equal(act, act2)
    assert torch.equal(added, added2) and torch.equal(in_place, added2)
    assert torch.equal(down, down2)
    wd_bits, x_bits = host_bits(wd), host_bits(x)
    assert within_bound(host_bits(down_prod), wd_bits, x_bits, inner, qr, min(tokens, 8))


@pytest.mark.parametrize("inter", [1, 13, 100, 1000])
@pytest.mark.parametrize("tokens,inner", [(1, 4096), (8, 4096), (5, 96), (12, 4096), (8, 6144)])
def test_swiglu_tiles_of_any_row_count(ctx, tokens, inner, inter):
    # a decode SwiGLU tile is 8 outputs (their gate rows, then their up rows,
    # in one MFMA operand): row counts that leave a partial last tile, token
    # rows staged in LDS (<= 8 of <= 4096) or read per step (12 tokens, inner
    # 6144), against the two plain products and mslim_attn_swiglu, and with
    # the RMSNorm fused against mslim_attn_rmsnorm first
    rng = np.random.default_rng(inter * 131 + tokens * 7 + inner)
    x = dev_bits(bf16(rng, tokens * inner, 2.0))
    nw = dev_bits(bf16(rng, inner, 0.5))
    wg, wu = dev_bits(bf16(rng, inter * inner, 0.05)), dev_bits(bf16(rng, inter * inner, 0.05))
    empty = lambda n: torch.empty(n, dtype=torch.int16, device="cuda")  # noqa: E731
    act, g, u, act2 = empty(tokens * inter), empty(tokens * inter), empty(tokens * inter), empty(tokens * inter)
    ctx.gemm_swiglu(wg, wu, x, act, inner, inter, tokens)
    ctx.gemm_bf16(wg, x, g, inner, inter, tokens)
    ctx.gemm_bf16(wu, x, u, inner, inter, tokens)
    ctx.swiglu(g, u, act2, tokens * inter)
    normed, fused, unfused = empty(tokens * inner), empty(tokens * inter), empty(tokens * inter)
    ctx.rmsnorm(x, nw, normed, tokens, inner, 1e-5)
    ctx.gemm_swiglu(wg, wu, normed, unfused, inner, inter, tokens)
    ctx.rmsnorm_gemm_swiglu(nw, 1e-5, wg, wu, x, fused, inner, inter, tokens)
    torch.cuda.synchronize()
    assert torch.equal(act, act2)
    assert torch.equal(fused, unfused)
    assert within_bound(host_bits(g), host_bits(wg), host_bits(x), inner, inter, min(tokens, 8))


@pytest.mark.parametrize("tokens,inner", [(1, 4096), (8, 4096), (3, 96), (9, 4096), (4, 4104), (40, 512),
                                          (2, 8192)])
def test_rmsnorm_fused_projections_equal_unfused(ctx, tokens, inner):
    # RMSNorm + projection entries equal mslim_attn_rmsnorm followed by the
    # plain, QKV and SwiGLU products, bit for bit: inside the decode kernel
    # (<= 8 rows of <= 4096), and through the normalised-rows buffer for
    # 9 rows, inner 4104 (no MFMA decode kernel), prompt chunks and inner 8192
    rng = np.random.default_rng(7 * tokens + inner)
    qr, kvr, inter = 320, 64, 208
    x = dev_bits(bf16(rng, tokens * inner, 3.0))
    nw = dev_bits(bf16(rng, inner, 0.5))
    eps = 1e-5
    wq, wk, wv = (dev_bits(bf16(rng, r * inner, 0.05)) for r in (qr, kvr, kvr))
    wg, wu = dev_bits(bf16(rng, inter * inner, 0.05)), dev_bits(bf16(rng, inter * inner, 0.05))
    empty = lambda n: torch.empty(tokens * n, dtype=torch.int16, device="cuda")  # noqa: E731
    normed = empty(inner)
    ctx.rmsnorm(x, nw, normed, tokens, inner, eps)
    plain, plain2 = empty(qr), empty(qr)
    ctx.gemm_bf16(wq, normed, plain, inner, qr, tokens)
    ctx.rmsnorm_gemm_bf16(nw, eps, wq, x, plain2, inner, qr, tokens)
    q, k, v, q2, k2, v2 = empty(qr), empty(kvr), empty(kvr), empty(qr), empty(kvr), empty(kvr)
    ctx.gemm_qkv(wq, wk, wv, normed, q, k, v, inner, qr, kvr, tokens)
    ctx.rmsnorm_gemm_qkv(nw, eps, wq, wk, wv, x, q2, k2, v2, inner, qr, kvr, tokens)
    act, act2 = empty(inter), empty(inter)
    ctx.gemm_swiglu(wg, wu, normed, act, inner, inter, tokens)
    ctx.rmsnorm_gemm_swiglu(nw, eps, wg, wu, x, act2, inner, inter, tokens)
    torch.cuda.synchronize()
    assert torch.equal(plain, plain2)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    assert torch.equal(q, plain)
    assert torch.equal(act, act2)
    # the normalised rows themselves are the oracle's
    want = oracle.rmsnorm_gpu(host_bits(x), host_bits(nw), tokens, inner, eps)
    assert np.array_equal(host_bits(normed), want)


def test_rmsnorm_fused_rejects_bad_arguments(ctx):
    x = torch.zeros(4 * 64, dtype=torch.int16, device="cuda")
    w = torch.zeros(32 * 64, dtype=torch.int16, device="cuda")
    out = torch.empty(4 * 32, dtype=torch.int16, device="cuda")
    nw = torch.zeros(64, dtype=torch.int16, device="cuda")
    with pytest.raises(mslim_attn.MslimAttnError, match="code=-1"):
        ctx.rmsnorm_gemm_bf16(None, 1e-5, w, x, out, 64, 32, 4)
    with pytest.raises(mslim_attn.MslimAttnError, match="code=-1"):
        ctx.rmsnorm_gemm_bf16(nw, float("nan"), w, x, out, 64, 32, 4)
    with pytest.raises(mslim_attn.MslimAttnError, match="code=-1"):
        ctx.rmsnorm_gemm_swiglu(nw, -1.0, w, w, x, out, 64, 32, 4)
