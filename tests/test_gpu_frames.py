"""GPU parity of the portable-backend decode (GpuBackend::decode,
gpu_backend.rs:149-377) against the f64 CpuReferenceBackend oracle
(portable.rs:575-646), through the C ABI.

Tolerance: |cpu - gpu| < 1e-4 per output element, the bound of the
reference's own GPU tests (gpu_backend.rs:410, :439).  Format
decoding is checked bit-exactly on every BF16 and F16 encoding.
"""
import numpy as np
import pytest
import torch

import mslim_attn
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-4
BF16, F16, F32 = mslim_attn.FORMAT_BF16, mslim_attn.FORMAT_F16, mslim_attn.FORMAT_F32


def _encode(values: np.ndarray, fmt: int) -> np.ndarray:
    """Raw little-endian frame bits of f32 values, rounded to nearest even
    (half 2.7.1 bf16/f16 from_f32, as the reference tests encode them)."""
    values = np.asarray(values, np.float32)
    if fmt == BF16:
        return oracle.write_bf16(values)
    if fmt == F16:
        return values.astype(np.float16).view(np.uint16)
    return values.copy()


def _oracle(q, kraw, kf, vraw, vf, qh, kvh, d):
    rc, out = oracle.cpu_reference_decode_formats(q, kraw, kf, vraw, vf, qh, kvh, d)
    assert rc == 0
    return out


# ---- the reference's own GPU tests, restated -----------------------------
@pytest.mark.parametrize("fmt", [BF16, F16, F32])
def test_gpu_roundtrip(ctx, fmt):
    # gpu_backend.rs:384-413: geometry (4, 2, 4), 4 tokens, query 0.15.
    qh, kvh, d = 4, 2, 4
    k = (np.arange(32) % 11 - 5).astype(np.float32) * np.float32(0.0625)
    v = (np.arange(32) % 13 - 6).astype(np.float32) * np.float32(0.0625)
    query = np.full(16, 0.15, np.float32)
    kraw, vraw = _encode(k, fmt), _encode(v, fmt)
    cpu = _oracle(query, kraw, fmt, vraw, fmt, qh, kvh, d)
    gpu, timings = ctx.backend_decode(query, kraw.tobytes(), fmt, vraw.tobytes(), fmt, 4, qh, kvh, d)
    assert np.all(np.abs(cpu - gpu) < TOL), (cpu, gpu)
    assert timings.kernel_ms > 0.0
    assert timings.input_kv_bytes == kraw.nbytes + vraw.nbytes
    assert timings.output_bytes == 16 * 4


@pytest.mark.parametrize("qh,kvh", [(4, 4), (4, 1)])
def test_gpu_geometry_roundtrip(ctx, qh, kvh):
    # gpu_backend.rs:415-441: head_dim 8, 5 tokens, F32 frames.
    d, tokens = 8, 5
    count = tokens * kvh * d
    key = ((np.arange(count) % 19) - 9).astype(np.float32) * np.float32(0.0625)
    value = ((np.arange(count) % 17) - 8).astype(np.float32) * np.float32(0.0625)
    query = ((np.arange(qh * d) % 7) - 3).astype(np.float32) * np.float32(0.125)
    cpu = _oracle(query, key, F32, value, F32, qh, kvh, d)
    gpu, _ = ctx.backend_decode(query, key.tobytes(), F32, value.tobytes(), F32, tokens, qh, kvh, d)
    assert np.all(np.abs(cpu - gpu) < TOL)


# ---- portable.rs known answers through the GPU backend --------------------
@pytest.mark.parametrize("qh,kvh", [(2, 2), (4, 2), (8, 1)])
def test_heads_map_to_their_kv_head(ctx, qh, kvh):
    # portable.rs:684-710: zero query returns the mapped kv head's V exactly.
    keys = np.zeros(kvh * 2, np.float32)
    values = np.array([x for h in range(kvh) for x in (h + 1.0, -(h + 1.0))], np.float32)
    out, _ = ctx.backend_decode(np.zeros(qh * 2, np.float32), keys.tobytes(), F32,
                                values.tobytes(), F32, 1, qh, kvh, 2)
    for head in range(qh):
        kv = head // (qh // kvh)
        assert out[head * 2:head * 2 + 2].tolist() == [values[kv * 2], values[kv * 2 + 1]]


def test_extreme_scores_are_stable(ctx):
    # portable.rs:713-727: scores +-1e8 give exactly 3.0.
    keys = np.array([10_000.0, -10_000.0], np.float32)
    values = np.array([3.0, 9.0], np.float32)
    out, _ = ctx.backend_decode(np.array([10_000.0], np.float32), keys.tobytes(), F32,
                                values.tobytes(), F32, 2, 1, 1, 1)
    assert out.tolist() == [3.0]


def test_mixed_formats_across_appended_frames(ctx):
    # portable.rs:729-745: BF16 keys [0, 1], F16 values [1, 2]; two frames.
    key = np.array([0x0000, 0x3F80], np.uint16)
    value = np.array([0x3C00, 0x4000], np.uint16)
    keys, values = np.concatenate([key, key]), np.concatenate([value, value])
    query = np.array([0.5, -0.25, 1.0, 2.0], np.float32)
    cpu = _oracle(query, keys, BF16, values, F16, 2, 1, 2)
    gpu, _ = ctx.backend_decode(query, keys.tobytes(), BF16, values.tobytes(), F16, 2, 2, 1, 2)
    assert np.all(np.abs(cpu - gpu) < TOL)
    zero, _ = ctx.backend_decode(np.zeros(4, np.float32), key.tobytes(), BF16, value.tobytes(), F16,
                                 1, 2, 1, 2)
    assert zero.tolist() == [1.0, 2.0, 1.0, 2.0]


def test_empty_cache_gives_zeros(ctx):
    # gpu_backend.rs:157-159, on both entry points.
    out, _ = ctx.backend_decode(np.ones(8, np.float32), b"", BF16, b"", BF16, 0, 2, 1, 4)
    assert out.tolist() == [0.0] * 8
    q = torch.ones(8, dtype=torch.float32, device="cuda")
    o = torch.full((8,), 7.0, dtype=torch.float32, device="cuda")
    ctx.frames_decode(q, 0, BF16, 0, BF16, o, 0, 2, 1, 4)
    torch.cuda.synchronize()
    assert o.cpu().tolist() == [0.0] * 8


def test_rejections(ctx):
    # gpu_backend.rs:150-156 and portable.rs:807-825.
    kv = np.zeros(2, np.float32).tobytes()
    with pytest.raises(mslim_attn.MslimAttnError) as e:
        ctx.backend_decode(np.array([np.nan, 1.0], np.float32), kv, F32, kv, F32, 1, 1, 1, 2)
    assert e.value.code == mslim_attn.ERR_NONFINITE and "GPU Q" in e.value.details
    with pytest.raises(mslim_attn.MslimAttnError) as e:
        ctx.backend_decode(np.zeros(6, np.float32), kv, F32, kv, F32, 1, 3, 2, 2)
    assert e.value.code == -1
    with pytest.raises(mslim_attn.MslimAttnError) as e:
        ctx.backend_decode(np.zeros(2, np.float32), kv, 4, kv, F32, 1, 1, 1, 2)
    assert e.value.code == -1
    inf_key = np.array([np.inf, 0.0], np.float32).tobytes()
    with pytest.raises(mslim_attn.MslimAttnError) as e:
        ctx.backend_decode(np.ones(2, np.float32), inf_key, F32, kv, F32, 1, 1, 1, 2)
    assert e.value.code == mslim_attn.ERR_NONFINITE and "GPU output" in e.value.details


# ---- exact format decoding ------------------------------------------------
@pytest.mark.parametrize("fmt", [BF16, F16])
def test_every_16_bit_encoding_decodes_exactly(ctx, fmt):
    # One token, zero query: softmax weight 1, so out = V exactly.  64 heads x
    # D = 1024 cover all 65,536 encodings (gpu_attention.cl:5-32 decode rules).
    bits = np.arange(65536, dtype=np.uint16)
    q = torch.zeros(65536, dtype=torch.float32, device="cuda")
    keys = torch.zeros(65536, dtype=torch.int16, device="cuda")
    values = torch.from_numpy(bits.view(np.int16)).cuda()
    out = torch.empty(65536, dtype=torch.float32, device="cuda")
    ctx.frames_decode(q, keys, fmt, values, fmt, out, 1, 64, 64, 1024)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = oracle.read_bf16(bits) if fmt == BF16 else bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite], want[finite])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))


# ---- random shapes, every format pair, split merges -----------------------
@pytest.mark.parametrize("kf", [BF16, F16, F32])
@pytest.mark.parametrize("vf", [BF16, F16, F32])
def test_random_cfg1_shape_all_format_pairs(ctx, kf, vf):
    rng = np.random.default_rng(100 * kf + vf)
    qh, kvh, d, t = 32, 8, 128, 1500  # several splits, ragged last tile
    query = rng.standard_normal(qh * d, dtype=np.float32)
    k = rng.standard_normal(t * kvh * d, dtype=np.float32)
    v = rng.standard_normal(t * kvh * d, dtype=np.float32)
    kraw, vraw = _encode(k, kf), _encode(v, vf)
    cpu = _oracle(query, kraw, kf, vraw, vf, qh, kvh, d)
    gpu, timings = ctx.backend_decode(query, kraw.tobytes(), kf, vraw.tobytes(), vf, t, qh, kvh, d)
    assert np.max(np.abs(cpu - gpu)) < TOL
    assert timings.scratch_bytes > 0  # split-KV partials were used
    # the device entry point runs the same kernels: identical bits
    dev_out = torch.empty(qh * d, dtype=torch.float32, device="cuda")
    ctx.frames_decode(torch.from_numpy(query).cuda(), torch.from_numpy(kraw.view(np.uint8)).cuda(), kf,
                      torch.from_numpy(vraw.view(np.uint8)).cuda(), vf, dev_out, t, qh, kvh, d)
    torch.cuda.synchronize()
    assert np.array_equal(dev_out.cpu().numpy(), gpu)


@pytest.mark.parametrize("qh,kvh,d,t", [(1, 1, 1, 3), (3, 1, 5, 300), (6, 3, 36, 70),
                                        (4, 2, 320, 513), (2, 1, 1024, 40), (64, 8, 128, 4097)])
def test_odd_geometries(ctx, qh, kvh, d, t):
    rng = np.random.default_rng(qh * 7 + d + t)
    query = rng.standard_normal(qh * d, dtype=np.float32) * np.float32(0.5)
    kraw = _encode(rng.standard_normal(t * kvh * d, dtype=np.float32), BF16)
    vraw = _encode(rng.standard_normal(t * kvh * d, dtype=np.float32), F16)
    cpu = _oracle(query, kraw, BF16, vraw, F16, qh, kvh, d)
    gpu, _ = ctx.backend_decode(query, kraw.tobytes(), BF16, vraw.tobytes(), F16, t, qh, kvh, d)
    assert np.max(np.abs(cpu - gpu)) < TOL
