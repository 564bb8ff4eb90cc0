"""The gfx950 product against the committed fixtures
(tests/golden/fixtures.json): decode within the stated tolerance, feeders,
record frames and the logical K/V digest bit for bit."""
import json
import os

import numpy as np
import pytest
import torch

import mslim_attn

pytestmark = pytest.mark.gpu

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.json")


@pytest.fixture(scope="module")
def fx():
    with open(FIXTURES) as f:
        return json.load(f)


def dev16(h):
    return torch.from_numpy(np.frombuffer(bytes.fromhex(h), np.int16).copy()).cuda()


def hex_of(t):
    return t.cpu().numpy().tobytes().hex()


def test_decode_fixture(ctx, fx):
    c = fx["decode"]
    qh, kvh, d, t = c["q_heads"], c["kv_heads"], c["head_dim"], c["tokens"]
    q, k, v = dev16(c["q_bf16"]), dev16(c["k_bf16"]), dev16(c["v_bf16"])
    out = torch.empty_like(q)
    ctx.decode_dense(q, k, v, out, [t], qh, kvh, d, seq_stride_tokens=t)
    torch.cuda.synchronize()
    got = (out.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    want = np.frombuffer(bytes.fromhex(c["out_f32"]), np.float32)
    assert np.max(np.abs(got.astype(np.float64) - want)) <= c["tolerance_max_abs"]


def test_feeder_fixtures(ctx, fx):
    r = fx["rmsnorm"]
    out = torch.empty(r["tokens"] * r["hidden"], dtype=torch.int16, device="cuda")
    ctx.rmsnorm(dev16(r["x"]), dev16(r["w"]), out, r["tokens"], r["hidden"], r["eps"])
    torch.cuda.synchronize()
    assert hex_of(out) == r["out"]
    for c in fx["rope"]:
        x = dev16(c["x"])
        out = torch.empty_like(x)
        ctx.rope(x, out, c["tokens"], c["heads"], c["head_dim"], c["start"], c["theta"], c["llama3"], *c["params"])
        torch.cuda.synchronize()
        assert hex_of(out) == c["out"]
    s = fx["swiglu"]
    g = dev16(s["gate"])
    out = torch.empty_like(g)
    ctx.swiglu(g, dev16(s["up"]), out, g.numel())
    torch.cuda.synchronize()
    assert hex_of(out) == s["out"]


def test_record_frame_fixtures(ctx, fx):
    """BF16 pages of device geometry: a pool of 4-token pages holds each
    record's payload, and frame prefix | payloads | footer == the fixture."""
    recs = [r for r in fx["coldstore_records"] if r["head_dim"] % 8 == 0]
    assert len(recs) == 2
    page_tokens = 4
    for r in recs:
        heads, dim, tokens = r["heads"], r["head_dim"], r["tokens"]
        pool = []
        for part in ("key", "value"):
            payload = np.frombuffer(bytes.fromhex(r[part]), np.uint16).reshape(heads, tokens, dim)
            page = np.zeros((1, heads, page_tokens, dim), np.uint16)
            page[0, :, :tokens, :] = payload
            pool.append(torch.from_numpy(page.view(np.int16).reshape(-1).copy()).cuda())
        rec = mslim_attn.PageRecord(r["page_id"], r["token_start"], r["layer"], tokens, 0, 0)
        rec_dev = torch.frombuffer(bytearray(bytes(rec)), dtype=torch.uint8).cuda()
        slot = mslim_attn.Context.record_frame_bytes(page_tokens)
        frames = torch.zeros(slot, dtype=torch.uint8, device="cuda")
        ctx.record_frames(pool[0], pool[1], 1, page_tokens, heads, dim, r["tile"], rec_dev, 1, frames)
        torch.cuda.synchronize()
        f = frames.cpu().numpy().tobytes()
        got = f[:104 + 16 * tokens] + bytes.fromhex(r["key"]) + bytes.fromhex(r["value"]) + f[-56:]
        assert got.hex() == r["record"]


def test_logical_sha_fixture(ctx, fx):
    c = fx["logical_kv_sha256"]
    keys = [dev16(h) for h in c["keys"]]
    values = [dev16(h) for h in c["values"]]
    assert ctx.logical_kv_sha256(keys, values, c["tokens"], c["kv_heads"], c["head_dim"]) == c["sha256"]
