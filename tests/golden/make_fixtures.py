#!/usr/bin/env python3
"""Writes tests/golden/fixtures.json: small input/output vectors for the
attention path, produced by the CPU oracle (oracle/), whose every function
used here is pinned against the reference's known answers and published
vectors (see the oracle's "pin:" notes).  The fixtures freeze those results
so a later change of the oracle or of the product shows up as a diff.

Contents:
  * bf16_encode   -- write_bf16 (gpu_llm.cl:10-21) on rounding ties, NaN
                     payloads, subnormals and overflow;
  * fnv1a64       -- published FNV-1a-64 vectors (cold_store.rs:909-922);
  * sha256        -- FIPS 180-4 vectors (sha2 0.11.1, cold_store.rs:924-930);
  * coldstore_records -- full record bytes (cold_store.rs:269-349) for the
                     reference's own test pages (cold_store.rs:976-985,
                     :1043-1054) and two BF16 pages of device-pool geometry;
  * decode        -- dense_attention_bf16 (native_cpu_adapter.rs:253-307) on
                     a 5-token GQA cache;
  * rmsnorm / rope / swiglu -- the GPU stage forms (gpu_llm.cl:72-146,
                     :225-237);
  * logical_kv_sha256 -- gpu_region_store.rs:341-371 on a 2-layer cache.

Run from the repository root: python tests/golden/make_fixtures.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.json")


def hexs(a) -> str:
    return np.ascontiguousarray(a).view(np.uint8).tobytes().hex()


def bf16_encode():
    bits = [0x00000000, 0x80000000, 0x3F800000, 0xBF800000,
            0x3F808000,  # 1 + 2^-8: tie, even -> 1.0
            0x3F818000,  # 1 + 3*2^-8: tie, odd -> round up
            0x3F80C000, 0x3F804000, 0x7F7FFFFF, 0x7F800000, 0xFF800000,
            0x7FC00001, 0x7F800001, 0xFFA12345, 0x00000001, 0x007FFFFF, 0x80400000,
            0x47EFFFFF, 0x3EAAAAAB]
    f = np.array(bits, np.uint32).view(np.float32)
    enc = oracle.write_bf16(f)
    return [[f"{b:08x}", f"{int(e):04x}"] for b, e in zip(bits, enc)]


def fnv_vectors():
    return [[m.hex(), f"{oracle.fnv1a64(m):016x}"] for m in (b"", b"a", b"foobar")]


def sha_vectors():
    msgs = [b"abc", b"", b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq"]
    return [[m.hex(), oracle.sha256(m).hex()] for m in msgs]


def record(page_id, layer, token_start, tokens, heads, head_dim, tile, key: bytes, value: bytes):
    rec = oracle.coldstore_record(page_id, layer, token_start, tokens, heads, head_dim, tile, key, value)
    return {"page_id": page_id, "layer": layer, "token_start": token_start, "tokens": tokens,
            "heads": heads, "head_dim": head_dim, "tile": tile, "key": key.hex(),
            "value": value.hex(), "record": rec.hex()}


def coldstore_records():
    out = []
    # cold_store.rs:976-985 geometry(0) with the pages of :1008-1010.
    out.append(record(0, 3, 0, 4, 2, 4, 4, bytes([7] * 64), bytes([11] * 64)))
    # cold_store.rs:1047-1053: head/token-tagged rows.
    key = bytes(b for h in range(2) for t in range(4) for b in [100 + h * 10 + t] * 4)
    value = bytes(b for h in range(2) for t in range(4) for b in [h * 10 + t] * 4)
    out.append(record(0, 3, 0, 4, 2, 4, 4, key, value))
    # BF16 pages of device-pool geometry (head_dim a multiple of 8).
    rng = np.random.default_rng(20261201)
    for page_id, tokens in ((5, 4), (6, 1)):
        k = oracle.write_bf16(rng.standard_normal(tokens * 2 * 8, dtype=np.float32))
        v = oracle.write_bf16(rng.standard_normal(tokens * 2 * 8, dtype=np.float32))
        out.append(record(page_id, 1, 4 * page_id, tokens, 2, 8, 1, k.tobytes(), v.tobytes()))
    return out


def decode_case():
    rng = np.random.default_rng(11)
    qh, kvh, d, t = 4, 2, 8, 5
    q = oracle.read_bf16(oracle.write_bf16(rng.standard_normal(qh * d, dtype=np.float32)))
    k = oracle.write_bf16(rng.standard_normal(t * kvh * d, dtype=np.float32))
    v = oracle.write_bf16(rng.standard_normal(t * kvh * d, dtype=np.float32))
    out = oracle.dense_attention_bf16(q, k, v, qh, kvh, d)
    return {"q_heads": qh, "kv_heads": kvh, "head_dim": d, "tokens": t,
            "q_bf16": hexs(oracle.write_bf16(q)), "k_bf16": hexs(k), "v_bf16": hexs(v),
            "out_f32": hexs(out), "tolerance_max_abs": 2e-2}


def feeders():
    rng = np.random.default_rng(12)
    x = oracle.write_bf16(rng.standard_normal(2 * 16, dtype=np.float32) * np.float32(3))
    w = oracle.write_bf16(rng.standard_normal(16, dtype=np.float32) * np.float32(0.02))
    rms = {"tokens": 2, "hidden": 16, "eps": 1e-5, "x": hexs(x), "w": hexs(w),
           "out": hexs(oracle.rmsnorm_gpu(x, w, 2, 16, 1e-5))}
    xr = oracle.write_bf16(rng.standard_normal(2 * 2 * 8, dtype=np.float32))
    rope = []
    for llama3, params in ((0, (1.0, 1.0, 2.0, 1.0)), (1, (8.0, 1.0, 4.0, 8192.0))):
        rope.append({"tokens": 2, "heads": 2, "head_dim": 8, "start": 4090, "theta": 500000.0,
                     "llama3": llama3, "params": list(params), "x": hexs(xr),
                     "out": hexs(oracle.rope_gpu(xr, 2, 2, 8, 4090, 500000.0, llama3, *params))})
    g = oracle.write_bf16(rng.standard_normal(24, dtype=np.float32) * np.float32(4))
    u = oracle.write_bf16(rng.standard_normal(24, dtype=np.float32))
    swi = {"gate": hexs(g), "up": hexs(u), "out": hexs(oracle.swiglu(g, u))}
    return rms, rope, swi


def logical_sha():
    rng = np.random.default_rng(13)
    tokens, kvh, d = 3, 2, 8
    keys = [rng.integers(0, 1 << 16, tokens * kvh * d, dtype=np.uint16) for _ in range(2)]
    values = [rng.integers(0, 1 << 16, tokens * kvh * d, dtype=np.uint16) for _ in range(2)]
    return {"tokens": tokens, "kv_heads": kvh, "head_dim": d,
            "keys": [hexs(k) for k in keys], "values": [hexs(v) for v in values],
            "sha256": oracle.logical_kv_sha256(keys, values, tokens, kvh, d * 2)}


def main():
    rms, rope, swi = feeders()
    fixtures = {
        "generator": "tests/golden/make_fixtures.py (CPU oracle)",
        "bf16_encode": bf16_encode(),
        "fnv1a64": fnv_vectors(),
        "sha256": sha_vectors(),
        "coldstore_records": coldstore_records(),
        "decode": decode_case(),
        "rmsnorm": rms,
        "rope": rope,
        "swiglu": swi,
        "logical_kv_sha256": logical_sha(),
    }
    with open(OUT, "w") as f:
        json.dump(fixtures, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
