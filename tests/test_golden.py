"""The committed fixtures (tests/golden/fixtures.json, written by
tests/golden/make_fixtures.py) against the CPU oracle: any change of an
oracle function's output shows up here.  The GPU product is checked against
the same fixtures in tests/test_gpu_golden.py, the C++ ColdStore in
tests/cpp/store_tests.cpp (cold_golden_fixture_records)."""
import json
import os

import numpy as np
import pytest

import oracle

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.json")


@pytest.fixture(scope="module")
def fx():
    with open(FIXTURES) as f:
        return json.load(f)


def u16(h):
    return np.frombuffer(bytes.fromhex(h), np.uint16)


def test_bf16_encode(fx):
    for f_hex, b_hex in fx["bf16_encode"]:
        f = np.array([int(f_hex, 16)], np.uint32).view(np.float32)
        assert int(oracle.write_bf16(f)[0]) == int(b_hex, 16), f_hex


def test_fnv_and_sha_vectors(fx):
    for m, h in fx["fnv1a64"]:
        assert f"{oracle.fnv1a64(bytes.fromhex(m)):016x}" == h
    for m, h in fx["sha256"]:
        assert oracle.sha256(bytes.fromhex(m)).hex() == h
    # the published values themselves
    assert dict(fx["fnv1a64"])["61"] == "af63dc4c8601ec8c"
    assert dict(fx["sha256"])["616263"].startswith("ba7816bf")


def test_coldstore_records(fx):
    recs = fx["coldstore_records"]
    # cold_store.rs:1141-1144 known answer, scaled to 64-byte payloads.
    assert len(bytes.fromhex(recs[0]["record"])) == 104 + 4 * 8 * 2 + 64 + 64 + 56
    for r in recs:
        got = oracle.coldstore_record(r["page_id"], r["layer"], r["token_start"], r["tokens"], r["heads"],
                                      r["head_dim"], r["tile"], bytes.fromhex(r["key"]), bytes.fromhex(r["value"]))
        assert got.hex() == r["record"]


def test_decode(fx):
    c = fx["decode"]
    q = oracle.read_bf16(u16(c["q_bf16"]))
    out = oracle.dense_attention_bf16(q, u16(c["k_bf16"]), u16(c["v_bf16"]), c["q_heads"], c["kv_heads"],
                                      c["head_dim"])
    assert out.tobytes().hex() == c["out_f32"]


def test_feeders(fx):
    r = fx["rmsnorm"]
    assert oracle.rmsnorm_gpu(u16(r["x"]), u16(r["w"]), r["tokens"], r["hidden"], r["eps"]).tobytes().hex() == r["out"]
    for c in fx["rope"]:
        got = oracle.rope_gpu(u16(c["x"]), c["tokens"], c["heads"], c["head_dim"], c["start"], c["theta"],
                              c["llama3"], *c["params"])
        assert got.tobytes().hex() == c["out"]
    s = fx["swiglu"]
    assert oracle.swiglu(u16(s["gate"]), u16(s["up"])).tobytes().hex() == s["out"]


def test_logical_sha(fx):
    c = fx["logical_kv_sha256"]
    keys = [u16(h) for h in c["keys"]]
    values = [u16(h) for h in c["values"]]
    assert oracle.logical_kv_sha256(keys, values, c["tokens"], c["kv_heads"], c["head_dim"] * 2) == c["sha256"]
