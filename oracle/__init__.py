"""CPU oracle for the M-SLIM attention hot path -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes wrapper over ``oracle/_build/liboracle.so`` (built from
``oracle/oracle.c`` by ``oracle/Makefile``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker: the product path never calls it.

Each wrapper names the reference file:line of the algorithm it restates; the
C header ``oracle/oracle.h`` records how each function is pinned.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = C.CDLL(_LIB_PATH)
    P = C.c_void_p
    I = C.c_int
    U32 = C.c_uint32
    U64 = C.c_uint64
    SZ = C.c_size_t
    F = C.c_float
    sigs = {
        "orc_read_bf16": (F, [C.c_uint16]),
        "orc_write_bf16": (C.c_uint16, [F]),
        "orc_half_bf16_from_f32": (C.c_uint16, [F]),
        "orc_bf16_round_independent": (C.c_uint16, [F]),
        "orc_bf16_encoder_mismatches": (U64, [U64, U64]),
        "orc_bf16_to_f32_array": (None, [P, P, SZ]),
        "orc_f32_to_bf16_array": (None, [P, P, SZ]),
        "orc_dense_attention_bf16": (I, [I, I, I, P, P, P, I, P]),
        "orc_cpu_reference_decode": (I, [I, I, I, P, P, P, I, I, P]),
        "orc_cpu_reference_decode_formats": (I, [I, I, I, P, P, I, P, I, I, P]),
        "orc_prefill_causal_cpu": (I, [I, I, I, P, P, P, I, I, P]),
        "orc_gpu_reference_attention": (I, [I, I, I, P, P, P, I, I, P]),
        "orc_rms_norm_cpu": (None, [P, P, I, F, P]),
        "orc_rmsnorm_gpu": (None, [P, P, I, I, F, P]),
        "orc_rope_inverse_frequency": (F, [I, I, F, I, F, F, F, F]),
        "orc_rope_gpu": (None, [P, P, I, I, I, I, F, I, F, F, F, F]),
        "orc_rope_cpu": (None, [P, I, I, I, F]),
        "orc_swiglu": (None, [P, P, SZ, P]),
        "orc_matmul_bf16": (None, [P, P, I, I, I, P]),
        "orc_matvec_cpu": (None, [P, P, I, I, P]),
        "orc_argmax_total_last": (C.c_int32, [P, I]),
        "orc_add_bf16": (None, [P, P, SZ, P]),
        "orc_argmax_bf16": (None, [P, I, I, P]),
        "orc_softmax": (None, [P, I]),
        "orc_fnv1a64": (U64, [P, SZ, U64]),
        "orc_sha256": (None, [P, SZ, P]),
        "orc_token_hashes": (I, [P, SZ, U32, U32, P]),
        "orc_coldstore_record": (SZ, [U64, U32, U64, U32, U32, U32, U32, P, SZ, P, SZ, P, SZ]),
        "orc_token_to_head_major": (None, [P, U32, U32, U32, P]),
        "orc_gather_token_major": (None, [P, SZ, U32, U32, U32, P, P, P, SZ, P]),
        "orc_logical_kv_sha256": (None, [U32, U64, U32, U32, P, P, P]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- BF16 codec (gpu_llm.cl:7-21; half 2.7.1 bf16::from_f32) -------------
def write_bf16(x) -> np.ndarray:
    """f32 -> BF16 bits, round-to-nearest-even, NaN quieted (gpu_llm.cl:10-21)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def read_bf16(bits) -> np.ndarray:
    """BF16 bits -> f32 (gpu_llm.cl:7-9)."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_bf16_to_f32_array(_p(bits), _p(out), bits.size)
    return out


def round_bf16(x) -> np.ndarray:
    return read_bf16(write_bf16(x))


def bf16_encoder_mismatches(start: int, count: int) -> int:
    return int(lib().orc_bf16_encoder_mismatches(start, count))


# ---- Attention -----------------------------------------------------------
def dense_attention_bf16(q: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray,
                         qh: int, kvh: int, d: int) -> np.ndarray:
    """native_cpu_adapter.rs:253-307; q f32 [QH*D], K/V BF16 [T][KVH][D]."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    k_bits = np.ascontiguousarray(k_bits, np.uint16)
    v_bits = np.ascontiguousarray(v_bits, np.uint16)
    tokens = k_bits.size // (kvh * d)
    out = np.empty(qh * d, np.float32)
    rc = lib().orc_dense_attention_bf16(qh, kvh, d, _p(q), _p(k_bits), _p(v_bits), tokens, _p(out))
    if rc:
        raise ValueError("dense_attention_bf16 rejected its geometry")
    return out


def cpu_reference_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, dtype: int,
                         qh: int, kvh: int, d: int):
    """portable.rs:575-646; returns (rc, out).  dtype 1=BF16, 2=F16, 3=F32."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    tokens = k.size // (kvh * d)
    out = np.empty(qh * d, np.float32)
    rc = lib().orc_cpu_reference_decode(qh, kvh, d, _p(q), _p(k), _p(v), dtype, tokens, _p(out))
    return rc, out


def cpu_reference_decode_formats(q: np.ndarray, k: np.ndarray, key_dtype: int, v: np.ndarray,
                                 value_dtype: int, qh: int, kvh: int, d: int):
    """portable.rs:575-646 with separate K and V formats; returns (rc, out)."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    tokens = k.size // (kvh * d)
    out = np.empty(qh * d, np.float32)
    rc = lib().orc_cpu_reference_decode_formats(qh, kvh, d, _p(q), _p(k), key_dtype, _p(v),
                                                value_dtype, tokens, _p(out))
    return rc, out


def prefill_causal_cpu(q: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray,
                       qh: int, kvh: int, d: int, queries: int, prior: int) -> np.ndarray:
    """Row i attends keys 0..prior+i with dense_attention_bf16
    (native_cpu_adapter.rs:486-534 processes prompts token by token)."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    k_bits = np.ascontiguousarray(k_bits, np.uint16)
    v_bits = np.ascontiguousarray(v_bits, np.uint16)
    out = np.empty(queries * qh * d, np.float32)
    rc = lib().orc_prefill_causal_cpu(qh, kvh, d, _p(q), _p(k_bits), _p(v_bits), queries, prior, _p(out))
    if rc:
        raise ValueError("prefill_causal_cpu rejected its geometry")
    return out


def gpu_reference_attention(q_bits, k_bits, v_bits, qh, kvh, d, queries, prior) -> np.ndarray:
    """gpu_llm.cl:150-212 / :462-541 three-kernel arithmetic; BF16 bits out."""
    q_bits = np.ascontiguousarray(q_bits, np.uint16)
    k_bits = np.ascontiguousarray(k_bits, np.uint16)
    v_bits = np.ascontiguousarray(v_bits, np.uint16)
    out = np.empty(queries * qh * d, np.uint16)
    rc = lib().orc_gpu_reference_attention(qh, kvh, d, _p(q_bits), _p(k_bits), _p(v_bits),
                                           queries, prior, _p(out))
    if rc:
        raise ValueError("gpu_reference_attention rejected its geometry")
    return out


def softmax(x) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().orc_softmax(_p(x), x.size)
    return x


# ---- Feeders -------------------------------------------------------------
def rms_norm_cpu(x, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm_cpu(_p(x), _p(w), x.size, eps, _p(out))
    return out


def rmsnorm_gpu(x_bits, w_bits, tokens: int, hidden: int, eps: float) -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    w_bits = np.ascontiguousarray(w_bits, np.uint16)
    out = np.empty(tokens * hidden, np.uint16)
    lib().orc_rmsnorm_gpu(_p(x_bits), _p(w_bits), tokens, hidden, eps, _p(out))
    return out


def rope_inverse_frequency(fd: int, head_dim: int, theta: float, llama3: int = 0,
                           factor: float = 1.0, low: float = 1.0, high: float = 2.0,
                           original_max: float = 1.0) -> float:
    return float(lib().orc_rope_inverse_frequency(fd, head_dim, theta, llama3, factor, low,
                                                  high, original_max))


def rope_gpu(x_bits, tokens, heads, head_dim, start, theta, llama3=0, factor=1.0,
             low=1.0, high=2.0, original_max=1.0) -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    out = np.empty(tokens * heads * head_dim, np.uint16)
    lib().orc_rope_gpu(_p(x_bits), _p(out), tokens, heads, head_dim, start, theta, llama3,
                       factor, low, high, original_max)
    return out


def rope_cpu(values, heads: int, dim: int, position: int, theta: float) -> np.ndarray:
    v = np.array(values, np.float32)
    lib().orc_rope_cpu(_p(v), heads, dim, position, theta)
    return v


def swiglu(gate_bits, up_bits) -> np.ndarray:
    g = np.ascontiguousarray(gate_bits, np.uint16)
    u = np.ascontiguousarray(up_bits, np.uint16)
    out = np.empty(g.size, np.uint16)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def add_bf16(a_bits, b_bits) -> np.ndarray:
    """gpu_llm.cl:214-222 llm_add: BF16(a + b)."""
    a = np.ascontiguousarray(a_bits, np.uint16).reshape(-1)
    b = np.ascontiguousarray(b_bits, np.uint16).reshape(-1)
    out = np.empty(a.size, np.uint16)
    lib().orc_add_bf16(_p(a), _p(b), a.size, _p(out))
    return out


def argmax_bf16(logits_bits, rows: int, vocab: int) -> np.ndarray:
    """gpu_llm.cl:239-270 llm_argmax per row: int32 [rows]."""
    x = np.ascontiguousarray(logits_bits, np.uint16).reshape(-1)
    out = np.empty(rows, np.int32)
    lib().orc_argmax_bf16(_p(x), rows, vocab, _p(out))
    return out


def embed_rows(table_bits, ids, hidden: int) -> np.ndarray:
    """gpu_llm.cl:24-33 llm_embed, one row per id: [len(ids)][hidden] bits."""
    table = np.ascontiguousarray(table_bits, np.uint16).reshape(-1, hidden)
    return table[np.asarray(ids, np.int64)].copy()


def matmul_bf16(w_bits, in_bits, inner: int, rows: int, tokens: int) -> np.ndarray:
    """hipblaslt_bridge.cpp:203-233 product: BF16 bits out [tokens][rows]."""
    w = np.ascontiguousarray(w_bits, np.uint16)
    x = np.ascontiguousarray(in_bits, np.uint16)
    out = np.empty(tokens * rows, np.uint16)
    lib().orc_matmul_bf16(_p(w), _p(x), inner, rows, tokens, _p(out))
    return out


def matvec_cpu(w_bits, x, rows: int, cols: int) -> np.ndarray:
    """native_cpu_adapter.rs:129-150: f32 [rows], each a left-to-right f32 sum
    of BF16 weight x f32 input products (no FMA), rounded to BF16."""
    w = np.ascontiguousarray(w_bits, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    assert w.size == rows * cols and x.size == cols
    out = np.empty(rows, np.float32)
    lib().orc_matvec_cpu(_p(w), _p(x), rows, cols, _p(out))
    return out


def argmax_total_last(logits) -> int:
    """native_cpu_adapter.rs:577-582: the last maximum under f32 total order."""
    x = np.ascontiguousarray(logits, np.float32).reshape(-1)
    return int(lib().orc_argmax_total_last(_p(x), x.size))


# ---- Integrity -----------------------------------------------------------
FNV_OFFSET = 0xCBF29CE484222325


def fnv1a64(data: bytes, state: int = FNV_OFFSET) -> int:
    buf = np.frombuffer(bytes(data), np.uint8) if data else np.zeros(1, np.uint8)
    return int(lib().orc_fnv1a64(_p(np.ascontiguousarray(buf)), len(data), state))


def sha256(data: bytes) -> bytes:
    buf = np.frombuffer(bytes(data), np.uint8) if data else np.zeros(1, np.uint8)
    out = np.zeros(32, np.uint8)
    lib().orc_sha256(_p(np.ascontiguousarray(buf)), len(data), _p(out))
    return out.tobytes()


def coldstore_record(page_id: int, layer: int, token_start: int, tokens: int, heads: int,
                     head_dim: int, tile: int, key: bytes, value: bytes) -> bytes:
    """cold_store.rs:269-349 record bytes (header, hash tables, payloads, footer)."""
    k = np.frombuffer(bytes(key), np.uint8)
    v = np.frombuffer(bytes(value), np.uint8)
    size = lib().orc_coldstore_record(page_id, layer, token_start, tokens, heads, head_dim, tile,
                                      _p(k), k.size, _p(v), v.size, None, 0)
    if size == 0:
        raise ValueError("invalid ColdStore page geometry")
    out = np.zeros(size, np.uint8)
    lib().orc_coldstore_record(page_id, layer, token_start, tokens, heads, head_dim, tile,
                               _p(k), k.size, _p(v), v.size, _p(out), size)
    return out.tobytes()


def token_to_head_major(token_major: np.ndarray, n: int, kvh: int, row_bytes: int) -> np.ndarray:
    tm = np.ascontiguousarray(token_major).view(np.uint8).reshape(-1)
    out = np.empty_like(tm)
    lib().orc_token_to_head_major(_p(tm), n, kvh, row_bytes, _p(out))
    return out


def gather_token_major(pool: np.ndarray, page_tokens: int, kvh: int, row_bytes: int,
                       page_of: np.ndarray, offset_of: np.ndarray,
                       positions: np.ndarray) -> np.ndarray:
    """gpu_region_store.rs:828-927: gather token-major rows through a page table."""
    pool = np.ascontiguousarray(pool).view(np.uint8).reshape(-1)
    page_of = np.ascontiguousarray(page_of, np.uint32)
    offset_of = np.ascontiguousarray(offset_of, np.uint32)
    positions = np.ascontiguousarray(positions, np.uint32)
    page_bytes = page_tokens * kvh * row_bytes
    out = np.empty(positions.size * kvh * row_bytes, np.uint8)
    lib().orc_gather_token_major(_p(pool), page_bytes, page_tokens, kvh, row_bytes, _p(page_of),
                                 _p(offset_of), _p(positions), positions.size, _p(out))
    return out


def logical_kv_sha256(keys: list, values: list, tokens: int, kvh: int, row_bytes: int) -> str:
    """gpu_region_store.rs:341-371 / gpu_llm/mod.rs:1981-2028 from token-major layers."""
    ks = [np.ascontiguousarray(k).view(np.uint8).reshape(-1) for k in keys]
    vs = [np.ascontiguousarray(v).view(np.uint8).reshape(-1) for v in values]
    kp = (C.c_void_p * len(ks))(*[_p(k) for k in ks])
    vp = (C.c_void_p * len(vs))(*[_p(v) for v in vs])
    out = np.zeros(32, np.uint8)
    lib().orc_logical_kv_sha256(len(ks), tokens, kvh, row_bytes, kp, vp, _p(out))
    return out.tobytes().hex()
