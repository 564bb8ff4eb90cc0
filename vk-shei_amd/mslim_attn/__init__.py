"""Python binding of libmslim_attn, the gfx950 attention hot path of M-SLIM.

The library is a C ABI (``include/mslim_attn.h``); this module binds it with
ctypes the way ``native_hip.rs`` binds the reference bridge with libloading:
fixed in-tree path, every symbol resolved up front, a context handle, and
failures turned into exceptions carrying ``"{stage} failed: code={code}:
{details}"`` (native_hip.rs:38-49).

PyTorch is used only as plumbing: tensors provide device memory and the current
HIP stream.  There is no CPU or torch fallback: if the library is missing or
the device is not gfx950 the calls raise.
"""
from __future__ import annotations

import ctypes as C
import math
import os
from typing import Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmslim_attn.so")

MAX_BATCH = 4096  # MSLIM_ATTN_MAX_BATCH; launches above 64 sequences copy their tables to the device
OPT_DECODE_MERGE = 1                        # mslim_attn_ctx_set_option options
DECODE_MERGE_FUSED, DECODE_MERGE_SEPARATE = 0, 1
OPT_PREFILL_SPLIT = 2
OPT_PREFILL_POOL = 3
DECODE_STATIC_SCRATCH_BYTES = 16 << 20      # mslim_attn_decode_paged_noalloc partials bound
FORMAT_BF16, FORMAT_F16, FORMAT_F32 = 1, 2, 3  # gpu_backend.rs:258-262
ERR_NONFINITE = -2


class DeviceInfo(C.Structure):
    """mslim_attn_device_info (GpuDeviceInfo, gpu_backend.rs:21-32)."""
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("vendor", C.c_char * 64),
                ("driver_version", C.c_int), ("compute_units", C.c_uint32),
                ("global_memory_bytes", C.c_uint64), ("max_allocation_bytes", C.c_uint64),
                ("lds_bytes_per_workgroup", C.c_uint32), ("max_clock_mhz", C.c_uint32),
                ("memory_clock_mhz", C.c_uint32), ("memory_bus_bits", C.c_uint32)]


class Timings(C.Structure):
    """mslim_attn_timings (GpuTimings, gpu_backend.rs:34-44)."""
    _fields_ = [("dispatch_ms", C.c_double), ("kernel_ms", C.c_double),
                ("input_kv_bytes", C.c_uint64), ("scratch_bytes", C.c_uint64),
                ("output_bytes", C.c_uint64)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}

EXPORTS = (
    "mslim_attn_last_error",
    "mslim_attn_ctx_new",
    "mslim_attn_ctx_destroy",
    "mslim_attn_get_device_info",
    "mslim_attn_check_bf16_encoding",
    "mslim_attn_ctx_set_stream",
    "mslim_attn_ctx_set_option",
    "mslim_attn_synchronize",
    "mslim_attn_buf_alloc",
    "mslim_attn_host_alloc",
    "mslim_attn_host_free",
    "mslim_attn_buf_upload",
    "mslim_attn_buf_free",
    "mslim_attn_buf_read",
    "mslim_attn_buf_write",
    "mslim_attn_decode_auto_split",
    "mslim_attn_decode_dense",
    "mslim_attn_decode_paged",
    "mslim_attn_decode_paged_noalloc",
    "mslim_attn_prefill_causal",
    "mslim_attn_prefill_split_tiles",
    "mslim_attn_prefill_pool_items",
    "mslim_attn_frames_decode",
    "mslim_attn_backend_decode",
    "mslim_attn_rmsnorm",
    "mslim_attn_rope",
    "mslim_attn_rope_rows",
    "mslim_attn_rope_qk",
    "mslim_attn_swiglu",
    "mslim_attn_pages_write",
    "mslim_attn_pages_append",
    "mslim_attn_rope_append",
    "mslim_attn_pages_gather",
    "mslim_attn_logical_kv_sha256",
    "mslim_attn_record_frame_bytes",
    "mslim_attn_record_frames",
    "mslim_attn_record_frames_staged",
    "mslim_attn_record_payloads",
    "mslim_attn_matrix_multiply",
    "mslim_attn_gemm_bf16",
    "mslim_attn_gemm_bf16_add",
    "mslim_attn_gemm_swiglu",
    "mslim_attn_gemm_qkv",
    "mslim_attn_rmsnorm_gemm_bf16",
    "mslim_attn_rmsnorm_gemm_qkv",
    "mslim_attn_rmsnorm_gemm_swiglu",
    "mslim_attn_rmsnorm_qkv_rope_append",
    "mslim_attn_add",
    "mslim_attn_embed",
    "mslim_attn_argmax",
)

RECORD_HEADER_BYTES = 104  # cold_store.rs:23
RECORD_FOOTER_BYTES = 56   # cold_store.rs:24


class PageRecord(C.Structure):
    """mslim_attn_page_record: header fields of one record and its pool page."""
    _fields_ = [("page_id", C.c_uint64), ("token_start", C.c_uint64), ("layer", C.c_uint32),
                ("tokens", C.c_uint32), ("pool_page", C.c_int32), ("first_row", C.c_uint32)]


class MslimAttnError(RuntimeError):
    def __init__(self, stage: str, code: int, details: str):
        super().__init__(f"{stage} failed: code={code}: {details}")
        self.stage = stage
        self.code = code
        self.details = details


class LibraryMissing(MslimAttnError):
    pass


_lib: Optional[C.CDLL] = None


def library() -> C.CDLL:
    """Load the in-tree libmslim_attn.so and declare every exported symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing("load libmslim_attn", -1,
                             f"{LIB_PATH} is not built (run __graft_entry__.build())")
    lib = C.CDLL(LIB_PATH)
    P, I, SZ, F, I64 = C.c_void_p, C.c_int, C.c_size_t, C.c_float, C.c_int64
    PI32 = C.POINTER(C.c_int32)
    sigs = {
        "mslim_attn_last_error": (C.c_char_p, []),
        "mslim_attn_ctx_new": (P, []),
        "mslim_attn_ctx_destroy": (None, [P]),
        "mslim_attn_get_device_info": (I, [P, C.POINTER(DeviceInfo)]),
        "mslim_attn_check_bf16_encoding": (I, [P, C.POINTER(C.c_uint64)]),
        "mslim_attn_ctx_set_stream": (I, [P, P]),
        "mslim_attn_ctx_set_option": (I, [P, I, I64]),
        "mslim_attn_synchronize": (I, [P]),
        "mslim_attn_buf_alloc": (P, [P, SZ]),
        "mslim_attn_host_alloc": (P, [P, SZ]),
        "mslim_attn_host_free": (I, [P, P]),
        "mslim_attn_buf_upload": (P, [P, P, SZ]),
        "mslim_attn_buf_free": (I, [P, P]),
        "mslim_attn_buf_read": (I, [P, P, SZ, P, SZ]),
        "mslim_attn_buf_write": (I, [P, P, SZ, P, SZ]),
        "mslim_attn_decode_auto_split": (I, [C.POINTER(C.c_int32), I, I]),
        "mslim_attn_decode_dense": (I, [P, P, P, P, P, I, PI32, I64, I, I, I, F, I]),
        "mslim_attn_decode_paged": (I, [P, P, P, P, P, I, PI32, P, I, I, I, I, I, F, I]),
        "mslim_attn_decode_paged_noalloc": (I, [P, P, P, P, P, I, PI32, P, I, I, I, I, I, F, I]),
        "mslim_attn_prefill_causal": (I, [P, P, P, P, P, I, I, I, I, I, F]),
        "mslim_attn_prefill_split_tiles": (I, [I, I, I, I, I]),
        "mslim_attn_prefill_pool_items": (I, [I, I, I, I, I]),
        "mslim_attn_frames_decode": (I, [P, P, P, I, P, I, P, I64, I, I, I]),
        "mslim_attn_backend_decode": (I, [P, P, P, I, P, I, I64, I, I, I, P, C.POINTER(Timings)]),
        "mslim_attn_rmsnorm": (I, [P, P, P, P, I, I, F]),
        "mslim_attn_rope": (I, [P, P, P, I, I, I, I, F, I, F, F, F, F]),
        "mslim_attn_rope_rows": (I, [P, P, P, I, I, I, P, F, I, F, F, F, F]),
        "mslim_attn_rope_qk": (I, [P, P, P, P, P, I, I, I, I, I, F, I, F, F, F, F]),
        "mslim_attn_swiglu": (I, [P, P, P, P, SZ]),
        "mslim_attn_pages_write": (I, [P, P, P, P, I, I, I, I64, I64, P, P]),
        "mslim_attn_pages_append": (I, [P, P, P, P, I, I, I, I, I, P, P, P]),
        "mslim_attn_rope_append": (I, [P, P, P, P, P, P, P, P, I, I, I, P, I, I, I, F, I, F, F, F, F]),
        "mslim_attn_pages_gather": (I, [P, P, P, I, I, I, I64, I64, P]),
        "mslim_attn_logical_kv_sha256": (I, [P, I, I64, I, I, P, P, P, I, C.c_char_p]),
        "mslim_attn_record_frame_bytes": (I64, [I]),
        "mslim_attn_record_frames": (I, [P, P, P, I64, I, I, I, C.c_uint32, P, I, P]),
        "mslim_attn_record_frames_staged": (I, [P, P, P, I, I, I, C.c_uint32, P, I, P]),
        "mslim_attn_record_payloads": (I, [P, P, P, I64, I, I, I, P, I, P, P, I]),
        "mslim_attn_matrix_multiply": (I, [P, P, P, P, I, I, I]),
        "mslim_attn_gemm_bf16": (I, [P, P, P, P, I, I, I]),
        "mslim_attn_gemm_bf16_add": (I, [P, P, P, P, P, I, I, I]),
        "mslim_attn_gemm_swiglu": (I, [P, P, P, P, P, I, I, I]),
        "mslim_attn_gemm_qkv": (I, [P, P, P, P, P, P, P, P, I, I, I, I]),
        "mslim_attn_rmsnorm_gemm_bf16": (I, [P, P, F, P, P, P, I, I, I]),
        "mslim_attn_rmsnorm_gemm_qkv": (I, [P, P, F, P, P, P, P, P, P, P, I, I, I, I]),
        "mslim_attn_rmsnorm_gemm_swiglu": (I, [P, P, F, P, P, P, P, I, I, I]),
        "mslim_attn_rmsnorm_qkv_rope_append": (I, [P, P, F, P, P, P, P, P, P, P, P, I, I, I, P, I, I, I, I, F, I, F,
                                                   F, F, F]),
        "mslim_attn_add": (I, [P, P, P, P, SZ]),
        "mslim_attn_embed": (I, [P, P, I, I, P, I, P, P]),
        "mslim_attn_argmax": (I, [P, P, I, I, P]),
    }
    for name in EXPORTS:
        res, args = sigs[name]
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = library().mslim_attn_last_error()
    return msg.decode("utf-8", "replace") if msg else "native error unavailable"


def _ptr(t) -> int:
    """Device pointer of a torch tensor (or an int that already is one)."""
    if isinstance(t, int):
        return t
    if t is None:
        return 0
    if not t.is_contiguous():
        raise ValueError("mslim_attn needs contiguous tensors")
    return t.data_ptr()


def _lens(seq_lens: Sequence[int]):
    arr = (C.c_int32 * len(seq_lens))(*[int(x) for x in seq_lens])
    return arr


def default_scale(head_dim: int) -> float:
    """f32 1/sqrt(D) as the reference computes it (native_cpu_adapter.rs:235-237)."""
    import numpy as np
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


class Context:
    """A gfx950 context: owns the split-KV workspace and a HIP stream."""

    def __init__(self, stream: Optional[int] = None):
        lib = library()
        handle = lib.mslim_attn_ctx_new()
        if not handle:
            raise MslimAttnError("mslim_attn_ctx_new", 0, last_error())
        self._h = handle
        self._lib = lib
        if stream is not None:
            self.set_stream(stream)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.mslim_attn_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, stage: str, rc: int) -> None:
        if rc != 0:
            raise MslimAttnError(stage, rc, last_error())

    @property
    def handle(self) -> int:
        return self._h

    def set_stream(self, stream: Optional[int]) -> None:
        """Run on HIP stream `stream` (0 or None is the null stream)."""
        self._check("set_stream", self._lib.mslim_attn_ctx_set_stream(self._h, stream or None))

    def set_option(self, option: int, value: int) -> None:
        self._check("set_option", self._lib.mslim_attn_ctx_set_option(self._h, option, value))

    def set_decode_merge(self, separate: bool) -> None:
        """Merge decode split partials in a second launch (True) or in the
        last workgroup of each (sequence, kv head) (False, the default)."""
        self.set_option(OPT_DECODE_MERGE, DECODE_MERGE_SEPARATE if separate else DECODE_MERGE_FUSED)

    def set_prefill_split(self, allowed: bool) -> None:
        """Let prefill split long row blocks on small launches (True, the
        default) or never (False)."""
        self.set_option(OPT_PREFILL_SPLIT, 1 if allowed else 0)

    def set_prefill_pool(self, allowed: bool) -> None:
        """Let unsplit prefill launches hand their shortest row blocks out at
        run time (True, the default) or map them statically (False); the
        output is the same bits either way."""
        self.set_option(OPT_PREFILL_POOL, 1 if allowed else 0)

    def use_torch_stream(self) -> None:
        import torch
        self.set_stream(torch.cuda.current_stream().cuda_stream)

    def device_info(self) -> dict:
        info = DeviceInfo()
        self._check("device_info", self._lib.mslim_attn_get_device_info(self._h, C.byref(info)))
        return {name: (getattr(info, name).decode() if isinstance(getattr(info, name), bytes)
                       else getattr(info, name)) for name, _ in DeviceInfo._fields_}

    def check_bf16_encoding(self) -> int:
        """Encodings (of all 2^32 f32) where the device's BF16 encoder differs from the rule."""
        n = C.c_uint64(0)
        self._check("check_bf16_encoding", self._lib.mslim_attn_check_bf16_encoding(self._h, C.byref(n)))
        return int(n.value)

    def synchronize(self) -> None:
        self._check("synchronize", self._lib.mslim_attn_synchronize(self._h))

    # ---- attention -----------------------------------------------------
    # ---- Device buffers (tv_hip_load_weight / free_weight / read_weight) ----
    def buf_upload(self, data: bytes) -> int:
        """Allocate a device buffer holding `data`; returns its device pointer."""
        buf = C.create_string_buffer(bytes(data), len(data))
        ptr = self._lib.mslim_attn_buf_upload(self._h, C.addressof(buf), len(data))
        if not ptr:
            raise MslimAttnError("buf_upload", -1, last_error())
        return int(ptr)

    def buf_alloc(self, nbytes: int) -> int:
        ptr = self._lib.mslim_attn_buf_alloc(self._h, nbytes)
        if not ptr:
            raise MslimAttnError("buf_alloc", -1, last_error())
        return int(ptr)

    def buf_free(self, ptr: int) -> None:
        self._check("buf_free", self._lib.mslim_attn_buf_free(self._h, ptr))

    def buf_read(self, ptr: int, offset: int, nbytes: int) -> bytes:
        out = C.create_string_buffer(nbytes)
        self._check("buf_read", self._lib.mslim_attn_buf_read(self._h, ptr, offset, C.addressof(out), nbytes))
        return out.raw

    def buf_write(self, ptr: int, offset: int, data: bytes) -> None:
        buf = C.create_string_buffer(bytes(data), len(data))
        self._check("buf_write", self._lib.mslim_attn_buf_write(self._h, ptr, offset, C.addressof(buf), len(data)))

    def decode_dense(self, q, k, v, out, seq_lens: Sequence[int], q_heads: int, kv_heads: int,
                     head_dim: int, seq_stride_tokens: int = 0, scale: Optional[float] = None,
                     split_tokens: int = 0) -> None:
        scale = default_scale(head_dim) if scale is None else scale
        self._check("decode_dense", self._lib.mslim_attn_decode_dense(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(out), len(seq_lens), _lens(seq_lens),
            seq_stride_tokens, q_heads, kv_heads, head_dim, scale, split_tokens))

    def decode_paged(self, q, k_pool, v_pool, out, seq_lens: Sequence[int], page_table,
                     pages_per_seq: int, page_tokens: int, q_heads: int, kv_heads: int,
                     head_dim: int, scale: Optional[float] = None, split_tokens: int = 0) -> None:
        scale = default_scale(head_dim) if scale is None else scale
        self._check("decode_paged", self._lib.mslim_attn_decode_paged(
            self._h, _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(out), len(seq_lens),
            _lens(seq_lens), _ptr(page_table), pages_per_seq, page_tokens, q_heads, kv_heads,
            head_dim, scale, split_tokens))

    def decode_paged_noalloc(self, q, k_pool, v_pool, out, seq_lens: Sequence[int], page_table,
                             pages_per_seq: int, page_tokens: int, q_heads: int, kv_heads: int,
                             head_dim: int, scale: Optional[float] = None, split_tokens: int = 0) -> None:
        """decode_paged with its split partials in the library's fixed device
        array: no allocation; calls that overlap on one GPU race."""
        scale = default_scale(head_dim) if scale is None else scale
        self._check("decode_paged_noalloc", self._lib.mslim_attn_decode_paged_noalloc(
            self._h, _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(out), len(seq_lens),
            _lens(seq_lens), _ptr(page_table), pages_per_seq, page_tokens, q_heads, kv_heads,
            head_dim, scale, split_tokens))

    def prefill_causal(self, q, k, v, out, queries: int, prior: int, q_heads: int,
                       kv_heads: int, head_dim: int, scale: Optional[float] = None) -> None:
        scale = default_scale(head_dim) if scale is None else scale
        self._check("prefill_causal", self._lib.mslim_attn_prefill_causal(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(out), queries, prior, q_heads, kv_heads,
            head_dim, scale))

    # ---- portable backend (exact K/V frames) -----------------------------
    def frames_decode(self, query, keys, key_format: int, values, value_format: int, out,
                      tokens: int, q_heads: int, kv_heads: int, head_dim: int) -> None:
        """Device buffers: f32 query/out, raw K/V frames [tokens][kv_heads][D]."""
        self._check("frames_decode", self._lib.mslim_attn_frames_decode(
            self._h, _ptr(query), _ptr(keys), key_format, _ptr(values), value_format, _ptr(out),
            tokens, q_heads, kv_heads, head_dim))

    def backend_decode(self, query, keys: bytes, key_format: int, values: bytes,
                       value_format: int, tokens: int, q_heads: int, kv_heads: int,
                       head_dim: int):
        """Blocking host-memory decode; returns (f32 numpy output, Timings)."""
        import numpy as np
        q = np.ascontiguousarray(query, np.float32)
        out = np.empty(q_heads * head_dim, np.float32)
        kb = np.frombuffer(bytes(keys), np.uint8) if keys is not None else None
        vb = np.frombuffer(bytes(values), np.uint8) if values is not None else None
        t = Timings()
        rc = self._lib.mslim_attn_backend_decode(
            self._h, q.ctypes.data, kb.ctypes.data if kb is not None and kb.size else None,
            key_format, vb.ctypes.data if vb is not None and vb.size else None, value_format,
            tokens, q_heads, kv_heads, head_dim, out.ctypes.data, C.byref(t))
        self._check("backend_decode", rc)
        return out, t

    # ---- feeders --------------------------------------------------------
    def rmsnorm(self, x, weight, out, tokens: int, hidden: int, eps: float) -> None:
        self._check("rmsnorm", self._lib.mslim_attn_rmsnorm(
            self._h, _ptr(x), _ptr(weight), _ptr(out), tokens, hidden, eps))

    def rope(self, x, out, tokens: int, heads: int, head_dim: int, start_position: int,
             theta: float, llama3_scaling: bool = False, factor: float = 1.0,
             low_freq_factor: float = 1.0, high_freq_factor: float = 2.0,
             original_max_position: float = 1.0) -> None:
        self._check("rope", self._lib.mslim_attn_rope(
            self._h, _ptr(x), _ptr(out), tokens, heads, head_dim, start_position, theta,
            int(bool(llama3_scaling)), factor, low_freq_factor, high_freq_factor,
            original_max_position))

    def rope_rows(self, x, out, tokens: int, heads: int, head_dim: int, positions,
                  theta: float, llama3_scaling: bool = False, factor: float = 1.0,
                  low_freq_factor: float = 1.0, high_freq_factor: float = 2.0,
                  original_max_position: float = 1.0) -> None:
        self._check("rope_rows", self._lib.mslim_attn_rope_rows(
            self._h, _ptr(x), _ptr(out), tokens, heads, head_dim, _ptr(positions), theta,
            int(bool(llama3_scaling)), factor, low_freq_factor, high_freq_factor,
            original_max_position))

    def rope_qk(self, q, q_out, k, k_out, tokens: int, q_heads: int, kv_heads: int, head_dim: int,
                start_position: int, theta: float, llama3_scaling: bool = False, factor: float = 1.0,
                low_freq_factor: float = 1.0, high_freq_factor: float = 2.0,
                original_max_position: float = 1.0) -> None:
        self._check("rope_qk", self._lib.mslim_attn_rope_qk(
            self._h, _ptr(q), _ptr(q_out), _ptr(k), _ptr(k_out), tokens, q_heads, kv_heads, head_dim,
            start_position, theta, int(bool(llama3_scaling)), factor, low_freq_factor, high_freq_factor,
            original_max_position))

    def swiglu(self, gate, up, out, n: int) -> None:
        self._check("swiglu", self._lib.mslim_attn_swiglu(self._h, _ptr(gate), _ptr(up),
                                                          _ptr(out), n))

    # ---- ColdStore-exact page pool --------------------------------------
    def pages_write(self, k_pool, v_pool, page_table_row, page_tokens: int, kv_heads: int,
                    head_dim: int, first_token: int, tokens: int, k_rows, v_rows) -> None:
        self._check("pages_write", self._lib.mslim_attn_pages_write(
            self._h, _ptr(k_pool), _ptr(v_pool), _ptr(page_table_row), page_tokens, kv_heads,
            head_dim, first_token, tokens, _ptr(k_rows), _ptr(v_rows)))

    def pages_append(self, k_pool, v_pool, page_table, pages_per_seq: int, page_tokens: int,
                     kv_heads: int, head_dim: int, batch: int, positions, k_rows, v_rows) -> None:
        self._check("pages_append", self._lib.mslim_attn_pages_append(
            self._h, _ptr(k_pool), _ptr(v_pool), _ptr(page_table), pages_per_seq, page_tokens,
            kv_heads, head_dim, batch, _ptr(positions), _ptr(k_rows), _ptr(v_rows)))

    def rope_append(self, q, k, v, q_out, k_pool, v_pool, page_table, pages_per_seq: int,
                    page_tokens: int, batch: int, positions, q_heads: int, kv_heads: int, head_dim: int,
                    theta: float, llama3_scaling: bool = False, factor: float = 1.0,
                    low_freq_factor: float = 1.0, high_freq_factor: float = 2.0,
                    original_max_position: float = 1.0) -> None:
        self._check("rope_append", self._lib.mslim_attn_rope_append(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(q_out), _ptr(k_pool), _ptr(v_pool), _ptr(page_table),
            pages_per_seq, page_tokens, batch, _ptr(positions), q_heads, kv_heads, head_dim, theta,
            int(bool(llama3_scaling)), factor, low_freq_factor, high_freq_factor, original_max_position))

    def pages_gather(self, pool, page_table_row, page_tokens: int, kv_heads: int, head_dim: int,
                     first_token: int, tokens: int, rows_out) -> None:
        self._check("pages_gather", self._lib.mslim_attn_pages_gather(
            self._h, _ptr(pool), _ptr(page_table_row), page_tokens, kv_heads, head_dim,
            first_token, tokens, _ptr(rows_out)))

    def logical_kv_sha256(self, keys: Sequence, values: Sequence, tokens: int, kv_heads: int,
                          head_dim: int, page_tables: Optional[Sequence] = None,
                          page_tokens: int = 0) -> str:
        n = len(keys)
        kp = (C.c_void_p * n)(*[_ptr(k) for k in keys])
        vp = (C.c_void_p * n)(*[_ptr(v) for v in values])
        tp = (C.c_void_p * n)(*[_ptr(t) for t in page_tables]) if page_tables else None
        out = C.create_string_buffer(65)
        self._check("logical_kv_sha256", self._lib.mslim_attn_logical_kv_sha256(
            self._h, n, tokens, kv_heads, head_dim, kp, vp, tp, page_tokens, out))
        return out.value.decode()

    # ---- ColdStore record frames ------------------------------------------
    @staticmethod
    def record_frame_bytes(page_tokens: int) -> int:
        return int(library().mslim_attn_record_frame_bytes(page_tokens))

    def record_frames(self, k_pool, v_pool, pool_pages: int, page_tokens: int, kv_heads: int,
                      head_dim: int, tile: int, records, count: int, frames) -> None:
        """`records`: device array of PageRecord; `frames`: device output of
        count * record_frame_bytes(page_tokens) bytes."""
        self._check("record_frames", self._lib.mslim_attn_record_frames(
            self._h, _ptr(k_pool), _ptr(v_pool), pool_pages, page_tokens, kv_heads, head_dim,
            tile, _ptr(records), count, _ptr(frames)))

    # ---- Projection GEMM --------------------------------------------------
    def matrix_multiply(self, weight, input_bits, inner: int, rows: int, tokens: int):
        """tv_hip_matrix_multiply: host BF16 bits in [tokens][inner], host out
        [tokens][rows]; weight is a device buffer [rows][inner]."""
        import numpy as np
        x = np.ascontiguousarray(input_bits, np.uint16)
        out = np.empty(tokens * rows, np.uint16)
        self._check("matrix_multiply", self._lib.mslim_attn_matrix_multiply(
            self._h, _ptr(weight), x.ctypes.data, out.ctypes.data, inner, rows, tokens))
        return out

    def gemm_bf16(self, weight, input_dev, output_dev, inner: int, rows: int, tokens: int) -> None:
        self._check("gemm_bf16", self._lib.mslim_attn_gemm_bf16(
            self._h, _ptr(weight), _ptr(input_dev), _ptr(output_dev), inner, rows, tokens))

    def gemm_bf16_add(self, weight, input_dev, residual, output_dev, inner: int, rows: int,
                      tokens: int) -> None:
        self._check("gemm_bf16_add", self._lib.mslim_attn_gemm_bf16_add(
            self._h, _ptr(weight), _ptr(input_dev), _ptr(residual), _ptr(output_dev), inner, rows, tokens))

    def gemm_swiglu(self, gate_weight, up_weight, input_dev, output_dev, inner: int, rows: int,
                    tokens: int) -> None:
        self._check("gemm_swiglu", self._lib.mslim_attn_gemm_swiglu(
            self._h, _ptr(gate_weight), _ptr(up_weight), _ptr(input_dev), _ptr(output_dev), inner, rows,
            tokens))

    def gemm_qkv(self, q_weight, k_weight, v_weight, input_dev, q_out, k_out, v_out, inner: int,
                 q_rows: int, kv_rows: int, tokens: int) -> None:
        self._check("gemm_qkv", self._lib.mslim_attn_gemm_qkv(
            self._h, _ptr(q_weight), _ptr(k_weight), _ptr(v_weight), _ptr(input_dev), _ptr(q_out),
            _ptr(k_out), _ptr(v_out), inner, q_rows, kv_rows, tokens))

    def rmsnorm_gemm_bf16(self, norm_weight, eps: float, weight, input_dev, output, inner: int, rows: int,
                          tokens: int) -> None:
        self._check("rmsnorm_gemm_bf16", self._lib.mslim_attn_rmsnorm_gemm_bf16(
            self._h, _ptr(norm_weight), eps, _ptr(weight), _ptr(input_dev), _ptr(output), inner, rows, tokens))

    def rmsnorm_gemm_qkv(self, norm_weight, eps: float, q_weight, k_weight, v_weight, input_dev, q_out, k_out,
                         v_out, inner: int, q_rows: int, kv_rows: int, tokens: int) -> None:
        self._check("rmsnorm_gemm_qkv", self._lib.mslim_attn_rmsnorm_gemm_qkv(
            self._h, _ptr(norm_weight), eps, _ptr(q_weight), _ptr(k_weight), _ptr(v_weight), _ptr(input_dev),
            _ptr(q_out), _ptr(k_out), _ptr(v_out), inner, q_rows, kv_rows, tokens))

    def rmsnorm_gemm_swiglu(self, norm_weight, eps: float, gate_weight, up_weight, input_dev, output, inner: int,
                            rows: int, tokens: int) -> None:
        self._check("rmsnorm_gemm_swiglu", self._lib.mslim_attn_rmsnorm_gemm_swiglu(
            self._h, _ptr(norm_weight), eps, _ptr(gate_weight), _ptr(up_weight), _ptr(input_dev), _ptr(output),
            inner, rows, tokens))

    def rmsnorm_qkv_rope_append(self, norm_weight, eps: float, q_weight, k_weight, v_weight, input_dev, q_out,
                                k_pool, v_pool, page_table, pages_per_seq: int, page_tokens: int, batch: int,
                                positions, inner: int, q_heads: int, kv_heads: int, head_dim: int, theta: float,
                                llama3_scaling: bool = False, factor: float = 1.0, low_freq_factor: float = 1.0,
                                high_freq_factor: float = 2.0, original_max_position: float = 1.0) -> None:
        self._check("rmsnorm_qkv_rope_append", self._lib.mslim_attn_rmsnorm_qkv_rope_append(
            self._h, _ptr(norm_weight), eps, _ptr(q_weight), _ptr(k_weight), _ptr(v_weight), _ptr(input_dev),
            _ptr(q_out), _ptr(k_pool), _ptr(v_pool), _ptr(page_table), pages_per_seq, page_tokens, batch,
            _ptr(positions), inner, q_heads, kv_heads, head_dim, theta, int(bool(llama3_scaling)), factor,
            low_freq_factor, high_freq_factor, original_max_position))

    def add(self, a, b, out, n: int) -> None:
        self._check("add", self._lib.mslim_attn_add(self._h, _ptr(a), _ptr(b), _ptr(out), n))

    def embed(self, table, vocab: int, hidden: int, ids, tokens: int, out, bad=None) -> None:
        self._check("embed", self._lib.mslim_attn_embed(self._h, _ptr(table), vocab, hidden, _ptr(ids),
                                                        tokens, _ptr(out), _ptr(bad)))

    def argmax(self, logits, rows: int, vocab: int, out) -> None:
        self._check("argmax", self._lib.mslim_attn_argmax(self._h, _ptr(logits), rows, vocab, _ptr(out)))

    def record_payloads(self, k_pool, v_pool, pool_pages: int, page_tokens: int, kv_heads: int,
                        head_dim: int, records, count: int, k_stage, v_stage, to_staging: bool) -> None:
        """Pool pages <-> compacted staging slots of kv_heads*page_tokens*head_dim BF16."""
        self._check("record_payloads", self._lib.mslim_attn_record_payloads(
            self._h, _ptr(k_pool), _ptr(v_pool), pool_pages, page_tokens, kv_heads, head_dim,
            _ptr(records), count, _ptr(k_stage), _ptr(v_stage), 0 if to_staging else 1))


def _host_ptr(a) -> int:
    return a.ctypes.data


def split_count(tokens: int, split_tokens: int) -> int:
    return math.ceil(tokens / split_tokens)


def auto_split(seq_lens: Sequence[int], kv_heads: int) -> int:
    """The split_tokens that split_tokens = 0 picks for this batch (host only)."""
    lib = library()
    arr = (C.c_int32 * len(seq_lens))(*[int(t) for t in seq_lens])
    out = lib.mslim_attn_decode_auto_split(arr, len(seq_lens), kv_heads)
    if out < 0:
        raise MslimAttnError("decode_auto_split", out, lib.mslim_attn_last_error().decode())
    return out


def prefill_split_tiles(queries: int, prior: int, q_heads: int, kv_heads: int, head_dim: int) -> int:
    """Key tiles per chunk of a split prefill launch of this shape (0: not split)."""
    lib = library()
    out = lib.mslim_attn_prefill_split_tiles(queries, prior, q_heads, kv_heads, head_dim)
    if out < 0:
        raise MslimAttnError("prefill_split_tiles", out, lib.mslim_attn_last_error().decode())
    return out


def prefill_pool_items(queries: int, prior: int, q_heads: int, kv_heads: int, head_dim: int) -> int:
    """Row blocks per XCD that a prefill launch of this shape hands out at run time (0: none)."""
    lib = library()
    out = lib.mslim_attn_prefill_pool_items(queries, prior, q_heads, kv_heads, head_dim)
    if out < 0:
        raise MslimAttnError("prefill_pool_items", out, lib.mslim_attn_last_error().decode())
    return out
