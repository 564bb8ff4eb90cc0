"""ctypes binding of include/mslim_region.h: the exact region store over a
canonical ColdStore (GpuRegionStore, src/gpu_region_store.rs:118-928),
exported by libmslim_host.  K/V rows cross the boundary token-major as BF16
bit arrays [tokens][kv_heads * head_dim] (uint16)."""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

from . import MslimAttnError
from .model import host_library

REGION_EXPORTS = (
    "mslim_region_last_error",
    "mslim_region_new",
    "mslim_region_destroy",
    "mslim_region_layer_tokens",
    "mslim_region_append",
    "mslim_region_read",
    "mslim_region_logical_kv_sha256",
)

_bound = False


def region_library() -> C.CDLL:
    global _bound
    lib = host_library()
    if not _bound:
        P, I, I64 = C.c_void_p, C.c_int, C.c_int64
        sigs = {
            "mslim_region_last_error": (C.c_char_p, []),
            "mslim_region_new": (P, [I, I, I, I, C.c_char_p, I]),
            "mslim_region_destroy": (None, [P]),
            "mslim_region_layer_tokens": (I64, [P, I]),
            "mslim_region_append": (I, [P, I, I64, P, P, I, I]),
            "mslim_region_read": (I, [P, I, I, C.POINTER(I64), I, P]),
            "mslim_region_logical_kv_sha256": (I, [P, C.c_char_p]),
        }
        for name in REGION_EXPORTS:
            res, args = sigs[name]
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _bound = True
    return lib


class RegionStore:
    """GpuRegionStore in exact mode: open (verifying every committed record)
    or create <directory>/pages-exact.kv, or a private temporary store when
    directory is None."""

    def __init__(self, q_heads: int, kv_heads: int, head_dim: int, layers: int,
                 directory: Optional[str] = None, stage_tokens: int = 64):
        self._lib = region_library()
        self.q_heads, self.kv_heads, self.head_dim, self.layers = q_heads, kv_heads, head_dim, layers
        self._h = self._lib.mslim_region_new(q_heads, kv_heads, head_dim, layers,
                                             None if directory is None else os.fsencode(directory),
                                             stage_tokens)
        if not self._h:
            raise MslimAttnError("region_new", -1, self._error())

    def _error(self) -> str:
        msg = self._lib.mslim_region_last_error()
        return msg.decode() if msg else ""

    def _check(self, stage: str, rc: int) -> None:
        if rc < 0:
            raise MslimAttnError(stage, rc, self._error())

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.mslim_region_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def layer_tokens(self, layer: int) -> int:
        n = self._lib.mslim_region_layer_tokens(self._h, layer)
        self._check("layer_tokens", n)
        return int(n)

    def append(self, layer: int, position: int, keys: np.ndarray, values: np.ndarray,
               page_tokens: int = 1) -> None:
        """Token-major BF16 bits [tokens][kv_heads * head_dim] of K and V;
        page_tokens 1 is the single-token writer (GpuRegionStore::append)."""
        row = self.kv_heads * self.head_dim
        k = np.ascontiguousarray(keys, dtype=np.uint16).reshape(-1, row)
        v = np.ascontiguousarray(values, dtype=np.uint16).reshape(-1, row)
        if k.shape != v.shape:
            raise ValueError("K and V rows differ in shape")
        self._check("append", self._lib.mslim_region_append(
            self._h, layer, position, k.ctypes.data, v.ctypes.data, k.shape[0], page_tokens))

    def read(self, layer: int, part: str, positions: Sequence[int]) -> np.ndarray:
        """Token-major BF16 bits of `positions`; part "k" or "v"."""
        pos = np.ascontiguousarray(positions, dtype=np.int64)
        out = np.zeros((pos.size, self.kv_heads * self.head_dim), np.uint16)
        self._check("read", self._lib.mslim_region_read(
            self._h, layer, {"k": 0, "v": 1}[part], pos.ctypes.data_as(C.POINTER(C.c_int64)), pos.size,
            out.ctypes.data))
        return out

    def logical_kv_sha256(self) -> str:
        out = C.create_string_buffer(65)
        self._check("logical_kv_sha256", self._lib.mslim_region_logical_kv_sha256(self._h, out))
        return out.value.decode()
