"""Logit comparison diagnostics of the validation matrix.

compare_logit_distributions restates src/conformance.rs:75-155: absolute
differences (max, mean, the p95 at index (n - 1) * 95 // 100 of the sorted
differences), the KL divergence of the candidate's softmax from the
reference's (stable softmax in float64, clamped at zero), top-1 indices (the
first maximum) and top-1/top-2 margins, and bitwise exactness.
within_one_bf16_ulp restates the BF16 neighbour test of
src/bin/mslim-adapter-parity.rs:38-57.  Inputs are float32 logits.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np


class ConformanceError(ValueError):
    """A comparison the reference rejects (empty, mismatched or non-finite)."""


def top_two(values: np.ndarray) -> Tuple[int, float, float]:
    """(index of the first maximum, maximum, runner-up), conformance.rs
    top_two: a later value equal to the maximum is the runner-up (margin 0);
    a single value has runner-up -inf."""
    values = np.asarray(values, dtype=np.float32).reshape(-1)
    index = int(np.argmax(values))
    rest = np.delete(values, index)
    second = rest.max() if rest.size else np.float32(-np.inf)
    return index, float(values[index]), float(second)


def compare_logit_distributions(reference, candidate) -> Dict[str, object]:
    ref = np.asarray(reference, dtype=np.float32).reshape(-1)
    cand = np.asarray(candidate, dtype=np.float32).reshape(-1)
    if ref.size == 0:
        raise ConformanceError("reference logits are empty")
    if ref.size != cand.size:
        raise ConformanceError("logit vocabularies differ")
    if not (np.isfinite(ref).all() and np.isfinite(cand).all()):
        raise ConformanceError("logit comparison requires finite values")
    diff = np.abs(ref - cand)  # float32, as the reference subtracts in f32
    ordered = np.sort(diff)
    p95 = ordered[((diff.size - 1) * 95) // 100]
    ref_max, cand_max = ref.max(), cand.max()
    ref_exp = np.exp((ref - ref_max).astype(np.float64))
    cand_exp = np.exp((cand - cand_max).astype(np.float64))
    ref_sum, cand_sum = ref_exp.sum(), cand_exp.sum()
    if not (np.isfinite(ref_sum) and np.isfinite(cand_sum)):
        raise ConformanceError("logit softmax normalization is not finite")
    ref_log_sum = np.log(ref_sum) + np.float64(ref_max)
    cand_log_sum = np.log(cand_sum) + np.float64(cand_max)
    p = ref_exp / ref_sum
    kl = float(max(0.0, np.sum(p * ((ref.astype(np.float64) - ref_log_sum)
                                    - (cand.astype(np.float64) - cand_log_sum)))))
    r1, rf, rs = top_two(ref)
    c1, cf, cs = top_two(cand)
    return {
        "compared": int(ref.size),
        "exact": bool(np.array_equal(ref.view(np.uint32), cand.view(np.uint32))),
        "max_abs_difference": float(diff.max()),
        "mean_abs_difference": float(diff.astype(np.float64).sum() / diff.size),
        "p95_abs_difference": float(p95),
        "kl_reference_to_candidate": kl,
        "reference_top1": r1,
        "candidate_top1": c1,
        "top1_equal": r1 == c1,
        "reference_top1_top2_margin": float(np.float32(rf) - np.float32(rs)),
        "candidate_top1_top2_margin": float(np.float32(cf) - np.float32(cs)),
    }


def _bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round float32 to BF16 bits, nearest even (finite inputs)."""
    u = values.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.int64) & 0xFFFF


def ordered_bf16(bits: np.ndarray) -> np.ndarray:
    """BF16 bit patterns mapped to integers in the order of their values
    (both zeros equal), so neighbouring values differ by one."""
    bits = np.asarray(bits, dtype=np.int64)
    return np.where(bits & 0x8000 == 0, 0x8000 + bits, 0x8000 - (bits & 0x7FFF))


def within_one_bf16_ulp(left, right) -> bool:
    a = np.asarray(left, dtype=np.float32).reshape(-1)
    b = np.asarray(right, dtype=np.float32).reshape(-1)
    if a.size != b.size:
        return False
    finite = np.isfinite(a) & np.isfinite(b)
    if not np.array_equal(a[~finite].view(np.uint32), b[~finite].view(np.uint32)):
        return False  # a non-finite value must match bit for bit
    da = ordered_bf16(_bf16_bits(a[finite]))
    db = ordered_bf16(_bf16_bits(b[finite]))
    return bool(np.all(np.abs(da - db) <= 1))
