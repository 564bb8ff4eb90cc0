"""Four-route validation matrix -- the model-level parity harness of the
reference (src/bin/mslim-adapter-parity.rs:64-163, with the logit
diagnostics of src/conformance.rs:75-155) over this build's routes.

Routes, each run twice with a session reset in between; the decode inputs
are teacher-forced (the probe prompt cycled, :290-295), so every route sees
the same token stream whatever it predicts:

  cpu-hot-dense        the reference CPU decoder restated (oracle.decoder.
                       CpuDecoderOracle), K/V held in memory -- the
                       native-cpu-runtime with an unbounded hot budget;
  cpu-exact-coldstore  the same decoder with every token's K/V appended to the
                       product region store (include/mslim_region.h,
                       single-token writer) and read back from its ColdStore
                       for attention -- native_hot_kv_bytes = 0
                       (native_cpu_adapter.rs:385-455);
  gpu-dense            the HIP decoder runner, dense K/V layout;
  gpu-exact-coldstore  the HIP runner over the ColdStore-exact page pool with a
                       ColdStore attached and immediate commit
                       (mslim_deferred_cold_commit = false).

Policy (:335-357): every route is deterministic (run-1 and run-2 give the
same logits bit for bit, the same tokens and the same logical K/V digest);
the two routes of each backend agree exactly (logits, tokens, digest); the
GPU ColdStore route's file holds exactly the runner's K/V (its
logical_kv_sha256 read from the file equals the runner's -- this build's
form of the physical-snapshot contract, :243-248).  CPU against GPU is a
diagnostic only (cross_backend_role), reported with the conformance
metrics.  TEST INFRASTRUCTURE: the CPU routes are the oracle.
"""
from __future__ import annotations

import tempfile
from dataclasses import dataclass, field
from typing import Dict, List

import numpy as np

import oracle
from oracle.decoder import CpuDecoderOracle, DecoderOracle, Spec

from mslim_attn.conformance import compare_logit_distributions, within_one_bf16_ulp

DEFAULT_DECODE_STEPS = 8  # mslim-adapter-parity.rs:21


@dataclass
class StepTrace:
    input_token: int
    predicted_token: int
    logits: np.ndarray  # float32


@dataclass
class ExecutionTrace:
    prefill_logits: np.ndarray
    prefill_token: int
    decode: List[StepTrace]
    kv: Dict[str, object] = field(default_factory=dict)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- routes -------------------------------------------------------------------

class CpuColdStoreDecoder(CpuDecoderOracle):
    """CpuDecoderOracle whose K/V live in the product region store: each token
    is committed through the single-token writer (GpuRegionStore::append) and
    attention reads the layer's keys and values back from the ColdStore.  A
    reset opens a fresh store in a new directory under `root`, as
    reset_session opens a fresh namespace (gpu_llm/mod.rs:1530-1577)."""

    def __init__(self, spec: Spec, weights, root: str):
        super().__init__(spec, weights)
        self.root = root
        self.stores = {}

    def reset(self, seq: int) -> None:
        from mslim_attn.region import RegionStore

        super().reset(seq)
        old = self.stores.pop(seq, None)
        if old is not None:
            old.close()
        directory = tempfile.mkdtemp(prefix=f"session-{seq}-", dir=self.root)
        s = self.s
        self.stores[seq] = RegionStore(s.q_heads, s.kv_heads, s.head_dim, s.layers, directory)

    def _append_kv(self, seq, layer, k_bits, v_bits):
        store = self.stores[seq]
        store.append(layer, store.layer_tokens(layer), k_bits, v_bits)

    def _layer_kv(self, seq, layer):
        store = self.stores[seq]
        n = store.layer_tokens(layer)
        return store.read(layer, "k", range(n)), store.read(layer, "v", range(n))

    def _tokens(self, seq):
        return self.stores[seq].layer_tokens(0)

    def close(self):
        for store in self.stores.values():
            store.close()
        self.stores.clear()


class CpuRoute:
    def __init__(self, name: str, decoder, digest):
        self.name, self.decoder, self._digest = name, decoder, digest

    def run_once(self, prompt, decode_inputs) -> ExecutionTrace:
        logits, token = self.decoder.prefill(0, prompt)
        steps = []
        for t in decode_inputs:
            row, predicted = self.decoder.step(0, t)
            steps.append(StepTrace(int(t), int(predicted), np.asarray(row, np.float32)))
        return ExecutionTrace(np.asarray(logits, np.float32), int(token), steps,
                              {"logical_kv_sha256": self._digest()})

    def reset(self):
        self.decoder.reset(0)


class GpuRoute:
    def __init__(self, name: str, model, cold_directory: str = None):
        self.name, self.model = name, model
        if cold_directory is not None:
            model.attach_cold_store(0, cold_directory)
            model.set_deferred_cold_commit(False)
        self.cold = cold_directory is not None

    def _logits(self) -> np.ndarray:
        return bf16_bits_to_f32(self.model.logits()[0])

    def run_once(self, prompt, decode_inputs) -> ExecutionTrace:
        token = self.model.prefill_only(0, [int(t) for t in prompt])
        prefill = self._logits()
        steps = []
        for t in decode_inputs:
            predicted = self.model.forward_batch([int(t)])[0]
            steps.append(StepTrace(int(t), int(predicted), self._logits()))
        kv = {"logical_kv_sha256": self.model.logical_kv_sha256(0)}
        if self.cold:
            report = self.model.cold_report(0)
            kv.update({"coldstore_logical_kv_sha256": self.model.cold_logical_kv_sha256(0),
                       "committed_tokens": report["committed_tokens"],
                       "position": self.model.position(0)})
        return ExecutionTrace(prefill, int(token), steps, kv)

    def reset(self):
        self.model.reset(0)


# ---- comparisons --------------------------------------------------------------

def relative_l2(reference, candidate) -> float:
    """|candidate - reference| / |reference| in float64 (this build's model
    tolerance measure, beside the reference's distribution metrics)."""
    a = np.asarray(reference, np.float64)
    b = np.asarray(candidate, np.float64)
    return float(np.linalg.norm(b - a) / np.linalg.norm(a))


def compare_traces(reference_name, reference: ExecutionTrace, candidate_name, candidate: ExecutionTrace) -> dict:
    """mslim-adapter-parity.rs compare_traces (:173-236)."""
    if len(reference.decode) != len(candidate.decode):
        raise ValueError("decode trace lengths differ")
    prefill = compare_logit_distributions(reference.prefill_logits, candidate.prefill_logits)
    prefill["relative_l2"] = relative_l2(reference.prefill_logits, candidate.prefill_logits)
    prefill_ulp = within_one_bf16_ulp(reference.prefill_logits, candidate.prefill_logits)
    rows = []
    exact, tokens_equal, top1, ulp_all = prefill["exact"], True, prefill["top1_equal"], prefill_ulp
    for step, (left, right) in enumerate(zip(reference.decode, candidate.decode)):
        if left.input_token != right.input_token:
            raise ValueError(f"comparison used different teacher-forced input at step {step}")
        distribution = compare_logit_distributions(left.logits, right.logits)
        distribution["relative_l2"] = relative_l2(left.logits, right.logits)
        ulp = within_one_bf16_ulp(left.logits, right.logits)
        exact &= distribution["exact"]
        tokens_equal &= left.predicted_token == right.predicted_token
        top1 &= distribution["top1_equal"]
        ulp_all &= ulp
        rows.append({"step": step, "input_token": left.input_token,
                     "reference_token": left.predicted_token, "candidate_token": right.predicted_token,
                     "token_equal": left.predicted_token == right.predicted_token,
                     "distribution": distribution, "within_one_bf16_ulp": ulp})
    digests_equal = reference.kv["logical_kv_sha256"] == candidate.kv["logical_kv_sha256"]
    return {
        "reference": reference_name,
        "candidate": candidate_name,
        "prefill": {"distribution": prefill, "within_one_bf16_ulp": prefill_ulp,
                    "tokens_equal": reference.prefill_token == candidate.prefill_token},
        "decode": rows,
        "all_logits_exact": bool(exact),
        "all_tokens_equal": bool(tokens_equal and reference.prefill_token == candidate.prefill_token),
        "all_top1_equal": bool(top1),
        "all_within_one_bf16_ulp": bool(ulp_all),
        "kv": {"reference": reference.kv, "candidate": candidate.kv, "logical_bytes_equal": digests_equal},
        "exact_same_backend_passed": bool(exact and tokens_equal
                                          and reference.prefill_token == candidate.prefill_token
                                          and digests_equal),
    }


def run_mode(route, prompt, decode_inputs):
    """mslim-adapter-parity.rs run_mode (:141-159): run, reset, run again."""
    first = route.run_once(prompt, decode_inputs)
    route.reset()
    second = route.run_once(prompt, decode_inputs)
    return first, compare_traces("run-1", first, "run-2", second)


def summary(comparison: dict) -> dict:
    """The headline figures of one comparison, worst case over its rows."""
    dists = [comparison["prefill"]["distribution"]] + [r["distribution"] for r in comparison["decode"]]
    return {
        "reference": comparison["reference"], "candidate": comparison["candidate"],
        "all_logits_exact": comparison["all_logits_exact"],
        "all_tokens_equal": comparison["all_tokens_equal"],
        "all_top1_equal": comparison["all_top1_equal"],
        "all_within_one_bf16_ulp": comparison["all_within_one_bf16_ulp"],
        "logical_bytes_equal": comparison["kv"]["logical_bytes_equal"],
        "max_abs_difference": max(d["max_abs_difference"] for d in dists),
        "max_p95_abs_difference": max(d["p95_abs_difference"] for d in dists),
        "max_mean_abs_difference": max(d["mean_abs_difference"] for d in dists),
        "max_kl": max(d["kl_reference_to_candidate"] for d in dists),
        "max_relative_l2": max(d["relative_l2"] for d in dists),
        "top1_equal_rows": sum(bool(d["top1_equal"]) for d in dists),
        "rows": len(dists),
        "min_reference_margin": min(d["reference_top1_top2_margin"] for d in dists),
    }


# ---- the matrix ----------------------------------------------------------------

def cpu_routes(spec: Spec, weights: dict, root: str):
    hot = CpuDecoderOracle(spec, weights)
    kvd_bytes = spec.head_dim * 2

    def hot_digest():
        sess = hot.sessions[0]
        return oracle.logical_kv_sha256(sess.keys, sess.values, sess.tokens, spec.kv_heads, kvd_bytes)

    cold = CpuColdStoreDecoder(spec, weights, root)
    return (CpuRoute("cpu-hot-dense", hot, hot_digest),
            CpuRoute("cpu-exact-coldstore", cold, lambda: cold.stores[0].logical_kv_sha256()), cold)


def cpu_half(spec: Spec, weights: dict, prompt, decode_inputs, root: str) -> dict:
    """The CPU routes and their same-backend comparison."""
    hot_route, cold_route, cold = cpu_routes(spec, weights, root)
    try:
        cpu_dense, cpu_dense_det = run_mode(hot_route, prompt, decode_inputs)
        cpu_exact, cpu_exact_det = run_mode(cold_route, prompt, decode_inputs)
    finally:
        cold.close()
    return {"traces": {"cpu-hot-dense": cpu_dense, "cpu-exact-coldstore": cpu_exact},
            "determinism": {"cpu_dense": cpu_dense_det, "cpu_exact": cpu_exact_det},
            "same_backend": compare_traces("cpu-hot-dense", cpu_dense, "cpu-exact-coldstore", cpu_exact)}


def run_matrix(ctx, spec: Spec, weights: dict, device_weights: dict, prompt, decode_steps: int, root: str,
               chunk_tokens: int = 16) -> dict:
    """All four routes; returns the receipt (mslim-adapter-parity.rs:354-412)."""
    from mslim_attn.model import Model, ModelSpec

    decode_inputs = [int(prompt[i % len(prompt)]) for i in range(decode_steps)]
    cpu = cpu_half(spec, weights, prompt, decode_inputs, root)
    mspec = ModelSpec(spec.layers, spec.hidden, spec.q_heads, spec.kv_heads, spec.head_dim, spec.intermediate,
                      spec.vocab, spec.rms_eps, spec.rope_theta)
    context = len(prompt) + decode_steps + 1
    gpu = {}
    determinism = {}
    for name, layout in (("gpu-dense", "dense"), ("gpu-exact-coldstore", "paged")):
        model = Model(ctx, mspec, device_weights, max_batch=1, chunk_tokens=chunk_tokens, max_context=context,
                      kv_layout=layout)
        try:
            cold_dir = None
            if layout == "paged":
                cold_dir = tempfile.mkdtemp(prefix="gpu-exact-", dir=root)
            route = GpuRoute(name, model, cold_dir)
            gpu[name], determinism[name] = run_mode(route, prompt, decode_inputs)
        finally:
            model.close()
    gpu_same = compare_traces("gpu-dense", gpu["gpu-dense"], "gpu-exact-coldstore", gpu["gpu-exact-coldstore"])
    cross = compare_traces("cpu-hot-dense", cpu["traces"]["cpu-hot-dense"], "gpu-dense", gpu["gpu-dense"])
    # this build's own diagnostic: the GPU-form oracle (the arithmetic the
    # runner restates) against the runner and against the CPU form
    gpu_form = DecoderOracle(spec, weights)
    form_trace = CpuRoute("oracle-gpu-form", _GpuFormAdapter(gpu_form), lambda: "").run_once(prompt, decode_inputs)
    form_trace.kv["logical_kv_sha256"] = oracle.logical_kv_sha256(
        gpu_form.sessions[0].keys, gpu_form.sessions[0].values, gpu_form.sessions[0].tokens, spec.kv_heads,
        spec.head_dim * 2)
    det = {"cpu_dense": cpu["determinism"]["cpu_dense"], "cpu_exact": cpu["determinism"]["cpu_exact"],
           "gpu_dense": determinism["gpu-dense"], "gpu_exact": determinism["gpu-exact-coldstore"]}
    deterministic = all(d["exact_same_backend_passed"] for d in det.values())
    same_backend = cpu["same_backend"]["exact_same_backend_passed"] and gpu_same["exact_same_backend_passed"]
    exact_kv = gpu["gpu-exact-coldstore"].kv
    physical = (exact_kv["coldstore_logical_kv_sha256"] == exact_kv["logical_kv_sha256"]
                and exact_kv["committed_tokens"] == exact_kv["position"])
    passed = deterministic and same_backend and physical
    return {
        "status": "passed" if passed else "failed",
        "probe_tokens": len(prompt),
        "decode_steps": decode_steps,
        "teacher_forced_decode_inputs": decode_inputs,
        "policy": {
            "activation_depends_on_cross_backend_bit_parity": False,
            "same_backend_requires_exact_logits": True,
            "same_backend_requires_equal_logical_kv_bytes": True,
            "same_backend_requires_equal_tokens": True,
            "approximation_epsilon": 0.0,
            "cross_backend_role": "diagnostic-only",
        },
        "frozen_runtime_configuration": {"prefill_chunk_tokens": chunk_tokens, "deferred_cold_commit": False,
                                          "cpu_coldstore_writer": "single-token", "page_tokens": 16},
        "determinism": {k: summary(v) | {"passed": v["exact_same_backend_passed"]} for k, v in det.items()},
        "same_backend": {"cpu_dense_vs_exact": summary(cpu["same_backend"]),
                         "gpu_dense_vs_exact": summary(gpu_same), "all_passed": same_backend},
        "cross_backend_diagnostic": summary(cross),
        "oracle_forms_diagnostic": {
            "gpu_form_vs_gpu_dense": summary(compare_traces("oracle-gpu-form", form_trace, "gpu-dense",
                                                            gpu["gpu-dense"])),
            "cpu_form_vs_gpu_form": summary(compare_traces("cpu-hot-dense", cpu["traces"]["cpu-hot-dense"],
                                                           "oracle-gpu-form", form_trace)),
        },
        "snapshot_contract": {"accelerator_exact_physical_snapshot": physical,
                              "physical_kv_tensor_bytes_compared_via_logical_sha256": True},
        "comparisons": {"cpu_same_backend": cpu["same_backend"], "gpu_same_backend": gpu_same,
                        "cross_backend": cross},
    }


class _GpuFormAdapter:
    """DecoderOracle (the GPU runtime's form) behind the prefill/step calls of
    a CPU route: prompt in one causal chunk, then token steps."""

    def __init__(self, decoder: DecoderOracle):
        self.d = decoder
        self.sessions = decoder.sessions

    def prefill(self, seq, prompt):
        bits, tok = self.d.prefill(seq, list(prompt))
        return bf16_bits_to_f32(np.asarray(bits).reshape(-1)), tok

    def step(self, seq, token):
        bits, tok = self.d.step(seq, int(token))
        return bf16_bits_to_f32(np.asarray(bits).reshape(-1)), tok

    def reset(self, seq):
        self.d.reset(seq)
