"""ctypes binding of the decoder runner in libmslim_host.so (include/mslim_model.h).

The runner chains the attention library's kernels in the order of the
reference's run_layer (src/gpu_llm/mod.rs:2056-2350) and run_batch_layer
(src/gpu_llm/prefill.rs:897-1061); its methods mirror GpuLlm's prefill_only,
forward_token (batched over slots), generate, position, reset_session and
logical_kv_sha256.
"""
import ctypes as C
import os
from dataclasses import dataclass
from typing import List, Optional, Sequence

from . import Context, MslimAttnError, LibraryMissing, library, _ptr

HOST_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmslim_host.so")

MODEL_EXPORTS = (
    "mslim_model_last_error",
    "mslim_model_new",
    "mslim_model_destroy",
    "mslim_model_prefill",
    "mslim_model_forward_batch",
    "mslim_model_generate",
    "mslim_model_position",
    "mslim_model_reset",
    "mslim_model_logits",
    "mslim_model_logical_kv_sha256",
    "mslim_model_prefill_settings",
    "mslim_model_set_prefill_settings",
    "mslim_model_attach_cold_store",
    "mslim_model_detach_cold_store",
    "mslim_model_flush_cold",
    "mslim_model_restore_session",
    "mslim_model_cold_logical_kv_sha256",
    "mslim_model_cold_report",
    "mslim_model_cold_directory",
    "mslim_model_set_deferred_cold_commit",
    "mslim_model_set_cancel_flag",
    "mslim_model_poisoned",
    "mslim_model_inject_failure",
)


class ColdReport(C.Structure):
    """mslim_model_cold_report (gpu_llm/mod.rs:192-208)."""
    _fields_ = [("attached", C.c_int), ("committed_tokens", C.c_int64), ("prefill_seal_seconds", C.c_double),
                ("last_commit_seconds", C.c_double), ("last_committed_token_layers", C.c_int64),
                ("last_restore_seconds", C.c_double)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}

LAYER_TENSORS = ("input_norm", "q", "k", "v", "o", "post_norm", "gate", "up", "down")

# MSLIM_MODEL_KV_PAGED / MSLIM_MODEL_KV_DENSE
KV_LAYOUTS = {"paged": 0, "dense": 1}


class Spec(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("layers", "hidden", "q_heads", "kv_heads", "head_dim",
                                        "intermediate", "vocab")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("llama3_scaling", C.c_int),
        ("rope_factor", C.c_float), ("rope_low_freq_factor", C.c_float),
        ("rope_high_freq_factor", C.c_float), ("rope_original_max_position", C.c_float)]


@dataclass
class ModelSpec:
    layers: int
    hidden: int
    q_heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    llama3_scaling: bool = False
    rope_factor: float = 1.0
    rope_low_freq_factor: float = 1.0
    rope_high_freq_factor: float = 2.0
    rope_original_max_position: float = 1.0

    def as_struct(self) -> Spec:
        return Spec(self.layers, self.hidden, self.q_heads, self.kv_heads, self.head_dim,
                    self.intermediate, self.vocab, self.rms_eps, self.rope_theta,
                    int(bool(self.llama3_scaling)), self.rope_factor, self.rope_low_freq_factor,
                    self.rope_high_freq_factor, self.rope_original_max_position)


_host: Optional[C.CDLL] = None


def host_library() -> C.CDLL:
    """Load the in-tree libmslim_host.so (which links libmslim_attn.so)."""
    global _host
    if _host is not None:
        return _host
    library()
    if not os.path.exists(HOST_LIB_PATH):
        raise LibraryMissing("load libmslim_host", -1,
                             f"{HOST_LIB_PATH} is not built (run __graft_entry__.build())")
    lib = C.CDLL(HOST_LIB_PATH)
    P, I, I64, PI32 = C.c_void_p, C.c_int, C.c_int64, C.POINTER(C.c_int32)
    sigs = {
        "mslim_model_last_error": (C.c_char_p, []),
        "mslim_model_new": (P, [P, C.POINTER(Spec), C.POINTER(C.c_void_p), I, I, I, I]),
        "mslim_model_destroy": (None, [P]),
        "mslim_model_prefill": (I, [P, I, PI32, I, PI32]),
        "mslim_model_forward_batch": (I, [P, PI32, I, PI32]),
        "mslim_model_generate": (I, [P, PI32, I, I, PI32, I, PI32, C.POINTER(I)]),
        "mslim_model_position": (I64, [P, I]),
        "mslim_model_reset": (I, [P, I]),
        "mslim_model_logits": (I, [P, C.POINTER(C.c_uint16), C.c_size_t, C.POINTER(I)]),
        "mslim_model_logical_kv_sha256": (I, [P, I, C.c_char_p]),
        "mslim_model_prefill_settings": (I, [P, C.c_char_p, C.c_size_t]),
        "mslim_model_set_prefill_settings": (I, [P, C.c_char_p]),
        "mslim_model_attach_cold_store": (I, [P, I, C.c_char_p]),
        "mslim_model_detach_cold_store": (I, [P, I]),
        "mslim_model_flush_cold": (I, [P, I]),
        "mslim_model_restore_session": (I, [P, I, I64]),
        "mslim_model_cold_logical_kv_sha256": (I, [P, I, C.c_char_p]),
        "mslim_model_cold_report": (I, [P, I, C.POINTER(ColdReport)]),
        "mslim_model_cold_directory": (I, [P, I, C.c_char_p, C.c_size_t]),
        "mslim_model_set_deferred_cold_commit": (I, [P, I]),
        "mslim_model_set_cancel_flag": (I, [P, PI32]),
        "mslim_model_poisoned": (I, [P, I]),
        "mslim_model_inject_failure": (I, [P, I, I]),
    }
    for name in MODEL_EXPORTS:
        res, args = sigs[name]
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _host = lib
    return lib


def _ids(values: Sequence[int]):
    return (C.c_int32 * len(values))(*[int(v) for v in values])


class Model:
    """A decoder runner with `max_batch` sequence slots on a Context; K/V in
    the ColdStore-exact paged pool ("paged") or dense token-major rows
    ("dense").

    `weights` maps "embed", "final_norm", "lm_head" and per layer l the names
    of LAYER_TENSORS ("layers.{l}.q", ...) to contiguous device BF16 tensors
    (torch.uint16/bfloat16) laid out [out][in].  The tensors must stay alive
    for the runner's lifetime; the Model keeps references to them.
    """

    def __init__(self, ctx: Context, spec: ModelSpec, weights: dict, max_batch: int = 1,
                 chunk_tokens: int = 128, max_context: int = 1024, kv_layout: str = "paged"):
        lib = host_library()
        names = ["embed", "final_norm", "lm_head"] + [
            f"layers.{l}.{t}" for l in range(spec.layers) for t in LAYER_TENSORS]
        missing = [n for n in names if n not in weights]
        if missing:
            raise KeyError(f"missing weights: {missing[:4]}")
        self._keep = [weights[n] for n in names]
        arr = (C.c_void_p * len(names))(*[_ptr(weights[n]) for n in names])
        self.spec = spec
        self._spec_struct = spec.as_struct()
        self._ctx = ctx
        self._lib = lib
        if kv_layout not in KV_LAYOUTS:
            raise ValueError(f"kv_layout must be one of {sorted(KV_LAYOUTS)}")
        self._h = lib.mslim_model_new(ctx.handle, C.byref(self._spec_struct), arr, max_batch,
                                      chunk_tokens, max_context, KV_LAYOUTS[kv_layout])
        if not self._h:
            raise MslimAttnError("mslim_model_new", -1, self._error())
        self.max_batch = max_batch

    def _error(self) -> str:
        msg = self._lib.mslim_model_last_error()
        return msg.decode("utf-8", "replace") if msg else ""

    def _check(self, stage: str, rc: int) -> None:
        if rc != 0:
            raise MslimAttnError(stage, rc, self._error())

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.mslim_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill_only(self, seq: int, prompt: Sequence[int]) -> int:
        out = C.c_int32(0)
        self._check("prefill", self._lib.mslim_model_prefill(self._h, seq, _ids(prompt), len(prompt),
                                                               C.byref(out)))
        return out.value

    def forward_batch(self, tokens: Sequence[int]) -> List[int]:
        out = (C.c_int32 * len(tokens))()
        self._check("forward_batch", self._lib.mslim_model_forward_batch(
            self._h, _ids(tokens), len(tokens), out))
        return list(out)

    def generate(self, prompt: Sequence[int], max_new: int, eos_ids: Sequence[int] = ()) -> List[int]:
        out = (C.c_int32 * max_new)()
        got = C.c_int(0)
        eos = _ids(eos_ids) if eos_ids else None
        self._check("generate", self._lib.mslim_model_generate(
            self._h, _ids(prompt), len(prompt), max_new, eos, len(eos_ids), out, C.byref(got)))
        return list(out[:got.value])

    def position(self, seq: int) -> int:
        p = self._lib.mslim_model_position(self._h, seq)
        if p < 0:
            raise MslimAttnError("position", -1, self._error())
        return p

    def reset(self, seq: int) -> None:
        self._check("reset", self._lib.mslim_model_reset(self._h, seq))

    def logits(self):
        """uint16 numpy array [rows][vocab] of BF16 bits."""
        import numpy as np
        cap = self.max_batch * self.spec.vocab
        buf = np.zeros(cap, np.uint16)
        rows = C.c_int(0)
        self._check("logits", self._lib.mslim_model_logits(
            self._h, buf.ctypes.data_as(C.POINTER(C.c_uint16)), cap, C.byref(rows)))
        return buf[:rows.value * self.spec.vocab].reshape(rows.value, self.spec.vocab)

    def prefill_settings(self) -> dict:
        """PrefillSettings (batch_tokens, weight_reuse_tokens, attention)."""
        import json
        out = C.create_string_buffer(1024)
        self._check("prefill_settings", self._lib.mslim_model_prefill_settings(self._h, out, 1024))
        return json.loads(out.value.decode())

    def set_prefill_settings(self, settings: dict) -> None:
        import json
        self._check("set_prefill_settings", self._lib.mslim_model_set_prefill_settings(
            self._h, json.dumps(settings).encode()))

    def logical_kv_sha256(self, seq: int) -> str:
        out = C.create_string_buffer(65)
        self._check("logical_kv_sha256", self._lib.mslim_model_logical_kv_sha256(self._h, seq, out))
        return out.value.decode()

    # ---- ColdStore-exact persistence ----------------------------------------
    def attach_cold_store(self, seq: int, directory: str) -> None:
        self._check("attach_cold_store", self._lib.mslim_model_attach_cold_store(
            self._h, seq, os.fsencode(directory)))

    def detach_cold_store(self, seq: int) -> None:
        self._check("detach_cold_store", self._lib.mslim_model_detach_cold_store(self._h, seq))

    def flush_cold(self, seq: int) -> None:
        """End-of-turn commit of every token past the committed prefix."""
        self._check("flush_cold", self._lib.mslim_model_flush_cold(self._h, seq))

    def restore_session(self, seq: int, tokens: int) -> None:
        self._check("restore_session", self._lib.mslim_model_restore_session(self._h, seq, tokens))

    def cold_logical_kv_sha256(self, seq: int) -> str:
        out = C.create_string_buffer(65)
        self._check("cold_logical_kv_sha256", self._lib.mslim_model_cold_logical_kv_sha256(self._h, seq, out))
        return out.value.decode()

    def cold_report(self, seq: int) -> dict:
        r = ColdReport()
        self._check("cold_report", self._lib.mslim_model_cold_report(self._h, seq, C.byref(r)))
        return r.as_dict()

    def set_deferred_cold_commit(self, deferred: bool) -> None:
        """Deferred (default) or immediate commit of each decode step's K/V."""
        self._check("set_deferred_cold_commit",
                    self._lib.mslim_model_set_deferred_cold_commit(self._h, 1 if deferred else 0))

    def cold_directory(self, seq: int) -> str:
        """Directory of the slot's ColdStore, "" when none is attached."""
        out = C.create_string_buffer(4096)
        self._check("cold_directory", self._lib.mslim_model_cold_directory(self._h, seq, out, 4096))
        return os.fsdecode(out.value)

    # ---- failure handling ----------------------------------------------

    def set_cancel_flag(self, flag) -> None:
        """Install a cancel flag: a ctypes c_int32 the caller keeps alive and
        sets nonzero to cancel (None clears).  Read at prompt chunk and layer
        boundaries of a prefill and at token boundaries of forward_batch and
        generate."""
        self._cancel = flag
        ptr = C.cast(C.byref(flag), C.POINTER(C.c_int32)) if flag is not None else None
        self._check("set_cancel_flag", self._lib.mslim_model_set_cancel_flag(self._h, ptr))

    def poisoned(self, seq: int) -> bool:
        rc = self._lib.mslim_model_poisoned(self._h, seq)
        if rc < 0:
            raise MslimAttnError("poisoned", rc, self._error())
        return rc == 1

    INJECT_ARGUMENT_ERROR = 1
    INJECT_CANCEL = 2

    def inject_failure(self, kind: int, layer: int) -> None:
        """Failure injection for tests: the next device step that reaches
        `layer` fails there once (INJECT_ARGUMENT_ERROR, INJECT_CANCEL)."""
        self._check("inject_failure", self._lib.mslim_model_inject_failure(self._h, kind, layer))


def synthetic_weights(spec: ModelSpec, seed: int, scale: float = 0.02, embed_scale: float = 0.02,
                      norm_spread: float = 0.1) -> dict:
    """Random-init BF16 device weights of the runner's layout from torch's
    seeded device generator: projections, LM head and embedding N(0, scale^2)
    (embedding N(0, embed_scale^2)), RMSNorm weights 1 + N(0, norm_spread^2),
    each rounded to BF16.  Generation order: embedding, final norm, LM head,
    then every layer's LAYER_TENSORS in order, so a seed fixes every tensor.
    Returns a dict of int16 device tensors (BF16 bits) keyed as Model expects.
    """
    import torch

    gen = torch.Generator(device="cuda").manual_seed(seed)

    def normal(shape, sc):
        return (torch.randn(shape, generator=gen, device="cuda") * sc).to(torch.bfloat16).view(torch.int16)

    def norm():
        return (1.0 + norm_spread * torch.randn(spec.hidden, generator=gen, device="cuda")).to(
            torch.bfloat16).view(torch.int16)

    qd, kvd = spec.q_heads * spec.head_dim, spec.kv_heads * spec.head_dim
    shapes = {"q": (qd, spec.hidden), "k": (kvd, spec.hidden), "v": (kvd, spec.hidden), "o": (spec.hidden, qd),
              "gate": (spec.intermediate, spec.hidden), "up": (spec.intermediate, spec.hidden),
              "down": (spec.hidden, spec.intermediate)}
    w = {"embed": normal((spec.vocab, spec.hidden), embed_scale), "final_norm": norm(),
         "lm_head": normal((spec.vocab, spec.hidden), scale)}
    for l in range(spec.layers):
        for name in LAYER_TENSORS:
            w[f"layers.{l}.{name}"] = norm() if name.endswith("norm") else normal(shapes[name], scale)
    return w
