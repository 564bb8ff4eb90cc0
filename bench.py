#!/usr/bin/env python3
"""Benchmark of the M-SLIM attention hot path on one MI355X.

Workload (the largest single-GPU configuration and
the one the targets are quoted on):
  * decode: batch 4 x 32,768-token context, 64 query / 8 KV heads, head_dim
    128, BF16 K/V in the ColdStore-exact page pool (16-token pages): cold
    pages in a seeded random permutation plus a contiguous 4,096-token hot
    recent window per sequence;
  * causal prefill of 8,192 tokens at the same head shape.
One step = one paged decode pass + one causal prefill pass.  The timed
region runs the K decode passes back to back and then the K prefill passes,
with events on the launch stream around each phase.  Inputs are resident in
HBM before timing starts.  The decode passes cycle through four distinct
layer caches (2.1 GB of K/V pages, eight times the 256 MB Infinity Cache), as
a model's decode walks its layers, so no pass finds the previous pass's bytes
in a cache.  A decode launched directly after a prefill is
timed separately and reported as `decode_after_prefill_ms`.

`value` is the decode's achieved HBM bandwidth (algorithmic K+V+Q+O bytes /
average decode launch time measured with HIP events on the launch stream);
the prefill's TFLOP/s is reported beside it under "prefill".  The CPU
baseline is the C oracle's restatement of the reference CPU attention
(native_cpu_adapter.rs:253-307), parallel over query heads like the
reference's rayon loop (:273-276), timed on a bounded sample of the same
workload on this host.

The ColdStore seal of every pool page (device record frames: per-token FNV
tables, checksums, SHA-256; cold_store.rs:269-349) is timed on the same pool
and reported under "coldstore_seal", with the oracle's restatement of the
reference codec timed on the host cores beside it.

Before each timed loop a short device sleep is queued behind the final
synchronize so that the first timed launch does not wait on host launch
latency; every timed call is then back-to-back device work.

The full decoder of BASELINE.json configs[4] (Llama-3-8B shape, 32 layers,
random N(0, 0.02) BF16 weights, batch 8, seeded 4,096-token prompts, 128
greedy steps) runs through the C++ decoder runner with K/V in the
ColdStore-exact page pool and is reported under "decoder": prefill and
decode tokens/s and the decode step's HBM roofline, plus a check that the
dense K/V layout yields the same tokens and K/V digest.  Its CPU baseline is
the oracle decoder on one host core, one layer timed and scaled to 32.

`--kernel decode|prefill|copy|decoder` runs only that workload (no CPU
baseline for the kernels) for counter collection: `copy` is a plain 1 GiB
device copy whose FETCH_SIZE / WRITE_SIZE readings calibrate the byte
counters.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--cpu-seconds 10]
                       [--kernel all|decode|prefill|copy|decoder] [--decoder-steps 128]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vk-shei_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode-attn HBM GB/s (% of peak) + causal prefill TFLOP/s, bf16 GQA d=128"
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense BF16 MFMA, published

B, T, QH, KVH, D = 4, 32768, 64, 8, 128
PAGE_TOKENS, HOT_WINDOW = 16, 4096
S_PREFILL = 8192
DECODE_LAYERS = 4  # distinct layer caches the timed decode cycles through


def decode_bytes() -> int:
    # K + V read once, Q read, O written (BF16).
    return B * T * KVH * D * 2 * 2 + B * QH * D * 2 * 2


def prefill_flops() -> int:
    # causal incl. diagonal, QK^T + PV at 2 FLOP/MAC: 2*D*QH*S*(S+1)
    return 2 * D * QH * S_PREFILL * (S_PREFILL + 1)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_page_pool(ctx, torch, k_dense, v_dense, seed: int):
    """Scatter the dense caches into a page pool: per sequence the cold pages
    are a seeded random permutation of pool slots, the hot window is one
    contiguous run of slots."""
    import numpy as np

    pages_per_seq = T // PAGE_TOKENS
    hot_pages = HOT_WINDOW // PAGE_TOKENS
    cold_pages = pages_per_seq - hot_pages
    total = B * pages_per_seq
    rng = np.random.default_rng(seed)
    cold_slots = rng.permutation(B * cold_pages).astype(np.int32)
    table = np.zeros((B, pages_per_seq), np.int32)
    for b in range(B):
        table[b, :cold_pages] = cold_slots[b * cold_pages:(b + 1) * cold_pages]
        table[b, cold_pages:] = B * cold_pages + b * hot_pages + np.arange(hot_pages, dtype=np.int32)
    table_t = torch.from_numpy(table).cuda()
    k_pool = torch.empty((total, KVH, PAGE_TOKENS, D), dtype=torch.int16, device="cuda")
    v_pool = torch.empty_like(k_pool)
    for b in range(B):
        ctx.pages_write(k_pool, v_pool, table_t[b], PAGE_TOKENS, KVH, D, 0, T, k_dense[b], v_dense[b])
    return k_pool, v_pool, table_t, pages_per_seq


def group_sizes(steps: int) -> list:
    """Sizes of the (at most four) groups of back-to-back timed launches."""
    n = min(4, steps)
    return [steps // n + (1 if i < steps % n else 0) for i in range(n)]


def device_peak_figures(ctx) -> dict:
    """The dense BF16 peak computed from what the device reports, beside the
    published figure the roofline fraction uses: CUs x peak engine clock x
    4,096 FLOP per clock per CU (gfx950 MFMA).  The memory clock and bus
    width are reported as read; HBM3E moves more than two transfers per
    reported clock, so no HBM peak is derived from them."""
    info = ctx.device_info()
    return {
        "name": info["name"], "arch": info["arch"], "compute_units": info["compute_units"],
        "max_clock_mhz": info["max_clock_mhz"], "memory_clock_mhz": info["memory_clock_mhz"],
        "memory_bus_bits": info["memory_bus_bits"],
        "bf16_tflops": round(info["compute_units"] * info["max_clock_mhz"] * 1e6 * 4096 / 1e12, 1),
    }


def cpu_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def cpu_decode_baseline(k_host, v_host, q_host, seconds: float):
    """Oracle dense_attention_bf16 over whole cfg4 sequences, one task per
    query head (rayon's par_chunks_mut over heads), until `seconds` pass."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor

    import oracle

    threads = cpu_threads()
    group = QH // KVH
    per_head_k = [np.ascontiguousarray(k_host[:, :, h, :]) for h in range(KVH)]
    per_head_v = [np.ascontiguousarray(v_host[:, :, h, :]) for h in range(KVH)]
    q_f32 = oracle.read_bf16(q_host)

    def head(args):
        b, qh = args
        kv = qh // group
        return oracle.dense_attention_bf16(q_f32[b, qh], per_head_k[kv][b], per_head_v[kv][b], 1, 1, D)

    seqs = 0
    start = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while True:
            b = seqs % B
            list(pool.map(head, [(b, h) for h in range(QH)]))
            seqs += 1
            if time.perf_counter() - start >= seconds:
                break
    elapsed = time.perf_counter() - start
    per_seq_bytes = decode_bytes() // B
    return {
        "value": round(seqs * per_seq_bytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{seqs} cfg4 decode sequences (32,768 tokens, 64/8 heads, d=128) through the "
                   f"oracle's dense_attention_bf16 (native_cpu_adapter.rs:253-307), one task per "
                   f"query head, {elapsed:.1f} s"),
    }


def cpu_prefill_baseline(q_host, k_host, v_host, seconds: float):
    """Per-row causal loop (the CPU decoder's prompt path) on sampled rows of
    the 8,192-token prefill; FLOP counted exactly for the rows done."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor

    import oracle

    threads = cpu_threads()
    group = QH // KVH
    per_head_k = [np.ascontiguousarray(k_host[:, h, :]) for h in range(KVH)]
    per_head_v = [np.ascontiguousarray(v_host[:, h, :]) for h in range(KVH)]
    q_f32 = oracle.read_bf16(q_host)
    rows = [int(r) for r in np.random.default_rng(7).permutation(S_PREFILL)]

    def head(args):
        r, qh = args
        kv = qh // group
        return oracle.dense_attention_bf16(q_f32[r, qh], per_head_k[kv][:r + 1], per_head_v[kv][:r + 1],
                                           1, 1, D)

    done, flops = 0, 0
    start = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while done < len(rows):
            r = rows[done]
            list(pool.map(head, [(r, h) for h in range(QH)]))
            flops += 4 * QH * D * (r + 1)
            done += 1
            if time.perf_counter() - start >= seconds:
                break
    elapsed = time.perf_counter() - start
    return {
        "value": round(flops / elapsed / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{done} random rows of the 8,192-token causal prefill (64/8 heads, d=128), each "
                   f"row a dense_attention_bf16 over its causal prefix, {elapsed:.1f} s; rate "
                   f"extrapolates to the full prefill by exact FLOP count"),
    }


def cpu_seal_baseline(k_pages, v_pages, seconds: float):
    """The reference's record codec (ColdStore::prepare_page: token hashes,
    FNV checksums, SHA-256; cold_store.rs:269-349) as restated by the C
    oracle, one page per task over the host cores, on pages of the bench
    pool until `seconds` pass."""
    from concurrent.futures import ThreadPoolExecutor

    import oracle

    threads = cpu_threads()
    total = k_pages.shape[0]

    def page(i):
        return oracle.coldstore_record(i, 0, i * PAGE_TOKENS, PAGE_TOKENS, KVH, D, 16,
                                       k_pages[i].tobytes(), v_pages[i].tobytes())

    done = 0
    start = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while True:
            list(pool.map(page, [(done + j) % total for j in range(threads * 4)]))
            done += threads * 4
            if time.perf_counter() - start >= seconds:
                break
    elapsed = time.perf_counter() - start
    payload = done * 2 * KVH * PAGE_TOKENS * D * 2
    return {
        "value": round(payload / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{done} pool pages (16 tokens, 8 heads, d=128, K+V 64 KiB) through the oracle's "
                   f"restatement of ColdStore::prepare_page, one page per task, {elapsed:.1f} s"),
    }


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# BASELINE cfg5: Llama-3-8B-shaped decoder, weights N(0, 0.02) BF16, greedy
# decode of 128 steps at batch 8 after seeded 4,096-token prompts.
DEC_LAYERS, DEC_HIDDEN, DEC_QH, DEC_KVH, DEC_D = 32, 4096, 32, 8, 128
DEC_FFN, DEC_VOCAB, DEC_BATCH, DEC_PROMPT, DEC_STEPS = 14336, 128256, 8, 4096, 128
DEC_CHUNK = 512


def decoder_weights(seed: int) -> dict:
    """Random-init cfg5 weights on the device: projections, embedding and LM
    head N(0, 0.02), RMSNorm weights 1 + N(0, 0.1^2), rounded to BF16."""
    from mslim_attn.model import synthetic_weights
    return synthetic_weights(decoder_spec(), seed)


def decoder_spec():
    from mslim_attn.model import ModelSpec
    return ModelSpec(DEC_LAYERS, DEC_HIDDEN, DEC_QH, DEC_KVH, DEC_D, DEC_FFN, DEC_VOCAB, 1e-5, 500000.0)


def decoder_step_bytes(contexts) -> int:
    """Algorithmic HBM bytes of one batched decode step: every weight read
    once (all layers, LM head, one embedding row per sequence) plus each
    sequence's K and V history read once per layer; activations are
    negligible (< 0.1 %)."""
    qd, kvd = DEC_QH * DEC_D, DEC_KVH * DEC_D
    layer = (qd * DEC_HIDDEN * 2 + kvd * DEC_HIDDEN * 2 + 3 * DEC_FFN * DEC_HIDDEN + 2 * DEC_HIDDEN) * 2
    head = DEC_VOCAB * DEC_HIDDEN * 2 + DEC_HIDDEN * 2 + len(contexts) * DEC_HIDDEN * 2
    kv = sum(contexts) * kvd * 2 * 2 * DEC_LAYERS
    return DEC_LAYERS * layer + head + kv


def cpu_decoder_baseline(host_layer: dict, host_head: dict, seconds: float):
    """The oracle's decoder layer (oracle/decoder.py: the reference layer
    order over the pinned stage restatements) on one host core: one decode
    token of layer 0 at position DEC_PROMPT timed, and the final norm + LM
    head timed, then scaled to the 32-layer model."""
    import numpy as np

    import oracle
    from oracle.decoder import DecoderOracle, Session, Spec

    spec = Spec(layers=1, hidden=DEC_HIDDEN, q_heads=DEC_QH, kv_heads=DEC_KVH, head_dim=DEC_D,
                intermediate=DEC_FFN, vocab=DEC_VOCAB)
    ref = DecoderOracle(spec, {**host_layer, **host_head})
    rng = np.random.default_rng(5)
    kvd = DEC_KVH * DEC_D
    hist = [oracle.write_bf16(rng.standard_normal(DEC_PROMPT * kvd, dtype=np.float32)).reshape(DEC_PROMPT, kvd)
            for _ in range(2)]
    x = host_head["embed_row"]
    layer_s, runs = 0.0, 0
    start = time.perf_counter()
    while True:
        sess = Session([hist[0]], [hist[1]])
        t0 = time.perf_counter()
        y = ref._layer(0, x, 1, DEC_PROMPT, sess)
        layer_s += time.perf_counter() - t0
        runs += 1
        if time.perf_counter() - start >= seconds / 2:
            break
    t0 = time.perf_counter()
    ref.logits(y.reshape(1, DEC_HIDDEN))
    head_s = time.perf_counter() - t0
    token_s = DEC_LAYERS * layer_s / runs + head_s
    return {
        "value": round(1.0 / token_s, 5),
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{runs} decode tokens through one full-width layer at position {DEC_PROMPT} "
                   f"({layer_s / runs:.3f} s each) and one final norm + LM head ({head_s:.3f} s) of the "
                   f"oracle decoder; extrapolated to {DEC_LAYERS} layers at batch 1"),
    }


def cold_store_run(torch, ctx, spec, weights, model, prompts, steps: int, plain_tokens) -> dict:
    """cfg5 again on the same runner with a ColdStore-exact store attached to
    every slot (the GPU-region runtime's persistence, gpu_llm/mod.rs:299-306):
    each prefill commits its prompt's K/V at its end (prefill.rs:760-790),
    the decode steps defer their commit, and the end-of-turn flush commits
    the turn's tokens (flush_deferred_cold, mod.rs:1614-1699).  Checks: the
    tokens equal the run without a store; the ColdStore digest read back
    from each file equals the runner's digest of the slot (slots 0 and the
    last); a fresh runner restores all slots from the files
    (restore_session, mod.rs:1335-1451) and its next batched step gives the
    same tokens and bit-identical logits as the uninterrupted runner."""
    import shutil
    import tempfile

    import numpy as np

    from mslim_attn.model import Model

    root = tempfile.mkdtemp(prefix="mslim-cfg5-cold-")
    try:
        dirs = []
        for b in range(DEC_BATCH):
            model.reset(b)
            dirs.append(os.path.join(root, f"slot{b}"))
            os.makedirs(dirs[-1])
            model.attach_cold_store(b, dirs[-1])
        torch.cuda.synchronize()
        log("bench: cfg5 prefill with ColdStore commit (paged)")
        t0 = time.perf_counter()
        first = [model.prefill_only(b, list(prompts[b])) for b in range(DEC_BATCH)]
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        seal_s = sum(model.cold_report(b)["prefill_seal_seconds"] for b in range(DEC_BATCH))
        log(f"bench: cfg5 {steps} decode steps with deferred commit (paged)")
        tokens, generated = first, [first]
        t0 = time.perf_counter()
        for _ in range(steps):
            tokens = model.forward_batch(tokens)
            generated.append(tokens)
        decode_s = time.perf_counter() - t0
        t0 = time.perf_counter()
        for b in range(DEC_BATCH):
            model.flush_cold(b)
        flush_s = time.perf_counter() - t0
        committed = [model.cold_report(b)["committed_tokens"] for b in range(DEC_BATCH)]
        log("bench: cfg5 ColdStore digests")
        digests_equal = all(model.cold_logical_kv_sha256(b) == model.logical_kv_sha256(b)
                            for b in (0, DEC_BATCH - 1))
        want_next = model.forward_batch(tokens)
        want_logits = model.logits().copy()
        for b in range(DEC_BATCH):  # release each file's exclusive writer
            model.detach_cold_store(b)
        log("bench: cfg5 restore of every slot into a fresh runner")
        fresh = Model(ctx, spec, weights, max_batch=DEC_BATCH, chunk_tokens=DEC_CHUNK,
                      max_context=DEC_PROMPT + steps + 1, kv_layout="paged")
        try:
            t0 = time.perf_counter()
            for b in range(DEC_BATCH):
                fresh.attach_cold_store(b, dirs[b])
            attach_s = time.perf_counter() - t0
            for b in range(DEC_BATCH):
                fresh.restore_session(b, DEC_PROMPT + steps)
            torch.cuda.synchronize()
            restore_s = time.perf_counter() - t0
            got_next = fresh.forward_batch(tokens)
            restored_equal = got_next == want_next and np.array_equal(fresh.logits(), want_logits)
        finally:
            fresh.close()
        file_bytes = sum(os.path.getsize(os.path.join(d, "pages-exact.kv")) for d in dirs)
    finally:
        shutil.rmtree(root, ignore_errors=True)
    return {
        "prefill_tokens_per_s": round(DEC_BATCH * DEC_PROMPT / prefill_s, 1),
        "prefill_s": round(prefill_s, 3),
        "prefill_seal_s": round(seal_s, 3),
        "decode_tokens_per_s": round(DEC_BATCH * steps / decode_s, 1),
        "decode_with_flush_tokens_per_s": round(DEC_BATCH * steps / (decode_s + flush_s), 1),
        "flush_s": round(flush_s, 3),
        "restore_s": round(restore_s, 3),
        "restore_open_s": round(attach_s, 3),
        "committed_tokens_per_slot": committed[0] if len(set(committed)) == 1 else committed,
        "coldstore_file_bytes": file_bytes,
        "tokens_equal_run_without_store": generated == plain_tokens,
        "cold_digest_equals_runner_digest": digests_equal,
        "restored_next_step_identical": restored_equal,
        "timing": ("host wall clock; prefill_s includes the end-of-prefill commit, flush_s the end-of-turn "
                   "commit of the decode tokens of all slots, restore_s the load of all slots: restore_open_s opening each store (every record verified on the "
                   "host, twice, as the reference's open and catalogue rebuild do), then the device-verified "
                   "copy into the page pool"),
    }


def decoder_leg(torch, ctx, args, np):
    """cfg5 through the C++ decoder runner (libmslim_host): batch-8 prefill of
    seeded 4,096-token prompts in 512-token causal chunks, then `steps`
    batched greedy decode steps over the ColdStore-exact paged K/V.  The same
    run on the dense K/V layout must give the same tokens."""
    from mslim_attn.model import Model

    log("bench: cfg5 decoder weights on device")
    weights = decoder_weights(seed=0x38423031)
    spec = decoder_spec()
    prompts = np.random.default_rng(20261202).integers(0, DEC_VOCAB, (DEC_BATCH, DEC_PROMPT))
    steps = args.decoder_steps
    runs = {}
    for layout in ("paged", "dense"):
        model = Model(ctx, spec, weights, max_batch=DEC_BATCH, chunk_tokens=DEC_CHUNK,
                      max_context=DEC_PROMPT + steps + 1, kv_layout=layout)
        # untimed warm-up: one short prompt and one step (hipBLASLt plans)
        model.prefill_only(0, list(prompts[0, :DEC_CHUNK + 1]))
        model.forward_batch([0] * DEC_BATCH)
        torch.cuda.synchronize()
        log(f"bench: cfg5 prefill ({layout})")
        t0 = time.perf_counter()
        first = [model.prefill_only(b, list(prompts[b])) for b in range(DEC_BATCH)]
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        log(f"bench: cfg5 {steps} decode steps ({layout})")
        tokens, generated = first, [first]
        t0 = time.perf_counter()
        for _ in range(steps):
            tokens = model.forward_batch(tokens)
            generated.append(tokens)
        decode_s = time.perf_counter() - t0
        runs[layout] = {"prefill_s": prefill_s, "decode_s": decode_s, "tokens": generated,
                        "digest": model.logical_kv_sha256(0)}
        if layout == "paged" and args.cold:
            runs["cold"] = cold_store_run(torch, ctx, spec, weights, model, prompts, steps, generated)
        model.close()
    p = runs["paged"]
    contexts = [DEC_PROMPT + i for i in range(steps)]
    step_bytes = sum(decoder_step_bytes([c] * DEC_BATCH) for c in contexts) / steps
    step_ms = p["decode_s"] / steps * 1e3
    achieved = step_bytes / (step_ms * 1e-3) / 1e9
    result = {
        "workload": (f"BASELINE cfg5: Llama-3-8B-shaped decoder ({DEC_LAYERS} layers, hidden {DEC_HIDDEN}, "
                     f"{DEC_QH}/{DEC_KVH} heads, d={DEC_D}, FFN {DEC_FFN}, vocab {DEC_VOCAB}), random N(0,0.02) "
                     f"BF16 weights, batch {DEC_BATCH} seeded {DEC_PROMPT}-token prompts, {steps} greedy steps, "
                     f"K/V in the ColdStore-exact 16-token page pool"),
        "decode_tokens_per_s": round(DEC_BATCH * steps / p["decode_s"], 1),
        "decode_ms_per_step": round(step_ms, 3),
        "prefill_tokens_per_s": round(DEC_BATCH * DEC_PROMPT / p["prefill_s"], 1),
        "prefill_s": round(p["prefill_s"], 3),
        "timing": "host wall clock around whole calls (each call ends in a blocking read of the greedy tokens)",
        "decode_roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": None,
            "bytes_per_step": int(step_bytes),
            "note": "algorithmic bytes per batched step (all weights + K/V histories) / wall time per step",
        },
        "paged_equals_dense_tokens": p["tokens"] == runs["dense"]["tokens"],
        "paged_equals_dense_kv_sha256": p["digest"] == runs["dense"]["digest"],
        "dense_decode_tokens_per_s": round(DEC_BATCH * steps / runs["dense"]["decode_s"], 1),
    }
    if "cold" in runs:
        result["coldstore"] = runs["cold"]
    if args.cpu_seconds > 0:
        log("bench: cfg5 CPU baseline (oracle decoder layer on one host core)")

        def host(t):
            return t.cpu().numpy().view(np.uint16).reshape(tuple(t.shape))

        layer0 = {k: host(v) for k, v in weights.items() if k.startswith("layers.0.")}
        head = {"final_norm": host(weights["final_norm"]), "lm_head": host(weights["lm_head"]),
                "embed": host(weights["embed"][:1]), "embed_row": host(weights["embed"][int(prompts[0, 0])])}
        result["cpu_baseline"] = cpu_decoder_baseline(layer0, head, args.cpu_seconds)
    del weights
    return result


QUEUE_FILL_CYCLES = 2_000_000  # device sleep ahead of a timed loop (about 1 ms)
PREFILL_WARM = 40              # untimed prefills queued right before the timed ones
CFG2_WARM = 600                # untimed cfg2 prefills (~30 ms) right before the timed ones
COPY_BYTES = 1 << 30             # calibration copy: 1 GiB read + 1 GiB written


def measured_traffic(name: str):
    """HBM bytes per launch from the committed counter summary
    profiles/<name>_traffic.json (FETCH_SIZE + WRITE_SIZE, calibrated), or
    None when it has not been measured."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def timed_calls(torch, fn, steps: int, warm: int = 0) -> float:
    """Average device time in ms of `steps` back-to-back calls of fn, after
    `warm` untimed calls queued on the same stream right before them."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(QUEUE_FILL_CYCLES)
    for _ in range(warm):
        fn()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def other_configs_leg(torch, ctx, np, steps: int) -> dict:
    """BASELINE cfg1-cfg3 at their own shapes, informational (the headline
    line is cfg4).  cfg1: dense decode, B=1, T=1,024, 32/8 heads.  cfg2:
    RoPE (theta 5e5, rotate-half) of Q and K at positions 0..2,047, then the
    causal prefill of 2,048 tokens, 32/8 heads.  cfg3: 32 sessions with
    lengths U[512, 8192] (seeded), 16-token pages under seeded random page
    tables, four distinct layer pools cycled; paged == dense is checked bit
    for bit on the first."""
    import mslim_attn

    gen = torch.Generator(device="cuda").manual_seed(0x43464733)

    def randn(shape):
        return torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)

    qh, kvh, d = 32, 8, 128
    out = {}
    # cfg1
    k1, v1, q1 = randn((1, 1024, kvh, d)), randn((1, 1024, kvh, d)), randn((1, qh, d))
    o1 = torch.empty_like(q1)
    f1 = lambda: ctx.decode_dense(q1, k1, v1, o1, [1024], qh, kvh, d)
    for _ in range(5):
        f1()
    ms1 = timed_calls(torch, f1, steps)
    bytes1 = 1024 * kvh * d * 2 * 2 + qh * d * 2 * 2
    out["cfg1_dense_decode"] = {"us": round(ms1 * 1e3, 2), "gbps": round(bytes1 / (ms1 * 1e-3) / 1e9, 1),
                                "bytes": bytes1, "note": "B=1, T=1,024: launch-bound (0.53 us at the HBM peak)"}
    # cfg2
    s2 = 2048
    q2, k2, v2 = randn((s2, qh, d)), randn((s2, kvh, d)), randn((s2, kvh, d))
    q2r, k2r, o2 = torch.empty_like(q2), torch.empty_like(k2), torch.empty_like(q2)

    def rope2():
        ctx.rope_qk(q2, q2r, k2, k2r, s2, qh, kvh, d, 0, 500000.0)

    f2 = lambda: ctx.prefill_causal(q2r, k2r, v2, o2, s2, 0, qh, kvh, d)
    rope2()
    for _ in range(PREFILL_WARM):
        f2()
    # Like the cfg4 prefill, timed at the sustained clock: ~30 ms of the same
    # launch queued on the stream right before the timed calls.
    ms2 = timed_calls(torch, f2, steps, warm=CFG2_WARM)
    ms2r = timed_calls(torch, rope2, steps)
    flops2 = 2 * d * qh * s2 * (s2 + 1)
    out["cfg2_prefill"] = {"us": round(ms2 * 1e3, 2), "tflops": round(flops2 / (ms2 * 1e-3) / 1e12, 1),
                           "flop": flops2, "rope_qk_us": round(ms2r * 1e3, 2),
                           "rope_qk_gbps": round(s2 * (qh + kvh) * d * 2 * 2 / (ms2r * 1e-3) / 1e9, 1),
                           "split_chunk_tiles": mslim_attn.prefill_split_tiles(s2, 0, qh, kvh, d),
                           "note": "256 (64-row block, 4-head group) tiles of 1 to 32 causal key "
                                   "tiles; the long rows split into chunks of split_chunk_tiles key "
                                   "tiles counted back from the diagonal, spread over the 8 XCDs "
                                   "longest first, the last chunk of a row merging the partials"}
    # cfg3
    lens = np.random.default_rng(20261203).integers(512, 8193, size=32).tolist()
    nb = len(lens)
    pps = max(-(-t // PAGE_TOKENS) for t in lens)
    npages = sum(-(-t // PAGE_TOKENS) for t in lens)
    tmax = pps * PAGE_TOKENS
    q3 = randn((nb, qh, d))
    layers = []
    for layer in range(DECODE_LAYERS):
        kd, vd = randn((nb, tmax, kvh, d)), randn((nb, tmax, kvh, d))
        perm = np.random.default_rng(1000 + layer).permutation(npages).astype(np.int32)
        table = np.zeros((nb, pps), np.int32)
        o = 0
        for b, t in enumerate(lens):
            n = -(-t // PAGE_TOKENS)
            table[b, :n] = perm[o:o + n]
            o += n
        table_t = torch.from_numpy(table).cuda()
        kp = torch.empty((npages, kvh, PAGE_TOKENS, d), dtype=torch.int16, device="cuda")
        vp = torch.empty_like(kp)
        for b, t in enumerate(lens):
            ctx.pages_write(kp, vp, table_t[b], PAGE_TOKENS, kvh, d, 0, t, kd[b], vd[b])
        layers.append((kp, vp, table_t, kd if layer == 0 else None, vd if layer == 0 else None))
        del kd, vd
    o3, o3d = torch.empty_like(q3), torch.empty_like(q3)
    kp, vp, tab, kd, vd = layers[0]
    ctx.decode_paged(q3, kp, vp, o3, lens, tab, pps, PAGE_TOKENS, qh, kvh, d)
    ctx.decode_dense(q3, kd, vd, o3d, lens, qh, kvh, d, seq_stride_tokens=tmax)
    torch.cuda.synchronize()
    equal = bool(torch.equal(o3, o3d))
    it = [0]

    def f3():
        kp, vp, tab = layers[it[0] % DECODE_LAYERS][:3]
        it[0] += 1
        ctx.decode_paged(q3, kp, vp, o3, lens, tab, pps, PAGE_TOKENS, qh, kvh, d)

    for _ in range(2 * DECODE_LAYERS):
        f3()
    ms3 = timed_calls(torch, f3, steps)
    bytes3 = sum(lens) * kvh * d * 2 * 2 + nb * qh * d * 2 * 2
    out["cfg3_paged_ragged_decode"] = {
        "us": round(ms3 * 1e3, 2), "gbps": round(bytes3 / (ms3 * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(bytes3 / (ms3 * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4), "bytes": bytes3,
        "tokens": int(sum(lens)), "auto_split_tokens": mslim_attn.auto_split(lens, kvh),
        "paged_equals_dense": equal}
    if not equal:
        raise SystemExit("cfg3: paged decode differs from dense decode")
    return out


def one_workload(torch, ctx, fn, args) -> int:
    for _ in range(args.warmup):
        fn()
    ms = timed_calls(torch, fn, args.steps)
    print(json.dumps({"kernel": args.kernel, "steps": args.steps, "ms_per_call": round(ms, 5)}), flush=True)
    ctx.close()
    return 0


def copy_only(torch, args) -> int:
    src = torch.ones(COPY_BYTES // 2, dtype=torch.int16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    ms = timed_calls(torch, lambda: dst.copy_(src), args.steps)
    print(json.dumps({"kernel": "copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
                      "steps": args.steps, "ms_per_call": round(ms, 5),
                      "gbps": round(2 * COPY_BYTES / (ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline budget per leg (0 skips the CPU baseline)")
    ap.add_argument("--kernel", choices=("all", "decode", "prefill", "copy", "decoder"), default="all",
                    help="run one workload only, for counter collection")
    ap.add_argument("--decoder-steps", type=int, default=DEC_STEPS,
                    help="greedy steps of the cfg5 decoder leg (0 skips the leg)")
    ap.add_argument("--no-cold", dest="cold", action="store_false",
                    help="skip the cfg5 run with ColdStore persistence")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              f"(no multi-GPU path is built: decode and prefill shard by kv head with no exchange, "
              f"and the decode merge takes split partials from other GPUs unchanged)",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import mslim_attn

    torch.cuda.set_device(0)
    if args.kernel == "copy":
        return copy_only(torch, args)
    ctx = mslim_attn.Context()
    ctx.use_torch_stream()
    device_peaks = device_peak_figures(ctx)
    if args.kernel == "decoder":
        print(json.dumps(decoder_leg(torch, ctx, args, np)), flush=True)
        ctx.close()
        return 0

    log("bench: generating cfg4 inputs on device")
    gen = torch.Generator(device="cuda").manual_seed(0x4D534C49)

    def randn(shape):
        return torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)

    # Layer l: dense K/V [B][T][KVH][D] and the same bytes in a page pool
    # with its own seeded page table.  Layer 0 also feeds the seal and the
    # CPU baseline.
    layers = []
    for l in range(DECODE_LAYERS):
        kd, vd = randn((B, T, KVH, D)), randn((B, T, KVH, D))
        layers.append((kd, vd) + build_page_pool(ctx, torch, kd, vd, seed=20261201 + l))
    k_dense, v_dense, k_pool, v_pool = layers[0][:4]
    q_dec = randn((B, QH, D))
    out_dec = torch.empty_like(q_dec)
    out_dense = torch.empty_like(q_dec)
    q_pre = randn((S_PREFILL, QH, D))
    k_pre = randn((S_PREFILL, KVH, D))
    v_pre = randn((S_PREFILL, KVH, D))
    out_pre = torch.empty_like(q_pre)
    lens = [T] * B

    turn = [0]

    def decode(layer=None):
        l = turn[0] % DECODE_LAYERS if layer is None else layer
        turn[0] += 1
        _, _, kp, vp, table, pages_per_seq = layers[l]
        ctx.decode_paged(q_dec, kp, vp, out_dec, lens, table, pages_per_seq, PAGE_TOKENS, QH, KVH, D)

    def decode_dense(layer=None):
        l = turn[0] % DECODE_LAYERS if layer is None else layer
        turn[0] += 1
        kd, vd = layers[l][:2]
        ctx.decode_dense(q_dec, kd, vd, out_dense, lens, QH, KVH, D, seq_stride_tokens=T)

    def prefill():
        ctx.prefill_causal(q_pre, k_pre, v_pre, out_pre, S_PREFILL, 0, QH, KVH, D)

    if args.kernel != "all":
        return one_workload(torch, ctx, decode if args.kernel == "decode" else prefill, args)

    # The paged ColdStore-exact decode must equal the dense decode bit for
    # bit, on every layer.
    paged_equals_dense = True
    for l in range(DECODE_LAYERS):
        decode(l)
        decode_dense(l)
        torch.cuda.synchronize()
        paged_equals_dense &= bool(torch.equal(out_dec, out_dense))

    log(f"bench: warmup {args.warmup} steps")
    for _ in range(args.warmup):
        decode()
        prefill()
    torch.cuda.synchronize()

    # Timed region: K steps = K decode launches back to back, then K prefill
    # launches back to back, with events on the launch stream around each
    # phase, so each kernel's average is its steady-state launch duration.
    # The chip raises its clock over ~30 ms of sustained MFMA work (the first
    # ten back-to-back prefills average ~1.25 ms, later ones ~1.0 ms), so the
    # prefill phase is preceded on the same stream, with no host wait, by
    # PREFILL_WARM untimed prefills; the events bracket exactly the K timed
    # launches of each phase.
    # Events bracket groups of back-to-back launches (four groups of
    # steps / 4): an event between every launch would add ~3 us of gap to
    # each.  The phase average is the sum of the groups over `steps`
    # launches; the roofline uses the median of the group averages.
    mk = lambda: torch.cuda.Event(enable_timing=True)
    groups = group_sizes(args.steps)
    ev_dec = [mk() for _ in range(len(groups) + 1)]
    ev_pre = [mk() for _ in range(len(groups) + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    torch.cuda._sleep(QUEUE_FILL_CYCLES)
    for g, n in enumerate(groups):
        ev_dec[g].record()
        for _ in range(n):
            decode()
    ev_dec[len(groups)].record()
    for _ in range(PREFILL_WARM):
        prefill()
    for g, n in enumerate(groups):
        ev_pre[g].record()
        for _ in range(n):
            prefill()
    ev_pre[len(groups)].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0 - ev_dec[len(groups)].elapsed_time(ev_pre[0]) * 1e-3  # less the warm prefills
    dec_avg = ev_dec[0].elapsed_time(ev_dec[len(groups)]) / args.steps
    pre_avg = ev_pre[0].elapsed_time(ev_pre[len(groups)]) / args.steps
    dec_med = float(np.median([ev_dec[g].elapsed_time(ev_dec[g + 1]) / n for g, n in enumerate(groups)]))
    pre_med = float(np.median([ev_pre[g].elapsed_time(ev_pre[g + 1]) / n for g, n in enumerate(groups)]))
    step_ms = dec_avg + pre_avg
    log(f"bench: {args.steps} steps, {step_ms:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f}), "
        f"decode {dec_avg * 1e3:.1f} us (median {dec_med * 1e3:.1f}), prefill {pre_avg * 1e3:.1f} us "
        f"(median {pre_med * 1e3:.1f})")

    # Informational: decode launched directly after a prefill (the prefill's
    # output is still being written back and the clock is recovering).
    pairs = [(mk(), mk()) for _ in range(args.steps)]
    torch.cuda.synchronize()
    torch.cuda._sleep(QUEUE_FILL_CYCLES)
    for a, b in pairs:
        prefill()
        a.record()
        decode()
        b.record()
    torch.cuda.synchronize()
    dec_after_prefill = sum(a.elapsed_time(b) for a, b in pairs) / args.steps

    # dense decode over the same layers, for reference
    for _ in range(3):
        decode_dense()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(QUEUE_FILL_CYCLES)
    e0.record()
    for _ in range(args.steps):
        decode_dense()
    e1.record()
    torch.cuda.synchronize()
    dense_ms = e0.elapsed_time(e1) / args.steps

    # ColdStore seal of every pool page (record frames on the device).
    total_pages = k_pool.shape[0]
    recs = (mslim_attn.PageRecord * total_pages)()
    for i in range(total_pages):
        recs[i] = mslim_attn.PageRecord(i, i * PAGE_TOKENS, 0, PAGE_TOKENS, i, 0)
    recs_dev = torch.frombuffer(bytearray(bytes(recs)), dtype=torch.uint8).cuda()
    slot = mslim_attn.Context.record_frame_bytes(PAGE_TOKENS)
    frames = torch.empty(total_pages * slot, dtype=torch.uint8, device="cuda")

    def seal():
        ctx.record_frames(k_pool, v_pool, total_pages, PAGE_TOKENS, KVH, D, 16, recs_dev, total_pages, frames)

    seal()
    seal_ms = timed_calls(torch, seal, max(3, args.steps // 4))
    seal_payload = total_pages * 2 * KVH * PAGE_TOKENS * D * 2

    dec_gbps = decode_bytes() / (dec_med * 1e-3) / 1e9
    pre_tflops = prefill_flops() / (pre_med * 1e-3) / 1e12
    dense_gbps = decode_bytes() / (dense_ms * 1e-3) / 1e9

    traffic = measured_traffic("decode_paged_cfg4")
    pre_traffic = measured_traffic("prefill_causal_s8192")

    log("bench: cfg1-cfg3 at their own shapes")
    others = other_configs_leg(torch, ctx, np, args.steps)

    decoder = decoder_leg(torch, ctx, args, np) if args.decoder_steps > 0 else None

    cpu = None
    if args.cpu_seconds > 0:
        log("bench: CPU baseline (oracle on host cores)")
        k_h = k_dense.cpu().numpy().view(np.uint16)
        v_h = v_dense.cpu().numpy().view(np.uint16)
        q_h = q_dec.cpu().numpy().view(np.uint16)
        cpu = cpu_decode_baseline(k_h, v_h, q_h, args.cpu_seconds)
        cpu["prefill"] = cpu_prefill_baseline(q_pre.cpu().numpy().view(np.uint16),
                                              k_pre.cpu().numpy().view(np.uint16),
                                              v_pre.cpu().numpy().view(np.uint16), args.cpu_seconds)
        cpu["coldstore_seal"] = cpu_seal_baseline(k_pool.cpu().numpy().view(np.uint16),
                                                  v_pool.cpu().numpy().view(np.uint16), args.cpu_seconds)
        cpu["host_cpu"] = cpu_model()
        cpu["host_nproc"] = os.cpu_count()

    result = {
        "metric": METRIC,
        "value": round(dec_gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: torch.randn N(0,1) with a fixed seed on device, rounded to bf16 (RNE)",
        "config": {
            "workload": "BASELINE cfg4: paged ColdStore-exact decode B=4 x T=32768 (4096-token hot "
                        "window + cold 16-token pages) and causal prefill S=8192, 64/8 heads, d=128",
            "batch": B, "context_tokens": T, "q_heads": QH, "kv_heads": KVH, "head_dim": D,
            "page_tokens": PAGE_TOKENS, "hot_window_tokens": HOT_WINDOW,
            "prefill_tokens": S_PREFILL,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec_gbps, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(dec_gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "timing": "median over four groups of back-to-back timed launches of the group's HIP-event average",
            "kernel": "decode_kernel<128,8,paged,fused,non-temporal> (one launch; the last workgroup of "
                      f"each (sequence, kv head) merges the splits), algorithmic bytes {decode_bytes()} per launch",
        },
        "prefill": {
            "value": round(pre_tflops, 2),
            "unit": "TFLOP/s",
            "ms": round(pre_avg, 4),
            "roofline": {
                "bound": "mfma",
                "achieved": round(pre_tflops, 2),
                "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(pre_tflops / PEAK_BF16_TFLOPS, 4),
                "traffic": pre_traffic,
                "timing": "median over four groups of back-to-back timed launches of the group's HIP-event average",
                "peak_from_device": device_peaks["bf16_tflops"],
                "kernel": f"prefill_mfma_kernel<128,8>, algorithmic FLOP {prefill_flops()} per launch",
            },
        },
        "coldstore_seal": {
            "value": round(seal_payload / (seal_ms * 1e-3) / 1e9, 2),
            "unit": "GB/s",
            "ms": round(seal_ms, 4),
            "records": total_pages,
            "kernel": "token_hashes_kernel + frame_kernel: ColdStore record frames (header, per-token "
                      "FNV tables, record FNV, SHA-256) of every cfg4 pool page; value = K+V payload "
                      "bytes sealed per second",
        },
        "decode_tokens_per_s": round(B / (dec_avg * 1e-3), 1),
        "prefill_tokens_per_s": round(S_PREFILL / (pre_avg * 1e-3), 1),
        "decode_ms": round(dec_avg, 5),
        "decode_ms_median": round(dec_med, 5),
        "prefill_ms_median": round(pre_med, 5),
        "device": device_peaks,
        "decode_after_prefill_ms": round(dec_after_prefill, 5),
        "decode_dense_gbps": round(dense_gbps, 2),
        "paged_equals_dense": paged_equals_dense,
        "other_configs": others,
        "decoder": decoder,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    ctx.close()
    ok = paged_equals_dense and (decoder is None or (decoder["paged_equals_dense_tokens"]
                                                     and decoder["paged_equals_dense_kv_sha256"]))
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
