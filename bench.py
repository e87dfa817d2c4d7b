"""Benchmark of the paged-attention hot path on one MI355X.

Default workload (configuration 2): Qwen3-8B-shape decode, one layer, batch 64,
contexts uniform in [128, 4096], bf16, block 16. One step = the KV store of
one new token per sequence + paged decode attention, inputs resident in HBM.
Prints ONE JSON line (rank 0). See --help for the other workloads.

Metric: "Decode paged-attn achieved HBM GB/s (% peak)": value = algorithmic
bytes of the step (store + attention) / wall-clock time per step. The
roofline object is for the dominant kernel (decode attention), timed with HIP
events on the stream the op launches on (torch's current stream).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _events_ms(fn, iters: int, pre=None) -> list:
    """Per-call durations (ms) of fn, HIP events on the current stream."""
    times = []
    for _ in range(iters):
        if pre is not None:
            pre()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    return times


def _settle(step, seconds: float = 0.3) -> None:
    """Untimed: repeats a step for `seconds` before the warm-up steps, so that
    the GPU has left its idle clocks when the timed steps start (on a fresh
    process the first tenth of a second of launches ran 3-7% slower)."""
    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(20):
            step()
        torch.cuda.synchronize()


def _launch_avg_ms(fn, iters: int = 50) -> float:
    """Average duration (ms) of one launch of fn, HIP events around `iters`
    back-to-back launches on the current stream. A spin kernel queued first,
    sized to outlast the host's enqueueing of all `iters` calls, keeps the GPU
    behind the host, so host-side call overhead does not show;
    what remains between launches is the dispatch gap of dependent kernels.
    A per-call event pair adds one more such gap per call, which is why the
    in-step figures read a few microseconds longer."""
    torch.cuda.synchronize()
    # about 0.4 ms + 40 us per launch at 2.4 GHz: longer than the host takes
    # to enqueue the launches (up to ~20 us per call through the Python layer)
    torch.cuda._sleep(1_000_000 + 100_000 * iters)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / iters


def cpu_baseline_decode(w, budget_s: float = 15.0) -> dict:
    """The reference's PyTorch decode path (restated in oracle/torch_ref.py from
    PA/tests/test_paged_attention.py:33-71) on host cores, over a bounded
    sample: the first sequences of the batch whose KV fits the time budget."""
    from oracle.torch_ref import ref_paged_attention
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    kc, vc = w.k_cache.cpu(), w.v_cache.cpu()
    q, bt, sl = w.query.cpu(), w.block_tables.cpu(), w.seq_lens.cpu()
    # calibrate on one sequence, then pick a sample that takes ~budget_s
    t0 = time.perf_counter()
    ref_paged_attention(q[:1], kc, vc, bt[:1], sl[:1], w.scale)
    per_seq = max(time.perf_counter() - t0, 1e-4)
    n = max(1, min(w.num_seqs, int(budget_s / 5 / per_seq)))
    reps = []
    for _ in range(5):
        t0 = time.perf_counter()
        ref_paged_attention(q[:n], kc, vc, bt[:n], sl[:n], w.scale)
        reps.append(time.perf_counter() - t0)
    elt = 2
    kv = sum(w.seq_lens_list[:n]) * w.num_kv_heads * w.head_dim * 2 * elt
    byt = kv + 2 * n * w.num_heads * w.head_dim * elt + n * w.max_blocks_per_seq * 4 + n * 4
    med = statistics.median(reps)
    return {"value": round(byt / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"ref_paged_attention (torch CPU, fp32 math) on the first {n} of "
                      f"{w.num_seqs} sequences ({sum(w.seq_lens_list[:n])} context tokens), "
                      f"median of 5 runs = {med * 1e3:.1f} ms; CPU: {_cpu_model()}"}


def fast_path(w) -> bool:
    """Whether the decode op runs decode_fast_kernel for this shape (the
    library's rule: head dim 128 with power-of-two blocks of 16-256, head dims
    64 / 256 with blocks of 16 / 32, at most 4096 sequences); otherwise the
    generic partition and merge kernels."""
    if w.num_seqs > 4096:
        return False
    bs = w.block_size
    if w.head_dim == 128:
        return bs % 16 == 0 and bs <= 256 and bs & (bs - 1) == 0
    return w.head_dim in (64, 256) and bs in (16, 32)


def bench_decode(args, w) -> dict:
    from nanopd_amd import paged_kernels as pk
    dev = w.k_cache.device
    out = torch.empty_like(w.query)
    ws = torch.zeros(max(1, pk.attention_workspace_bytes(
        w.num_seqs, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks_per_seq)),
        dtype=torch.uint8, device=dev)

    def store():
        pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables,
                          w.store_positions)

    def attend():
        pk.paged_attention_forward(out, w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                   w.scale, w.block_size, w.max_blocks_per_seq, workspace=ws)

    _settle(lambda: [store(), attend()])
    for _ in range(args.warmup):
        store()
        attend()
    torch.cuda.synchronize()
    # timed region: exactly `steps` steps, wall clock, sync on both sides
    t0 = time.perf_counter()
    for _ in range(args.steps):
        store()
        attend()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    # per-call figures, outside the timed region
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for a, b in ev:
        store()
        a.record()
        attend()
        b.record()
    torch.cuda.synchronize()
    attn_ms = [a.elapsed_time(b) for a, b in ev]
    attn_avg = _launch_avg_ms(attend, args.steps)
    store_ms = _launch_avg_ms(store, args.steps)
    # cold-cache variant: read a 1 GiB buffer (> 256 MB MALL + L2) before each
    # call, so the KV rows come from HBM; a read leaves no dirty lines behind
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device=dev)
    cold = statistics.mean(_events_ms(attend, 10, pre=lambda: flush_buf.max()))
    del flush_buf
    # the roofline counts the bytes the call must move from HBM at least: a
    # block shared by two tables (config 4's copy-on-write forks) counts once
    uniq = w.attention_unique_bytes()
    step_bytes = uniq + w.store_bytes()
    achieved = uniq / (attn_avg * 1e-3) / 1e9
    return {
        "ms_per_step": ms_step,
        "value": step_bytes / (ms_step * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _profiled_traffic(f"decode_fast_kernel/{w.name}")
                     if fast_path(w) else None},
        "detail": {
            "attention_us_mean": round(attn_avg * 1e3, 2),
            "attention_us_in_step_mean": round(statistics.mean(attn_ms) * 1e3, 2),
            "attention_us_in_step_median": round(statistics.median(attn_ms) * 1e3, 2),
            "attention_us_cold_l2_flushed": round(cold * 1e3, 2),
            "attention_gbs_cold": round(uniq / (cold * 1e-3) / 1e9, 1),
            "store_us_mean": round(store_ms * 1e3, 2),
            "store_gbs": round(w.store_bytes() / (store_ms * 1e-3) / 1e9, 1),
            "attention_bytes": uniq,
            "attention_bytes_per_sequence_sum": w.attention_bytes(),
            "store_bytes": w.store_bytes(),
            "kv_tokens": sum(w.seq_lens_list),
            "kernels": ("decode_fast_kernel (partitions + fused log-sum-exp merge)"
                        if fast_path(w) else
                        "decode_partition_kernel + merge_partitions_kernel (generic)"),
        },
    }


def cpu_baseline_prefill(w, budget_s: float = 15.0) -> dict:
    """The reference's prefill attention (oracle/torch_ref.py ref_prefill_sdpa,
    restating nanoPD/engine/model_runner.py:152-168: SDPA over the packed chunks
    with a block-diagonal causal mask, no paged prefix) on host cores, over
    the first chunks whose run fits the time budget. Its FLOPs are counted
    for the work it does (the chunk-causal part only)."""
    from oracle.torch_ref import ref_prefill_sdpa
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    npf = w.num_prefill_seqs
    chunks = w.chunk_lens[:npf]
    H, D = w.num_heads, w.head_dim
    q, k, v = w.query.cpu(), w.new_k.cpu(), w.new_v.cpu()
    t0 = time.perf_counter()
    ref_prefill_sdpa(q[:chunks[0]], k[:chunks[0]], v[:chunks[0]], chunks[:1], w.scale)
    per_chunk = max(time.perf_counter() - t0, 1e-4)
    n = max(1, min(npf, int(budget_s / 5 / per_chunk)))
    t = sum(chunks[:n])
    reps = []
    start = time.perf_counter()
    while len(reps) < 5 or time.perf_counter() - start < budget_s:
        t0 = time.perf_counter()
        ref_prefill_sdpa(q[:t], k[:t], v[:t], chunks[:n], w.scale)
        reps.append(time.perf_counter() - t0)
    med = statistics.median(reps)
    flops = 4 * H * D * sum(c * (c + 1) // 2 for c in chunks[:n])
    return {"value": round(flops / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"ref_prefill_sdpa (torch CPU SDPA, fp32, chunk-only causal as the reference "
                      f"computes it) on {n} of {npf} chunks of {chunks[0]} tokens, median of "
                      f"{len(reps)} runs = {med * 1e3:.1f} ms; CPU: {_cpu_model()}"}


def bench_prefill(args, w) -> dict:
    """Configuration 3: one step = slot store of every new token, the prefill
    op over the 4 chunks (paged prefix + chunk), the decode op over the 48
    decode rows. Roofline: the prefill kernel against the bf16 MFMA peak,
    counting the useful (unmasked causal) FLOPs."""
    from nanopd_amd import paged_kernels as pk
    npf, tp = w.num_prefill_seqs, w.num_prefill_tokens
    mb = w.block_tables.size(1)
    bt_p, cu_p, cl_p = (w.block_tables[:npf].contiguous(), w.cu_seqlens_q[:npf + 1].contiguous(),
                        w.context_lens[:npf].contiguous())
    bt_d, cl_d = w.block_tables[npf:].contiguous(), w.context_lens[npf:].contiguous()
    out = torch.empty_like(w.query)
    max_q = max(w.chunk_lens[:npf])

    def store():
        pk.paged_kv_store_slots(w.k_cache, w.v_cache, w.new_k, w.new_v, w.slot_mapping)

    def prefill():
        pk.paged_prefill_attention(out[:tp], w.query[:tp], w.k_cache, w.v_cache, bt_p, cu_p, cl_p,
                                   w.scale, w.block_size, mb, max_q)

    def decode():
        pk.paged_attention_forward(out[tp:], w.query[tp:], w.k_cache, w.v_cache, bt_d, cl_d,
                                   w.scale, w.block_size, mb)

    _settle(lambda: [store(), prefill(), decode()])
    for _ in range(args.warmup):
        store()
        prefill()
        decode()
    torch.cuda.synchronize()
    # timed region: exactly `steps` steps, wall clock, sync on both sides
    t0 = time.perf_counter()
    for _ in range(args.steps):
        store()
        prefill()
        decode()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    # per-call figures, outside the timed region
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for a, b in ev:
        store()
        a.record()
        prefill()
        b.record()
        decode()
    torch.cuda.synchronize()
    pf_step_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    pf_ms = _launch_avg_ms(prefill, args.steps)
    flops = w.prefill_flops()
    tflops = flops / (pf_ms * 1e-3) / 1e12
    # the same prefill over an FP8 copy of the pool (per-kv-head scales,
    # amax / 448), outside the timed region
    ks = (w.k_cache.float().abs().amax(dim=(0, 2, 3)) / 448).clamp_min(1e-8).contiguous()
    vs = (w.v_cache.float().abs().amax(dim=(0, 2, 3)) / 448).clamp_min(1e-8).contiguous()
    k8 = (w.k_cache.float() / ks[None, :, None, None]).to(torch.float8_e4m3fn)
    v8 = (w.v_cache.float() / vs[None, :, None, None]).to(torch.float8_e4m3fn)

    def prefill_fp8():
        pk.paged_prefill_attention_fp8(out[:tp], w.query[:tp], k8, v8, bt_p, cu_p, cl_p, w.scale,
                                       w.block_size, mb, max_q, ks, vs)

    _settle(prefill_fp8)
    pf8_ms = _launch_avg_ms(prefill_fp8, args.steps)
    del k8, v8
    return {
        "ms_per_step": ms_step,
        "value": flops / (ms_step * 1e-3) / 1e12,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": _profiled_traffic(f"prefill_kernel/{w.name}")},
        "detail": {
            "prefill_us_mean": round(pf_ms * 1e3, 2),
            "prefill_us_in_step_mean": round(pf_step_ms * 1e3, 2),
            "store_us_mean": round(_launch_avg_ms(store, args.steps) * 1e3, 2),
            "decode_us_mean": round(_launch_avg_ms(decode, args.steps) * 1e3, 2),
            "prefill_fp8_pool_us_mean": round(pf8_ms * 1e3, 2),
            "prefill_flops": flops,
            "prefill_tokens": tp,
            "decode_seqs": len(w.chunk_lens) - npf,
            "kernels": "prefill_kernel (MFMA 16x16x32) + kv_store_kernel + decode_fast_kernel",
        },
    }


def sources_sha(paths) -> str:
    """First 16 hex digits of the SHA-256 of the given repository files, in
    order: the version of the kernel sources a stored counter reading was
    taken on."""
    import hashlib
    h = hashlib.sha256()
    for p in paths:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def _profiled_traffic(key: str):
    """HBM bytes per launch of a kernel, from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE runs, scaled by a plain copy's counter
    reading). Each entry names the kernel sources it was measured on and their
    hash; when the sources have changed since, the reading is stale and None
    is returned (as where no profile was taken)."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            rec = json.load(f).get(key)
    except (OSError, ValueError):
        return None
    if rec is None or "sources" not in rec:
        return None
    try:
        if sources_sha(rec["sources"]) != rec.get("sources_sha"):
            return None
    except OSError:
        return None
    return rec.get("bytes")


def bench_e2e(args, dev) -> int:
    """Configuration 5: random-init Qwen3-8B served by the collocated engine
    (chunked prefill 512, up to 16 running sequences, greedy), requests with
    lognormal prompt/output lengths (median 512 / 128, sigma 1, clipped to
    [32, 8192] / [8, 1024]) arriving as a Poisson process at 8 req/s."""
    from nanopd_amd.engine import Engine, Request, make_requests, serve
    from nanopd_amd.graphs import DecodeGraphs
    from nanopd_amd.qwen3 import QWEN3_8B, PagedQwen3
    t0 = time.perf_counter()
    model = PagedQwen3(QWEN3_8B, num_blocks=args.kv_blocks, block_size=16, device=dev, seed=0,
                       kv_cache_dtype="fp8" if args.kv_fp8 else "auto")
    torch.cuda.synchronize()
    t_init = time.perf_counter() - t0
    # warm-up: kernels, GEMM heuristics and allocator, on short requests
    warm = Engine(model)
    for r in make_requests(4, seed=99, prompt_median=700, out_median=8, out_clip=(8, 16)):
        warm.add(Request(r.rid, r.prompt, r.max_new_tokens))
    warm.drain()
    torch.cuda.synchronize()
    graphs, t_graphs = None, 0.0
    if not args.no_graphs:
        # decode-only steps replay HIP graphs; every (batch, table width)
        # bucket is captured before the timed run
        t0 = time.perf_counter()
        graphs = DecodeGraphs(model, max_width=(8192 + 1024 + 15) // 16)
        graphs.capture_all()
        torch.cuda.synchronize()
        t_graphs = time.perf_counter() - t0
    eng = Engine(model, max_batch_size=16, budget=1024, chunk=512, graphs=graphs)
    reqs = make_requests(args.requests, seed=5)
    res = serve(eng, reqs, progress_every=32)
    print(json.dumps({
        "metric": "Collocated continuous-batching output tok/s, Qwen3-8B (random init)",
        "value": round(res["tok_per_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": 1,
        "ms_per_step": round(res["wall_s"] * 1e3 / max(res["steps"], 1), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0, 0.02), random prompt token ids)",
        "config": {"workload": "cfg5_qwen3_8b_collocated", "requests": args.requests,
                   "arrival_rate": 8.0, "chunk": 512, "max_running": 16, "block_size": 16,
                   "kv_blocks": args.kv_blocks, "params": QWEN3_8B.num_params,
                   "kv_cache": "fp8 e4m3, scale 1/16" if args.kv_fp8 else "bf16",
                   "decode_steps": "hip graphs" if graphs is not None else "eager"},
        "detail": {**{k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()},
                   "init_s": round(t_init, 1), "graph_capture_s": round(t_graphs, 1)},
    }), flush=True)
    return 0


def bench_copy(args, dev) -> int:
    """Device copy of 256 MiB (reads 256 MiB, writes 256 MiB): counter
    calibration for the roofline traffic field."""
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    _settle(lambda: [dst.copy_(src)])
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        dst.copy_(src)
    b.record()
    b.synchronize()
    ms = a.elapsed_time(b) / args.steps
    print(json.dumps({"metric": "device copy GB/s (read + write)", "value": round(2 * n / ms / 1e6, 1),
                      "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
                      "vs_baseline": None, "dtype": "u8", "data": "synthetic",
                      "config": {"workload": "copy_256MiB", "bytes_read": n, "bytes_written": n}}),
          flush=True)
    return 0


def bench_decode_fp8(args, w) -> int:
    """Configuration 2 (or 4: `--workload long-fp8`) over an FP8 (e4m3) pool:
    the same sequences, tables and queries, the bf16 pool's values quantised
    with per-kv-head scales (amax / 448). One step = the fp8 store of one new
    token per sequence + fp8 decode attention. Algorithmic bytes count 1 byte
    per K/V element of each distinct pool row."""
    from nanopd_amd import paged_kernels as pk
    dev = w.k_cache.device
    kvh = w.num_kv_heads
    ks = (w.k_cache.float().abs().amax(dim=(0, 2, 3)) / 448).clamp_min(1e-8).contiguous()
    vs = (w.v_cache.float().abs().amax(dim=(0, 2, 3)) / 448).clamp_min(1e-8).contiguous()
    k8 = (w.k_cache.float() / ks[None, :, None, None]).to(torch.float8_e4m3fn)
    v8 = (w.v_cache.float() / vs[None, :, None, None]).to(torch.float8_e4m3fn)
    out = torch.empty_like(w.query)
    ws = torch.zeros(max(1, pk.attention_workspace_bytes(
        w.num_seqs, w.num_heads, kvh, w.head_dim, w.block_size, w.max_blocks_per_seq)),
        dtype=torch.uint8, device=dev)
    bt = w.block_tables.cpu()
    pos = [n - 1 for n in w.seq_lens_list]
    slots = torch.tensor([int(bt[i, p // w.block_size]) * w.block_size + p % w.block_size
                          for i, p in enumerate(pos)], dtype=torch.int32, device=dev)
    sk = w.store_k.transpose(0, 1)            # [T, kvh, D] views of the stored tokens
    sv = w.store_v.transpose(0, 1)

    def store():
        pk.paged_kv_store_slots_fp8(k8, v8, sk, sv, slots, ks, vs)

    def attend():
        pk.paged_attention_forward_fp8(out, w.query, k8, v8, w.block_tables, w.seq_lens, w.scale,
                                       w.block_size, w.max_blocks_per_seq, ks, vs, workspace=ws)

    _settle(lambda: [store(), attend()])
    for _ in range(args.warmup):
        store()
        attend()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        store()
        attend()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    attn_ms = _launch_avg_ms(attend, args.steps)
    elt = 2
    ctx = sum(w.seq_lens_list)
    # K/V rows at 1 byte per element, each distinct pool row once (a block
    # that a fork shares with its parent counts once), plus the bf16 q and out
    # rows, tables and seq_lens
    attn_bytes = w.unique_kv_bytes() // elt + w._qo_meta_bytes()
    t = len(pos)
    store_bytes = 2 * t * kvh * w.head_dim * (elt + 1) + 4 * t
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "Decode paged-attn achieved HBM GB/s (% peak), FP8 e4m3 KV pool",
        "value": round((attn_bytes + store_bytes) / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8e4m3/bf16",
        "data": f"synthetic ({w.name}'s seeded pool quantised per kv head)",
        "config": {"workload": f"{w.name}_fp8", "num_seqs": w.num_seqs,
                   "num_heads": w.num_heads, "num_kv_heads": kvh, "head_dim": w.head_dim,
                   "block_size": w.block_size, "context_tokens": ctx,
                   "step": "fp8 kv store (1 token/seq) + fp8 paged decode attention"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _profiled_traffic(f"decode_fast_kernel/{w.name}_fp8")},
        "detail": {"attention_us_mean": round(attn_ms * 1e3, 2), "attention_bytes": attn_bytes,
                   "context_tokens_per_s": round(ctx / (attn_ms * 1e-3), 1),
                   "kernels": "decode_fast_kernel<.., fp8> (e4m3 -> bf16 in registers)"},
    }), flush=True)
    return 0


def bench_transfer(args, dev) -> int:
    """KV transfer pack / unpack at configuration 5's shape: one 4096-token
    sequence (256 blocks of 16) of random-init Qwen3-8B (36 layers, 8 kv heads
    of 128, bf16), gathered from a shuffled pool into the transfer layout and
    scattered back into another pool at another block list. Roofline: HBM,
    every byte read once and written once."""
    from nanopd_amd import paged_kernels as pk
    L, N, kvh, bs, D, n = 36, 1024, 8, 16, 128, 256
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    k = torch.randn((L, N, kvh, bs, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((L, N, kvh, bs, D), generator=g, device=dev).to(torch.bfloat16)
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    src = torch.randperm(N, generator=torch.Generator().manual_seed(1))[:n].to(torch.int32).to(dev)
    dst = torch.randperm(N, generator=torch.Generator().manual_seed(2))[:n].to(torch.int32).to(dev)
    wk = torch.empty((L, n, kvh, bs, D), dtype=torch.bfloat16, device=dev)
    wv = torch.empty_like(wk)

    def step():
        pk.extract_kv(k, v, src, wk, wv)
        pk.load_kv(k2, v2, dst, wk, wv)

    _settle(lambda: [step()])
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    gather_ms = _launch_avg_ms(lambda: pk.extract_kv(k, v, src, wk, wv), args.steps)
    scatter_ms = _launch_avg_ms(lambda: pk.load_kv(k2, v2, dst, wk, wv), args.steps)
    per_op = 2 * 2 * L * n * kvh * bs * D * 2      # K + V, read + write
    gbs = per_op / (gather_ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "KV transfer pack + unpack HBM GB/s (read + write)",
        "value": round(2 * per_op / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) pool, shuffled block lists)",
        "config": {"workload": "transfer_qwen3_8b_4096_tokens", "layers": L, "blocks": n,
                   "num_kv_heads": kvh, "block_size": bs, "head_dim": D,
                   "step": "extract_kv (gather into the wire layout) + load_kv (scatter)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": _profiled_traffic("kv_blocks_kernel/transfer_qwen3_8b_4096_tokens")},
        "detail": {"gather_us": round(gather_ms * 1e3, 2), "scatter_us": round(scatter_ms * 1e3, 2),
                   "bytes_per_op": per_op,
                   "scatter_gbs": round(per_op / (scatter_ms * 1e-3) / 1e9, 1)},
    }), flush=True)
    return 0


def cpu_baseline_store(w, reps: int = 5) -> dict:
    """The reference's Python scatter loop (restated in oracle/torch_ref.py
    from nanoPD/docs/en/03-cuda_kernels_en.md:69-78) on host cores, over the
    whole workload: per token, K and V of every kv head into the pool at its
    slot (a one-entry table per token: block = slot // bs, position = slot %
    bs)."""
    from oracle.torch_ref import ref_kv_store_loop
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    kc, vc = w.k_cache.cpu(), w.v_cache.cpu()
    ks, vs = w.new_k.cpu().transpose(0, 1), w.new_v.cpu().transpose(0, 1)   # [kvh, T, D]
    sl = w.slot_mapping.cpu().long()
    tables, pos = (sl // w.block_size)[:, None], sl % w.block_size
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        ref_kv_store_loop(kc, vc, ks, vs, tables, pos)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(w.store_bytes() / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"ref_kv_store_loop (torch CPU, per-token slice assignment) over all "
                      f"{w.new_k.size(0)} tokens of the step, median of {reps} runs = "
                      f"{med * 1e3:.1f} ms; CPU: {_cpu_model()}"}


def bench_store(args, w) -> int:
    """The KV store of configuration 3's mixed step: every new token's K and V
    (2096 tokens x 8 kv heads x 128, bf16) scattered into the pool at its slot
    (npd_paged_kv_store_slots, kv_store_kernel). One step = one store.
    Roofline: HBM, the K/V rows read once and written once plus the slots."""
    from nanopd_amd import paged_kernels as pk

    def store():
        pk.paged_kv_store_slots(w.k_cache, w.v_cache, w.new_k, w.new_v, w.slot_mapping)

    _settle(store)
    for _ in range(args.warmup):
        store()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        store()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    launch_ms = _launch_avg_ms(store, max(args.steps, 50))
    call_ms = statistics.mean(_events_ms(store, args.steps))
    byt = w.store_bytes()
    gbs = byt / (launch_ms * 1e-3) / 1e9
    line = {
        "metric": "Paged KV store achieved HBM GB/s (% peak)",
        "value": round(byt / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 values, shuffled block tables)",
        "config": {"workload": w.name + "_store", "tokens": int(w.new_k.size(0)),
                   "num_kv_heads": w.num_kv_heads, "head_dim": w.head_dim,
                   "block_size": w.block_size,
                   "step": "paged_kv_store_slots of every new token of the mixed step"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": _profiled_traffic(f"kv_store_kernel/{w.name}")},
        "detail": {"store_us_launch_avg": round(launch_ms * 1e3, 3),
                   "store_us_per_call_events": round(call_ms * 1e3, 3),
                   "store_bytes": byt, "kernels": "kv_store_kernel<16, slots>"},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_store(w)
    print(json.dumps(line), flush=True)
    return 0


def emit_prefill(args, w) -> int:
    from nanopd_amd import paged_kernels as pk
    pk.paged_kv_store_slots(w.k_cache, w.v_cache, w.new_k, w.new_v, w.slot_mapping)
    res = bench_prefill(args, w)
    line = {
        "metric": "Chunked-prefill attention TFLOP/s (useful causal FLOPs per mixed step)",
        "value": round(res["value"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 values, shuffled block tables)",
        "config": {"workload": w.name, "num_heads": w.num_heads, "num_kv_heads": w.num_kv_heads,
                   "head_dim": w.head_dim, "block_size": w.block_size,
                   "chunks": w.chunk_lens[:w.num_prefill_seqs],
                   "prefixes": w.ctx_before[:w.num_prefill_seqs],
                   "decodes": len(w.chunk_lens) - w.num_prefill_seqs,
                   "step": "slot store of all new tokens + prefill op + decode op"},
        "roofline": res["roofline"],
        "detail": res["detail"],
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_prefill(w)
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=["decode", "decode-fp8", "long", "long-fp8", "prefill",
                                           "store", "copy", "e2e", "transfer"],
                    default="decode",
                    help="decode: config 2 (default); long: config 4 (8 seqs, 8k-32k); "
                         "prefill: config 3 (4 chunks of 512 on paged prefixes + 48 decodes); "
                         "store: config 3's KV store (2096 tokens into the pool by slot); "
                         "e2e: config 5 (Qwen3-8B collocated serving, tok/s); "
                         "decode-fp8: config 2 over an FP8 (e4m3) pool; "
                         "long-fp8: config 4 over an FP8 pool (its forks' shared "
                         "partitions read once); "
                         "transfer: KV transfer pack + unpack of a 4096-token Qwen3-8B sequence; "
                         "copy: a plain 256 MiB device copy, the calibration kernel for "
                         "the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--num-heads", type=int, default=32,
                    help="decode / decode-fp8: query heads over config 2's 8 kv heads (32: "
                         "config 2 itself; 40 / 64: groups of 5 / 8)")
    ap.add_argument("--head-dim", type=int, default=128,
                    help="decode: head dim over config 2's contexts (64 / 128 / 256: the tuned "
                         "kernel; other multiples of 8 in [32, 256]: the generic one)")
    ap.add_argument("--block-size", type=int, default=16,
                    help="decode: block size over config 2's contexts (8, or other than 16 / 32 at "
                         "head dim 64 / 256: the generic kernel)")
    ap.add_argument("--requests", type=int, default=256, help="e2e: number of requests")
    ap.add_argument("--kv-blocks", type=int, default=12288, help="e2e: KV pool blocks of 16")
    ap.add_argument("--kv-fp8", action="store_true",
                    help="e2e: FP8 (e4m3) KV pool instead of bf16")
    ap.add_argument("--no-graphs", action="store_true",
                    help="e2e: launch decode-only steps kernel by kernel instead of from HIP graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(sharding across GPUs is described, not built)"}))
        return 2
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    from nanopd_amd import _lib, workloads
    _lib.load()
    dev = torch.device("cuda:0")
    if args.workload == "copy":
        return bench_copy(args, dev)
    if args.workload == "e2e":
        return bench_e2e(args, dev)
    if args.workload == "transfer":
        return bench_transfer(args, dev)
    if args.workload == "decode-fp8":
        return bench_decode_fp8(args, workloads.config2(dev, num_heads=args.num_heads))
    if args.workload == "prefill":
        return emit_prefill(args, workloads.config3(dev))
    if args.workload == "store":
        return bench_store(args, workloads.config3(dev))
    if args.workload == "decode":
        w = workloads.config2(dev, num_heads=args.num_heads, head_dim=args.head_dim,
                              block_size=args.block_size)
    else:
        w = workloads.config4(dev)
        from nanopd_amd import paged_kernels as pk
        pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables,
                          w.store_positions)
        pk.copy_blocks(w.k_cache, w.v_cache, w.cow_pairs)
        if args.workload == "long-fp8":
            return bench_decode_fp8(args, w)
    res = bench_decode(args, w)
    line = {
        "metric": "Decode paged-attn achieved HBM GB/s (% peak); collocated tok/s, Qwen3-8B",
        "value": round(res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 values, shuffled block tables)",
        "config": {"workload": w.name, "num_seqs": w.num_seqs, "num_heads": w.num_heads,
                   "num_kv_heads": w.num_kv_heads, "head_dim": w.head_dim,
                   "block_size": w.block_size, "context_tokens": sum(w.seq_lens_list),
                   "step": "kv store (1 token/seq) + paged decode attention"},
        "pct_peak": round(100 * res["value"] / HBM_PEAK_GBS, 2),
        "roofline": res["roofline"],
        "detail": res["detail"],
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_decode(w)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
