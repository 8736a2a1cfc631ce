"""Benchmark of the ragged paged-attention path on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--quick]

Headline (the benchmark's configuration 2): one mixed Sarathi step under a 512-token budget,
SmolLM2-360M attention shape (15 query / 5 KV heads, head_dim 64), 48 decode rows
(context U[128,4096]) + 4 prefill chunks (U[32,256] rows truncated by the budget,
prior context U[0,2048]), block size 16, block tables a random scatter over a
64k-block F32 pool (2.7 GB). A step is one ragged attention call over one such
batch (work-list build, split-K stage 1, reduce). Eight independent batches with
their own random tables are rotated, so consecutive steps read different blocks
of the 2.7 GB pool and the 256 MB Infinity Cache cannot hold a step's 276 MB.

value = query rows / second over the timed steps (inputs resident in HBM).
roofline: the attention kernel (attn_main), algorithmic bytes (K/V once per sequence +
tables + Q + O + lengths) / its average duration from HIP events recorded on the
launch stream inside the timed region, against 8 TB/s.
cpu_baseline: the oracle (C++ restatement of the reference CPU path) on the same
batch, single-threaded on this host, timed over a bounded number of calls.
Extra fields: the 64-sequence variant, configs 1 and 3, GEMV and a copy kernel.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12
PMC_COPY_BYTES = 512 << 20
METRIC = "ragged paged-attn tokens/s + % HBM peak; batched decode tok/s at 1 MI355X"
POOL_LAYOUT = 0  # KANSO_POOL_TOKEN_MAJOR unless --pool-layout head
PARTITION = 0  # 0: kanso_ragged_partition_size per batch; -1: the library's choice; > 0: fixed
CHUNK_PARTITION = 0  # > 0: a fixed chunk partition (else from the lengths, or the library's)
WORK = True  # pass the decode work list built from the host-side plan, as the engine does


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class AttnBench:
    """Device-resident inputs for a rotation of attention batches over one pool."""

    def __init__(self, ctx, batches, kv_dtype, seed):
        import torch
        import kanso_infer_amd as K
        self.K, self.torch, self.ctx = K, torch, ctx
        self.batches = batches
        self.kv_dtype = kv_dtype
        b0 = batches[0]
        self.num_blocks = b0.num_blocks
        rows = b0.num_blocks * b0.block_size * b0.num_kv_heads
        g = torch.Generator(device="cuda:0")
        g.manual_seed(seed)
        dev = torch.device("cuda:0")
        if kv_dtype == K.KANSO_KV_F32:
            self.k = torch.randn(rows * b0.head_dim, generator=g, device=dev)
            self.v = torch.randn(rows * b0.head_dim, generator=g, device=dev)
            self.ks = self.vs = None
        else:
            # quantize N(0,1) rows into the pool with the fused append kernel itself
            self.k = torch.zeros(rows * b0.head_dim, dtype=torch.int8, device=dev)
            self.v = torch.zeros_like(self.k)
            if kv_dtype in (K.KANSO_KV_INT8, K.KANSO_KV_FP8):
                self.ks = torch.ones(rows, dtype=torch.float32, device=dev)
            else:
                self.ks = torch.zeros(rows * b0.head_dim // 32, dtype=torch.float16, device=dev)
            self.vs = torch.ones_like(self.ks)
            chunk = 1 << 16
            tok = b0.num_blocks * b0.block_size
            width = b0.num_kv_heads * b0.head_dim
            for t0 in range(0, tok, chunk):
                n = min(chunk, tok - t0)
                kk = torch.randn(n * width, generator=g, device=dev)
                vv = torch.randn(n * width, generator=g, device=dev)
                slots = torch.arange(t0, t0 + n, dtype=torch.int64, device=dev)
                K.kv_append(ctx, kv_dtype, kk, vv, slots, b0.num_blocks, b0.block_size,
                            b0.num_kv_heads, b0.head_dim, self.k, self.v, self.ks, self.vs)
            ctx.check_device_status()
        self.dev_batches = []
        for i, b in enumerate(batches):
            q = torch.randn(b.total_q * b.num_heads * b.head_dim, generator=g, device=dev)
            self.dev_batches.append(dict(
                q=q, out=torch.empty_like(q),
                tables=torch.from_numpy(b.block_tables.ravel().view(np.int32)).to(dev),
                cu=torch.from_numpy(b.cu_seqlens).to(dev),
                lens=torch.from_numpy(b.context_lens.astype(np.int32)).to(dev)))
        torch.cuda.synchronize()

    def partition(self, b):
        """The split-K partition the caller passes: PARTITION if set (-1 = the library's
        own choice), else kanso_ragged_partition_size from the batch's host-side
        lengths, as the engine computes it from its plan."""
        if PARTITION:
            return max(PARTITION, 0)
        return self.K.ragged_partition_size(
            self.ctx, q_lens=b.q_lens, context_lens=b.context_lens, num_heads=b.num_heads,
            num_kv_heads=b.num_kv_heads, head_dim=b.head_dim, block_size=b.block_size,
            max_blocks=b.max_blocks, kv_dtype=self.kv_dtype, num_blocks=self.num_blocks)

    def call(self, i):
        b, d = self.batches[i % len(self.batches)], self.dev_batches[i % len(self.batches)]
        if "P" not in d:
            d["P"] = self.partition(b)
            # the chunk partition from the same lengths (non-zero only for batches
            # without decode rows), unless a fixed or library partition is asked for
            d["CP"] = CHUNK_PARTITION if CHUNK_PARTITION else 0 if PARTITION else self.K.ragged_chunk_partition_size(
                self.ctx, q_lens=b.q_lens, context_lens=b.context_lens, num_heads=b.num_heads,
                num_kv_heads=b.num_kv_heads, head_dim=b.head_dim, block_size=b.block_size,
                max_blocks=b.max_blocks, kv_dtype=self.kv_dtype, num_blocks=self.num_blocks)
            # the decode work list from the same host-side plan (the engine builds it
            # per step and uploads it with the plan); None where the batch cannot
            # take one or a partition is not given
            w = None
            if WORK and d["P"]:
                w = self.K.ragged_work(
                    q_lens=b.q_lens, context_lens=b.context_lens, block_tables=b.block_tables,
                    num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
                    block_size=b.block_size, partition_size=d["P"], kv_dtype=self.kv_dtype,
                    num_blocks=self.num_blocks, max_q_len=int(b.q_lens.max()), pool_layout=POOL_LAYOUT,
                    chunk_partition_size=d["CP"])
            d["work"] = None if w is None else self.torch.from_numpy(w[0].view(np.int32)).to("cuda:0")
            d["work_chunk"] = 0 if w is None else w[1]
        self.K.ragged_paged_attention(
            self.ctx, q=d["q"], k_pool=self.k, v_pool=self.v, k_scales=self.ks, v_scales=self.vs,
            block_tables=d["tables"], cu_seqlens=d["cu"], context_lens=d["lens"], out=d["out"],
            num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
            block_size=b.block_size, scale=b.scale, kv_dtype=self.kv_dtype,
            num_blocks=self.num_blocks, max_q_len=int(b.q_lens.max()),
            pool_layout=POOL_LAYOUT, partition_size=d["P"], chunk_partition_size=d["CP"], work=d["work"],
            work_chunk_items=d["work_chunk"])

    def run(self, steps, warmup):
        torch = self.torch
        for i in range(warmup):
            self.call(i)
        # then at least ~0.3 s of the same work untimed, so clocks and caches are in
        # their steady state whatever the order of the measurements
        torch.cuda.synchronize()
        t_end = time.perf_counter() + 0.3
        i = warmup
        while time.perf_counter() < t_end:
            for _ in range(20):
                self.call(i)
                i += 1
            torch.cuda.synchronize()
        self.ctx.check_device_status()
        torch.cuda.synchronize()
        # throughput: the calls alone, no per-kernel events in the timed region
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            self.call(i)
        stop.record()
        torch.cuda.synchronize()
        total_ms = start.elapsed_time(stop)
        # per-kernel durations: a second pass with HIP events around each launch
        self.ctx.set_profiling(True)
        for i in range(steps):
            self.call(i)
        torch.cuda.synchronize()
        k_ms, k_n = self.ctx.kernel_time("attention")
        r_ms, r_n = self.ctx.kernel_time("reduce")
        self.ctx.set_profiling(False)
        self.ctx.check_device_status()
        rows = np.mean([b.total_q for b in self.batches])
        abytes = np.mean([b.algorithmic_bytes(self.kv_dtype) for b in self.batches])
        ms = total_ms / steps
        st1 = k_ms / max(k_n, 1)
        return dict(ms_per_step=ms, tokens_per_s=rows / (ms * 1e-3),
                    stage1_ms=st1, reduce_ms=r_ms / max(r_n, 1),
                    algorithmic_bytes=int(abytes),
                    stage1_gbps=abytes / (st1 * 1e-3) / 1e9,
                    call_gbps=abytes / (ms * 1e-3) / 1e9)


def config3_append(ab, steps=200):
    """Config 3's fused append + quantize of the step's new K/V rows (one token per
    sequence, written at its last position), timed alone (HIP events around each
    launch) and together with the attention call it precedes in a decode step.
    Algorithmic bytes per token: K and V f32 rows read, the slot read, the quantized
    rows and their scales written."""
    torch, K, ctx = ab.torch, ab.K, ab.ctx
    b0 = ab.batches[0]
    hkv, d, bs = b0.num_kv_heads, b0.head_dim, b0.block_size
    g = torch.Generator(device="cuda:0")
    g.manual_seed(33)
    calls = []
    for b in ab.batches:
        last = b.context_lens - 1
        blk = b.block_tables[np.arange(b.num_seqs), last // bs].astype(np.int64)
        slots = torch.from_numpy(blk * bs + last % bs).to("cuda:0")
        kk = torch.randn(b.num_seqs * hkv * d, generator=g, device="cuda:0")
        calls.append((slots, kk, torch.randn_like(kk)))

    def append(i):
        slots, kk, vv = calls[i % len(calls)]
        K.kv_append(ctx, ab.kv_dtype, kk, vv, slots, ab.num_blocks, bs, hkv, d, ab.k, ab.v, ab.ks, ab.vs)

    for i in range(10):
        append(i)
    torch.cuda.synchronize()
    ctx.set_profiling(True)
    for i in range(steps):
        append(i)
    torch.cuda.synchronize()
    a_ms, a_n = ctx.kernel_time("append")
    ctx.set_profiling(False)
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for i in range(steps):
        append(i)
        ab.call(i)
    e_ev.record()
    torch.cuda.synchronize()
    ctx.check_device_status()
    n_tok = b0.num_seqs
    scale_b = (2 * hkv * (d // 32) * 2) if ab.kv_dtype == K.KANSO_KV_Q8_0 else 2 * hkv * 4
    per_tok = 2 * hkv * d * 4 + 8 + 2 * hkv * d + scale_b
    us = a_ms / max(a_n, 1) * 1e3
    return dict(tokens=n_tok, us=round(us, 2), bytes_per_token=per_tok,
                gbps=round(n_tok * per_tok / (us * 1e-6) / 1e9, 1),
                hbm_frac=round(n_tok * per_tok / (us * 1e-6) / HBM_PEAK, 5),
                ms_per_step_append_plus_attention=round(s_ev.elapsed_time(e_ev) / steps, 4),
                timing="append: HIP events around each launch; step: one event pair around "
                       "append + attention calls")


def copy_bandwidth(torch, nbytes=2 << 30, iters=10):
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").normal_()
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / iters
    return 2 * nbytes / (ms * 1e-3) / 1e9


def gemv_bench(ctx, torch, K, oracle_mod, quick):
    """Q8_0 / Q4_K GEMV at the SmolLM2 projection shapes; each timing rotates over
    weight copies totalling > 1 GB. kind q8_0: GGUF blocks (kanso_gemv_q8_0);
    q8_0_packed: the same bytes in the decoder's packed layout (kanso_gemm_q8_0)."""
    dev = torch.device("cuda:0")
    shapes = [("q", 960, 960), ("kv", 320, 960), ("gate_up", 2560, 960), ("down", 960, 2560)]
    out = []
    for kind in ("q8_0", "q8_0_packed", "q4_k"):
        for name, rows, cols in shapes:
            cols_eff = cols if kind != "q4_k" or cols % 256 == 0 else 1024
            label = name if cols_eff == cols else name + "_padded"
            rng = np.random.default_rng(rows + cols)
            wf = (rng.standard_normal((rows, cols_eff)) * 0.02).astype(np.float32)
            if cols_eff != cols:
                wf[:, cols:] = 0.0
            w = (oracle_mod.quantize_row_q8_0(wf) if kind != "q4_k"
                 else oracle_mod.quantize_row_q4_k(wf))
            one = torch.from_numpy(w).to(dev)
            if kind == "q8_0_packed":
                one = K.pack_q8_0_matrix(ctx, one, rows, cols_eff)
            wbytes = one.numel()
            copies = max(32, int((1.1e9) // wbytes) + 1)
            arena = one.repeat(copies)
            fn = {"q8_0": K.gemv_q8_0, "q8_0_packed": K.gemm_q8_0, "q4_k": K.gemv_q4_k}[kind]
            for batch in ([1, 8, 32] if quick else [1, 4, 8, 16, 32]):
                x = torch.randn(batch * cols_eff, device=dev)
                y = torch.empty(batch * rows, device=dev)
                for i in range(4):
                    fn(ctx, arena[i * wbytes:(i + 1) * wbytes], x, y, rows, cols_eff)
                torch.cuda.synchronize()
                n = min(copies, 200)
                # us: HIP events around each launch on its stream (kernel duration
                # plus event overhead); us_back_to_back: one event pair around n
                # eager launches, bounded by the host's submission rate
                ctx.set_profiling(True)
                for i in range(n):
                    fn(ctx, arena[i * wbytes:(i + 1) * wbytes], x, y, rows, cols_eff)
                g_ms, g_n = ctx.kernel_time("gemv")
                ctx.set_profiling(False)
                us = g_ms / max(g_n, 1) * 1e3
                s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s_ev.record()
                for i in range(n):
                    fn(ctx, arena[i * wbytes:(i + 1) * wbytes], x, y, rows, cols_eff)
                e_ev.record()
                torch.cuda.synchronize()
                us_b2b = s_ev.elapsed_time(e_ev) / n * 1e3
                abytes = w.size + batch * (cols_eff + rows) * 4  # stored GGUF bytes
                out.append(dict(kind=kind, shape=label, out=rows, inp=cols_eff, batch=batch,
                                us=round(us, 2), us_back_to_back=round(us_b2b, 2), gbps=round(abytes / (us * 1e-6) / 1e9, 1),
                                frac=round(abytes / (us * 1e-6) / HBM_PEAK, 4)))
            del arena
            torch.cuda.empty_cache()
    return out


def engine_bench(ctx, K, torch, num_requests=64, kv_dtype=0):
    """Config 5: SmolLM2-360M-architecture random-init model (32 layers, Q8_0 weights
    N(0, 0.02^2), tied embeddings, F32 KV) under the C++ continuous-batching engine:
    512-token budget, max_running 64, block size 16, greedy. Value = generated
    tokens / wall seconds of the whole run (execute_engine_run, src/bench.rs:447-537).
    kv_dtype != 0: the same run on a 1-byte pool (Engine::new_with_budget_and_kv)."""
    from kanso_infer_amd import workloads
    from kanso_infer_amd.engine import Engine, Model, ModelConfig, run_benchmark_workload
    cfg = ModelConfig.smollm2_360m(max_position=4096)
    t0 = time.perf_counter()
    model = Model(ctx, cfg)
    model.init_random(seed=0x5EED0057, std=0.02)
    reqs = workloads.config5_workload(num_requests=num_requests)
    total_blocks = workloads.config5_total_blocks(reqs)
    model.alloc_kv(total_blocks, 16, 512, 65, kv_dtype=kv_dtype)
    log(f"config5: model ready in {time.perf_counter() - t0:.1f} s, {total_blocks} KV blocks")
    # warm-up on a throwaway engine (same model and pool), so first-call costs stay out
    warm = Engine(model, 64, total_blocks, 16, 512)
    from kanso_infer_amd.engine import TraceEntry
    run_benchmark_workload(warm, [TraceEntry(300, 8, 0), TraceEntry(40, 8, 0), TraceEntry(600, 4, 1)])
    warm.close()
    eng = Engine(model, 64, total_blocks, 16, 512)
    kv_tok = cfg.kv_cache_bytes_per_token_f32()
    if kv_dtype:  # 1-byte elements plus the row scales (f32 per row; f16 per 32 for Q8_0)
        d = cfg.head_dim
        row = d + 4 if kv_dtype in (K.KANSO_KV_INT8, K.KANSO_KV_FP8) else d + 2 * d // 32
        kv_tok = kv_tok * row // (4 * d)
    wbytes = cfg.weight_bytes_q8_0()
    acc = dict(kv_bytes=0, steps_with_work=0, tokens=0, max_batch=0, step_times=[])

    def on_step(e, outs):
        plan = e.last_plan()
        if plan["context_lens"].size:
            acc["kv_bytes"] += int(plan["context_lens"].astype(np.int64).sum()) * kv_tok
            acc["steps_with_work"] += 1
            acc["tokens"] += int(plan["query_lens"].sum())
            acc["max_batch"] = max(acc["max_batch"], int(plan["context_lens"].size))

    rep = run_benchmark_workload(eng, reqs, on_step=on_step)
    # every step with work reads all weights once and each sequence's whole context
    step_bytes = acc["kv_bytes"] + acc["steps_with_work"] * wbytes
    out = {
        "metric": "batched decode tok/s (config 5, continuous batching)",
        "tokens_per_s": round(rep["total_tokens_per_sec"], 1),
        "generated_tokens": rep["total_tokens"],
        "processed_tokens": acc["tokens"],
        "wall_s": round(rep["total_duration_secs"], 3),
        "steps": rep["steps"],
        "steps_with_work": acc["steps_with_work"],
        "ms_per_step": round(1000 * rep["total_duration_secs"] / max(rep["steps"], 1), 3),
        "decode_ms_per_step": round(rep["decode_ms_per_step"], 3),
        "max_sequences_per_step": acc["max_batch"],
        "checksum_fnv1a64": f"{rep['checksum']:016x}",
        "checksum_oracle": config5_oracle_fixture(rep["generated"]) if kv_dtype == 0 and num_requests == 64 else None,
        "prefix_hit_rate": round(rep["prefix_hit_rate"], 4),
        "bytes_read_per_step": int(step_bytes / max(acc["steps_with_work"], 1)),
        "hbm_frac": round(step_bytes / rep["total_duration_secs"] / HBM_PEAK, 4),
        "workload": f"{len(reqs)} requests, prompt log-uniform [16,2048], gen U[32,512], Poisson "
                    "40 req/s at 5 ms/step, budget 512, max_running 64, bs 16, greedy; "
                    "SmolLM2-360M shape (32 L, 960, GQA 15:5, 2560, vocab 49152), Q8_0 weights "
                    "random N(0,0.02^2), F32 KV",
    }
    eng.close()
    model.close()
    return out


def verify_bench(ctx, K, torch, num_seqs=16, context=1000, rows=5, reps=20):
    """Speculative verify rows (forward_batch_all_rows, src/model.rs:1382-1410) on the
    config-5 model: num_seqs sequences with `context` cached tokens each score `rows`
    candidate tokens in one step (every row through the lm_head and greedy argmax),
    against a plain decode step of the same sequences (one row each)."""
    from kanso_infer_amd.engine import Model, ModelConfig
    cfg = ModelConfig.smollm2_360m(max_position=4096)
    model = Model(ctx, cfg)
    model.init_random(seed=0x5EED0057, std=0.02)
    per_seq = -(-(context + rows) // 16)
    model.alloc_kv(num_seqs * per_seq, 16, 512, 65)
    rng = np.random.default_rng(0x5EED0090)
    tables = [np.arange(s * per_seq, (s + 1) * per_seq, dtype=np.uint32) for s in range(num_seqs)]
    toks = [rng.integers(0, cfg.vocab_size, context + rows).astype(np.uint32) for _ in range(num_seqs)]

    def step(seqs):  # seqs: (s, start, q_len)
        plan, arena, tabs = [], [], []
        for s, start, ql in seqs:
            plan.append([start, ql, len(tabs), per_seq, (len(arena) - start) % (1 << 32)])
            arena.extend(toks[s][start:start + ql])
            tabs.extend(tables[s])
        return np.array(plan, np.uint32), np.array(arena, np.uint32), np.array(tabs, np.uint32)

    for s in range(num_seqs):  # prefill in chunks under the 512-token budget
        for lo in range(0, context, 500):
            model.forward(*step([(s, lo, min(500, context - lo))]))
    dec = step([(s, context, 1) for s in range(num_seqs)])
    ver = step([(s, context, rows) for s in range(num_seqs)])

    def timed(fn, args):
        # at least 0.5 s of the same call first: the first process on a fresh box ran
        # its first seconds at about half speed
        t_end = time.perf_counter() + 0.5
        while time.perf_counter() < t_end:
            fn(*args)
        t0 = time.perf_counter()
        for _ in range(reps):
            fn(*args)
        return (time.perf_counter() - t0) / reps

    t_dec = timed(model.forward, dec)
    t_ver = timed(model.forward_all_rows, ver)
    model.close()
    return dict(sequences=num_seqs, context=context, rows_per_sequence=rows,
                decode_step_ms=round(t_dec * 1e3, 3), verify_step_ms=round(t_ver * 1e3, 3),
                verify_rows_per_s=round(num_seqs * rows / t_ver, 1),
                verify_over_decode=round(t_ver / t_dec, 3),
                timing="host wall clock per synchronous forward (the entry point synchronises)")


def config5_cpu_baseline(threads=None):
    """The oracle (C++ restatement of the reference CPU path, OpenMP) running the full
    SmolLM2-360M-shape model: one decode step of 16 sequences with contexts
    U[128, 1024] over a paged F32 pool. A bounded sample of config 5's work: a full
    run would take hours on the host."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import engine_ref
    from model_ref import OracleModel, random_weights
    threads = threads or min(os.cpu_count() or 1, 16)
    cfg = dict(hidden=960, num_heads=15, num_kv_heads=5, head_dim=64, num_layers=32,
               intermediate=2560, vocab=49152)
    t0 = time.perf_counter()
    w = random_weights(cfg, seed=1)
    rng = np.random.default_rng(2)
    S = 16
    ctx = rng.integers(128, 1025, S)
    need = (ctx + 15) // 16
    nblocks = int(need.sum())
    om = OracleModel(cfg, w, nblocks, 16, nthreads=threads)
    for a in om.k + om.v:
        a[:] = rng.standard_normal(a.size, dtype=np.float32)
    plan = engine_ref.StepPlan([], [], [], [], [], [], [], [])
    off = 0
    for s in range(S):
        table = list(range(off, off + int(need[s])))
        off += int(need[s])
        pos = int(ctx[s]) - 1
        plan.tokens.append(int(rng.integers(0, cfg["vocab"])))
        plan.positions.append(pos)
        plan.slot_mapping.append(table[pos // 16] * 16 + pos % 16)
        plan.block_tables.append(table)
        plan.context_lens.append(int(ctx[s]))
        plan.query_lens.append(1)
        plan.request_ids.append(s + 1)
    setup = time.perf_counter() - t0
    t1 = time.perf_counter()
    om.logits(plan)
    el = time.perf_counter() - t1
    return dict(value=round(S / el, 2), unit="tokens/s", cores=threads, kind="port",
                sample=f"one decode step, 16 sequences, contexts U[128,1024] (mean {ctx.mean():.0f}), "
                       f"32 layers, {el:.1f} s on {threads} threads (setup {setup:.1f} s)")


def config5_oracle_fixture(generated):
    """The oracle engine's token stream of this very run (32 layers, the 64-request
    trace, budget 512, the same init weights), committed by
    tests/golden/make_config5_checksum.py, against the GPU run's tokens."""
    path = ROOT / "tests" / "golden" / "config5_oracle.json"
    if not path.exists():
        return dict(available=False, reason=f"{path.name} not generated")
    info = json.loads(path.read_text())
    want = np.load(path.with_name("config5_oracle_tokens.npy"))
    got = np.asarray(generated, np.uint32)
    n = min(got.size, want.size)
    diff = np.flatnonzero(got[:n] != want[:n])
    return dict(oracle=info["checksum"], match=bool(got.size == want.size and diff.size == 0),
                tokens=int(want.size), first_difference=int(diff[0]) if diff.size else None,
                workload="the full config-5 run: 32 layers, 64 requests, budget 512 (oracle engine on the "
                         "host restatement of kanso_model_init_random's weights)")


def config5_checksum_parity(ctx, K, torch, kv_dtype=0):
    """Greedy token streams of the GPU engine and of the oracle engine (scheduler
    restatement + CPU forward) on the same random-init weights: SmolLM2 widths, 4 of
    the 32 layers, 6 requests with bench.rs-pattern and random prompts, chunked
    prefill (budget 64). Returns both FNV-1a checksums."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import engine_ref
    import oracle as oracle_mod
    from kanso_infer_amd.engine import Engine, Model, ModelConfig, fnv1a_64
    from model_ref import OracleModel, random_weights
    cfg = dict(hidden=960, num_heads=15, num_kv_heads=5, head_dim=64, num_layers=4,
               intermediate=2560, vocab=49152)
    w = random_weights(cfg, seed=9)
    bs, budget, total_blocks, max_running = 16, 64, 64, 4
    gm = Model(ctx, ModelConfig(960, 15, 5, 4, 2560, 49152, max_position=4096))
    gm.load_weights(w)
    gm.alloc_kv(total_blocks, bs, budget, max_running + 1, kv_dtype=kv_dtype)
    eng = Engine(gm, max_running, total_blocks, bs, budget)
    om = OracleModel(cfg, w, total_blocks, bs, nthreads=min(os.cpu_count() or 1, 16),
                     kv_dtype=kv_dtype)
    ref = engine_ref.Engine(om.forward, max_running, total_blocks, bs, budget,
                            reset_block=om.reset_block)
    rng = np.random.default_rng(7)
    reqs = []
    for i in range(6):
        plen = int(rng.integers(3, 60))
        prompt = ([(i % 3 * 10 + p) % 30 for p in range(plen)] if i % 2 == 0
                  else rng.integers(0, cfg["vocab"], plen).tolist())
        reqs.append((prompt, int(rng.integers(4, 20)), int(rng.integers(0, 6))))
    order = sorted(range(len(reqs)), key=lambda i: reqs[i][2])
    nxt = step = 0
    a_tok, b_tok = [], []
    while True:
        while nxt < len(order) and reqs[order[nxt]][2] <= step:
            p, g, _ = reqs[order[nxt]]
            eng.add_request(p, g)
            ref.add_request(p, g)
            nxt += 1
        if nxt >= len(order) and not eng.has_unfinished_requests():
            break
        a_tok.extend(o.token_id for o in eng.step())
        b_tok.extend(t for _, t, _ in ref.step())
        step += 1
    eng.close()
    gm.close()
    return dict(gpu=f"{fnv1a_64(a_tok):016x}", oracle=f"{oracle_mod.fnv1a_64(b_tok):016x}",
                match=a_tok == b_tok, tokens=len(a_tok), steps=step,
                workload="SmolLM2 widths, 4 layers, 6 requests, budget 64, max_running 4, "
                         "pool 64 blocks")


TRAFFIC_PROFILE = ROOT / "profiles" / "attention_config2_hbm_traffic.md"


def profiled_traffic():
    """HBM bytes per headline call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (calibrated against a copy of known size), or None if absent."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        return None
    return None


def cpu_baseline(batch, seconds=12.0, nthreads=1):
    """Oracle (C++ restatement of the reference CPU path) on the headline batch, on
    `nthreads` host threads (OpenMP over (row, KV head)), over a pool compacted to
    exactly the blocks the batch reads."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as oracle_mod
    ids = np.unique(batch.block_tables)
    lut = np.zeros(int(ids.max()) + 1, np.uint32)
    lut[ids] = np.arange(ids.size, dtype=np.uint32)
    tables = lut[batch.block_tables]
    rng = np.random.default_rng(1)
    n = ids.size * batch.block_size * batch.num_kv_heads * batch.head_dim
    k = rng.standard_normal(n, dtype=np.float32)
    v = rng.standard_normal(n, dtype=np.float32)
    q = rng.standard_normal(batch.total_q * batch.num_heads * batch.head_dim, dtype=np.float32)
    kw = dict(num_heads=batch.num_heads, num_kv_heads=batch.num_kv_heads,
              head_dim=batch.head_dim, block_size=batch.block_size, scale=batch.scale,
              num_blocks=int(ids.size))
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle_mod.ragged_attention(q, k, v, tables, batch.cu_seqlens, batch.context_lens,
                                    nthreads=nthreads, **kw)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds or calls >= 100:
            break
    per_call = el / calls
    who = "single thread" if nthreads == 1 else f"{nthreads} threads"
    return dict(value=round(batch.total_q / per_call, 1), unit="tokens/s", cores=nthreads, kind="port",
                sample=f"{calls} oracle calls on the headline batch ({batch.total_q} query rows, "
                       f"{batch.num_seqs} sequences), {who}, {el:.1f} s",
                ms_per_call=round(per_call * 1e3, 2))


def reference_probes(ctx, torch, K, copy_gbps, copies=32, calls=200):
    """The reference's own budget probes (src/bench/probes.rs), on this device.

    paged_attn_ctx4096_b1: kanso_paged_attention_v2 at ctx 4096 / batch 1 with the
    SmolLM2 geometry (heads = KV heads = 5, D = 64, probes.rs:112-139, q / K / V = 0.01),
    time per call over the floor 2 * ctx * Hkv * D * 4 B / peak (the gate asks <= 2.0).
    gemv_q8_0_1024: 1024 x 1024 Q8_0 GEMV of d = 0.01, qs = 1 blocks with x = 1
    (probes.rs:59-87): weight bytes / time as a share of peak (the gate asks >= 60%).
    Both rotate over distinct buffers (no Infinity Cache reuse) and divide by the
    nominal 8 TB/s and by the copy bandwidth measured in this run."""
    dev = torch.device("cuda:0")
    ctx_len, hkv, d, bs = 4096, 5, 64, 16
    blocks = ctx_len // bs
    params = K.PagedAttentionParams(1, hkv, hkv, d, bs, blocks, 1.0 / np.sqrt(d))
    per = blocks * bs * hkv * d
    kp = torch.full((copies * per,), 0.01, device=dev)
    vp = torch.full_like(kp, 0.01)
    q = torch.full((hkv * d,), 0.01, device=dev)
    out = torch.empty_like(q)
    lens = torch.tensor([ctx_len], dtype=torch.int32, device=dev)
    tabs = [torch.arange(i * blocks, (i + 1) * blocks, dtype=torch.int32, device=dev) for i in range(copies)]
    for i in range(4):
        K.paged_attention_v2(ctx, params, q, kp, vp, tabs[i], lens, out)
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for i in range(calls):
        K.paged_attention_v2(ctx, params, q, kp, vp, tabs[i % copies], lens, out)
    e_ev.record()
    torch.cuda.synchronize()
    attn_us = s_ev.elapsed_time(e_ev) / calls * 1e3
    floor_bytes = 2 * ctx_len * hkv * d * 4
    del kp, vp
    # GEMV probe
    blk = np.concatenate([np.array([0.01], np.float16).view(np.uint8), np.ones(32, np.uint8)])
    wbytes = 1024 * 1024 // 32 * 34
    ncopy = int(1.1e9 // wbytes) + 1
    arena = torch.from_numpy(np.tile(blk, 1024 * 1024 // 32)).to(dev).repeat(ncopy)
    x = torch.ones(1024, device=dev)
    y = torch.empty(1024, device=dev)
    for i in range(4):
        K.gemv_q8_0(ctx, arena[i * wbytes:(i + 1) * wbytes], x, y, 1024, 1024)
    torch.cuda.synchronize()
    ctx.set_profiling(True)
    for i in range(calls):
        K.gemv_q8_0(ctx, arena[(i % ncopy) * wbytes:((i % ncopy) + 1) * wbytes], x, y, 1024, 1024)
    g_ms, g_n = ctx.kernel_time("gemv")
    ctx.set_profiling(False)
    gemv_us = g_ms / max(g_n, 1) * 1e3
    assert abs(float(y[0]) - float(np.float16(0.01)) * 1024) < 1e-2  # probes.rs closed form
    del arena
    torch.cuda.empty_cache()
    return dict(
        paged_attn_ctx4096_b1=dict(us_per_call=round(attn_us, 2),
                                   over_floor_8tbs=round(attn_us * 1e-6 / (floor_bytes / HBM_PEAK), 2),
                                   over_floor_measured=round(attn_us * 1e-6 / (floor_bytes / (copy_gbps * 1e9)), 2),
                                   gate="<= 2.0", timing="back-to-back calls, one event pair"),
        gemv_q8_0_1024=dict(us=round(gemv_us, 2),
                            pct_of_8tbs=round(wbytes / (gemv_us * 1e-6) / HBM_PEAK * 100, 2),
                            pct_of_measured=round(wbytes / (gemv_us * 1e-6) / (copy_gbps * 1e9) * 100, 2),
                            gate=">= 60", timing="HIP events around each launch"))


def gemm_probe(ctx, torch, K, oracle_mod, launches=10):
    """Launches only, for a rocprofv3 counter pass: the packed Q8_0 product at the
    SmolLM2 shapes (q, gate+up, down) at 16, 32 and 512 tokens, and the GGUF-layout
    GEMV at batch 32, `launches` times each."""
    dev = torch.device("cuda:0")
    for name, rows, cols in (("q", 960, 960), ("gate_up", 5120, 960), ("down", 960, 2560)):
        rng = np.random.default_rng(rows)
        w = oracle_mod.quantize_row_q8_0((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        wd = torch.from_numpy(w).to(dev)
        pk = K.pack_q8_0_matrix(ctx, wd, rows, cols)
        for T in (16, 32, 512):
            x, y = torch.randn(T * cols, device=dev), torch.empty(T * rows, device=dev)
            for _ in range(launches):
                K.gemm_q8_0(ctx, pk, x, y, rows, cols)
        x, y = torch.randn(32 * cols, device=dev), torch.empty(32 * rows, device=dev)
        for _ in range(launches):
            K.gemv_q8_0(ctx, wd, x, y, rows, cols)
        torch.cuda.synchronize()


def gemv_pass(ctx, torch, K, oracle_mod, launches=12):
    """Launches only, for rocprofv3 (kernel trace, FETCH_SIZE, WRITE_SIZE): the
    config-4 GEMVs (q8_0 GGUF blocks, q8_0 packed, q4_k; the SmolLM2 shapes; batch 1,
    8 and 32), each `launches` times over rotating weight copies (> 1 GB, so every
    launch reads cold weights), after a PMC_COPY_BYTES calibration copy. Prints the
    launch order, one line per (kind, shape, batch), for matching the dispatches."""
    dev = torch.device("cuda:0")
    a = torch.empty(PMC_COPY_BYTES // 4, dtype=torch.float32, device=dev).normal_()
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    shapes = [("q", 960, 960), ("kv", 320, 960), ("gate_up", 2560, 960), ("down", 960, 2560)]
    for kind in ("q8_0", "q8_0_packed", "q4_k"):
        for name, rows, cols in shapes:
            cols_eff = cols if kind != "q4_k" or cols % 256 == 0 else 1024
            rng = np.random.default_rng(rows + cols)
            wf = (rng.standard_normal((rows, cols_eff)) * 0.02).astype(np.float32)
            w = (oracle_mod.quantize_row_q8_0(wf) if kind != "q4_k"
                 else oracle_mod.quantize_row_q4_k(wf))
            one = torch.from_numpy(w).to(dev)
            if kind == "q8_0_packed":
                one = K.pack_q8_0_matrix(ctx, one, rows, cols_eff)
            wbytes = one.numel()
            copies = int(1.1e9 // wbytes) + 1
            arena = one.repeat(copies)
            fn = {"q8_0": K.gemv_q8_0, "q8_0_packed": K.gemm_q8_0, "q4_k": K.gemv_q4_k}[kind]
            for batch in (1, 8, 32):
                x = torch.randn(batch * cols_eff, device=dev)
                y = torch.empty(batch * rows, device=dev)
                torch.cuda.synchronize()
                print(json.dumps(dict(kind=kind, shape=name, out=rows, inp=cols_eff, batch=batch,
                                      weight_bytes=wbytes, launches=launches)), flush=True)
                for i in range(launches):
                    fn(ctx, arena[i * wbytes:(i + 1) * wbytes], x, y, rows, cols_eff)
                torch.cuda.synchronize()
            del arena
            torch.cuda.empty_cache()


def host_bandwidth(threads):
    """STREAM triad of the host (the oracle library, OpenMP), 1 thread and `threads`."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as oracle_mod
    return dict(stream_triad_gbps_1_thread=round(oracle_mod.stream_triad_gbps(1 << 26, 1), 1),
                stream_triad_gbps=round(oracle_mod.stream_triad_gbps(1 << 26, threads), 1),
                threads=threads, array_mib=512)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only: skip extras")
    ap.add_argument("--skip-gemv", action="store_true", help="skip the GEMV table")
    ap.add_argument("--skip-config5", action="store_true", help="skip the config-5 engine run")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="short run for rocprofv3 --pmc: a 512 MiB copy (calibration) then 20 "
                         "headline attention calls; prints nothing else")
    ap.add_argument("--pool-layout", choices=("token", "head"), default="token",
                    help="row order inside a KV block for the attention benchmarks")
    ap.add_argument("--verify-only", action="store_true",
                    help="only the speculative verify-step timing (one JSON line)")
    ap.add_argument("--config5-only", action="store_true",
                    help="run only the config-5 engine benchmark and print its JSON")
    ap.add_argument("--config5-kv", choices=("f32", "int8", "fp8", "q8_0"), default="f32",
                    help="KV pool kind of the --config5-only run")
    ap.add_argument("--partition", type=int, default=0,
                    help="split-K partition of the attention benchmarks: 0 = from the batch's "
                         "lengths (kanso_ragged_partition_size), -1 = the library's own choice")
    ap.add_argument("--no-work", action="store_true",
                    help="attention calls without the decode work list (the table-driven path)")
    ap.add_argument("--chunk-partition", type=int, default=0,
                    help="fixed partition of the MFMA chunk rows (a multiple of 32; 0 = the "
                         "library's rule)")
    ap.add_argument("--gemv-pass", action="store_true",
                    help="config-4 GEMV launches only (cold weights), for rocprofv3 kernel-trace "
                         "and FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="launches of the Q8_0 products only (for a rocprofv3 counter pass)")
    ap.add_argument("--decode-only", action="store_true",
                    help="also time the headline batches' decode rows alone")
    args = ap.parse_args()
    global POOL_LAYOUT, PARTITION, CHUNK_PARTITION, WORK
    POOL_LAYOUT = 1 if args.pool_layout == "head" else 0
    PARTITION = args.partition
    CHUNK_PARTITION = args.chunk_partition
    WORK = not args.no_work
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU component (the path "
              "would shard by sequences, one engine and KV pool per GPU); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import kanso_infer_amd as K
    from kanso_infer_amd import workloads

    ctx = K.Context(0)
    if args.gemv_pass:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as oracle_mod
        gemv_pass(ctx, torch, K, oracle_mod)
        ctx.close()
        return
    if args.gemm_probe:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as oracle_mod
        gemm_probe(ctx, torch, K, oracle_mod)
        ctx.close()
        return
    if args.verify_only:
        print(json.dumps(verify_bench(ctx, K, torch)), flush=True)
        ctx.close()
        return
    if args.config5_only:
        kv = {"f32": K.KANSO_KV_F32, "int8": K.KANSO_KV_INT8, "fp8": K.KANSO_KV_FP8,
              "q8_0": K.KANSO_KV_Q8_0}[args.config5_kv]
        r5 = engine_bench(ctx, K, torch, kv_dtype=kv)
        r5["checksum_parity"] = config5_checksum_parity(ctx, K, torch, kv_dtype=kv)
        if not args.no_cpu:
            r5["cpu_baseline"] = config5_cpu_baseline()
        ctx.close()
        print(json.dumps(r5), flush=True)
        return
    log("building headline batches (config 2, 64k-block pool)")
    nb = 65536
    head = [workloads.config2_mixed(num_blocks=nb, seed_offset=i) for i in range(8)]
    hb = AttnBench(ctx, head, K.KANSO_KV_F32, seed=2)
    if args.pmc_pass:
        # Calibration: torch's copy kernel moving exactly PMC_COPY_BYTES each way.
        a = torch.empty(PMC_COPY_BYTES // 4, dtype=torch.float32, device="cuda:0").normal_()
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        for i in range(20):
            hb.call(i)
        torch.cuda.synchronize()
        ctx.check_device_status()
        ctx.close()
        return
    res = hb.run(args.steps, args.warmup)
    log(f"config2: {res}")

    extras = {}
    extras["partitions"] = [d["P"] for d in hb.dev_batches]
    extras["work_list"] = [d["work"] is not None for d in hb.dev_batches]
    if WORK and not args.quick:
        # the same batches through the table-driven path (no work list)
        WORK = False
        tp = AttnBench.__new__(AttnBench)
        tp.__dict__.update(hb.__dict__)
        tp.dev_batches = [{k: v for k, v in d.items() if k not in ("P", "work", "work_chunk")} for d in hb.dev_batches]
        rt = tp.run(args.steps, args.warmup)
        WORK = True
        extras["headline_table_path"] = dict(
            tokens_per_s=round(rt["tokens_per_s"], 1), ms_per_step=round(rt["ms_per_step"], 5),
            stage1_gbps=round(rt["stage1_gbps"], 1),
            hbm_frac_stage1=round(rt["stage1_gbps"] * 1e9 / HBM_PEAK, 4))
        log(f"config2, table path: {extras['headline_table_path']}")
    if not args.quick and PARTITION == 0:
        # the same batches with the library's own partition (no host lengths)
        PARTITION = -1
        lib = AttnBench.__new__(AttnBench)
        lib.__dict__.update(hb.__dict__)
        lib.dev_batches = [{k: v for k, v in d.items() if k not in ("P", "work", "work_chunk")} for d in hb.dev_batches]
        rl = lib.run(args.steps, args.warmup)
        PARTITION = 0
        extras["headline_library_partition"] = dict(
            tokens_per_s=round(rl["tokens_per_s"], 1), ms_per_step=round(rl["ms_per_step"], 5),
            stage1_gbps=round(rl["stage1_gbps"], 1),
            partitions=[d["P"] for d in lib.dev_batches])
        log(f"config2, library partition: {extras['headline_library_partition']}")
    if args.decode_only:
        dec = [workloads.config2_mixed(num_chunks=0, num_blocks=nb, seed_offset=i) for i in range(8)]
        hd = AttnBench.__new__(AttnBench)
        hd.__dict__.update(hb.__dict__)
        hd.batches = dec
        hd.dev_batches = []
        for b in dec:
            q = torch.randn(b.total_q * b.num_heads * b.head_dim, device="cuda:0")
            hd.dev_batches.append(dict(
                q=q, out=torch.empty_like(q),
                tables=torch.from_numpy(b.block_tables.ravel().view(np.int32)).cuda(),
                cu=torch.from_numpy(b.cu_seqlens).cuda(),
                lens=torch.from_numpy(b.context_lens.astype(np.int32)).cuda()))
        rd = hd.run(args.steps, args.warmup)
        extras["config2_decode_rows_only"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                              for k, v in rd.items()}
        log(f"config2 decode rows only: {rd}")
    if not args.quick:
        s64 = [workloads.config2_mixed(num_decodes=60, num_blocks=nb, seed_offset=100 + i)
               for i in range(8)]
        # same pool, different batches: reuse the pool of the headline
        hb64 = AttnBench.__new__(AttnBench)
        hb64.__dict__.update(hb.__dict__)
        hb64.batches = s64
        hb64.dev_batches = []
        g = torch.Generator(device="cuda:0")
        g.manual_seed(64)
        for b in s64:
            q = torch.randn(b.total_q * b.num_heads * b.head_dim, generator=g, device="cuda:0")
            hb64.dev_batches.append(dict(
                q=q, out=torch.empty_like(q),
                tables=torch.from_numpy(b.block_tables.ravel().view(np.int32)).cuda(),
                cu=torch.from_numpy(b.cu_seqlens).cuda(),
                lens=torch.from_numpy(b.context_lens.astype(np.int32)).cuda()))
        r64 = hb64.run(args.steps, args.warmup)
        extras["config2_64seq"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                   for k, v in r64.items()}
        extras["config2_64seq"]["hbm_frac_stage1"] = round(r64["stage1_gbps"] * 1e9 / HBM_PEAK, 4)
        log(f"config2 64-seq: {r64}")
        del hb64
        del hb.k, hb.v
        torch.cuda.empty_cache()

        c1 = [workloads.config1_decode(seed_offset=i) for i in range(8)]
        # config 1 pools hold only the needed blocks; rotate 8 batches over a shared
        # large pool instead so timings are not cache-resident
        for b in c1:
            b.num_blocks = nb
        rng = np.random.default_rng(5)
        for b in c1:
            need = (b.context_lens + 15) // 16
            ids = rng.choice(nb, size=int(need.sum()), replace=False).astype(np.uint32)
            off = 0
            for s, n_ in enumerate(need):
                b.block_tables[s, :n_] = ids[off:off + n_]
                b.block_tables[s, n_:] = ids[off + n_ - 1]
                off += n_
        b1 = AttnBench(ctx, c1, K.KANSO_KV_F32, seed=1)
        r1 = b1.run(args.steps, args.warmup)
        extras["config1_decode"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                    for k, v in r1.items()}
        log(f"config1: {r1}")
        del b1
        torch.cuda.empty_cache()

        for kv, name in ((K.KANSO_KV_INT8, "config3_int8"), (K.KANSO_KV_Q8_0, "config3_q8_0"),
                         (K.KANSO_KV_FP8, "config3_fp8")):
            c3 = [workloads.config3_quant_decode(num_blocks=131072, seed_offset=i) for i in range(8)]
            b3 = AttnBench(ctx, c3, kv, seed=3)
            r3 = b3.run(args.steps, args.warmup)
            r3["hbm_frac_stage1"] = r3["stage1_gbps"] * 1e9 / HBM_PEAK
            extras[name] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r3.items()}
            extras[name]["append"] = config3_append(b3, args.steps)
            log(f"{name}: {extras[name]}")
            del b3
            torch.cuda.empty_cache()

        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as oracle_mod
        if not args.skip_gemv:
            extras["gemv"] = gemv_bench(ctx, torch, K, oracle_mod, quick=False)
        extras["copy_kernel_gbps"] = round(copy_bandwidth(torch), 1)
        extras["reference_probes"] = reference_probes(ctx, torch, K, extras["copy_kernel_gbps"])
        log(f"reference probes: {extras['reference_probes']}")
        torch.cuda.empty_cache()
    if not args.quick and not args.skip_config5:
        extras["verify_rows"] = verify_bench(ctx, K, torch)
        log(f"verify rows: {extras['verify_rows']}")
        extras["config5_engine"] = engine_bench(ctx, K, torch)
        log(f"config5: {extras['config5_engine']}")
        extras["config5_engine"]["checksum_parity"] = config5_checksum_parity(ctx, K, torch)
        log(f"config5 parity: {extras['config5_engine']['checksum_parity']}")
        # the same run with an INT8 pool (the reference's kv_mode = Int8)
        r8 = engine_bench(ctx, K, torch, kv_dtype=K.KANSO_KV_INT8)
        r8["checksum_parity"] = config5_checksum_parity(ctx, K, torch, kv_dtype=K.KANSO_KV_INT8)
        extras["config5_engine_int8_kv"] = {k: v for k, v in r8.items() if k != "workload"}
        log(f"config5 int8 kv: {extras['config5_engine_int8_kv']}")
        if not args.no_cpu:
            extras["config5_engine"]["cpu_baseline"] = config5_cpu_baseline()
            log(f"config5 cpu: {extras['config5_engine']['cpu_baseline']}")

    cpu = None if args.no_cpu else cpu_baseline(head[0])
    if cpu:
        log(f"cpu baseline: {cpu}")
        threads = min(os.cpu_count() or 1, 16)  # the box's share of host cores
        extras["cpu_baseline_all_threads"] = cpu_baseline(head[0], seconds=5.0, nthreads=threads)
        extras["host_memory"] = host_bandwidth(threads)
        log(f"cpu baseline mt: {extras['cpu_baseline_all_threads']} host {extras['host_memory']}")

    achieved = res["stage1_gbps"] * 1e9
    line = {
        "metric": METRIC,
        "value": round(res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "config2: mixed Sarathi step, 48 decode + 4 prefill-chunk sequences, "
                        "512-token budget, SmolLM2-360M attention (H15/Hkv5/D64), bs16, "
                        "F32 KV, random scatter over a 64k-block pool",
            "query_rows": int(np.mean([b.total_q for b in head])),
            "sequences": int(np.mean([b.num_seqs for b in head])),
            "rotation": "8 batches",
            "partition": "per batch from its host-side lengths (kanso_ragged_partition_size), "
                         "as the engine passes it from its plan",
            "work_list": ("rows from the work list built on the host from the same plan "
                          "(kanso_ragged_build_work, uploaded once per batch outside the timed "
                          "region as the engine uploads it with each step's plan)") if WORK else None,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved / 1e9, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK, 4),
            "traffic": profiled_traffic(),
            "traffic_source": "profiles/attention_config2_hbm_traffic.md (all kernels of one call)",
            "kernel": "attn_main (persistent ragged paged attention: MFMA prefill-chunk "
                      "workgroups + split-K decode waves)",
            "algorithmic_bytes_per_launch": res["algorithmic_bytes"],
            "avg_launch_ms": round(res["stage1_ms"], 5),
        },
        "hbm_frac_whole_call": round(res["call_gbps"] * 1e9 / HBM_PEAK, 4),
        "reduce_ms": round(res["reduce_ms"], 5),
        "cpu_baseline": cpu,
    }
    line.update(extras)
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
