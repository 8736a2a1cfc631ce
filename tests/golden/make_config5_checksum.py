"""Writes the oracle's greedy token stream of the full config-5 run
(tests/golden/config5_oracle.json + config5_oracle_tokens.npy).

TEST INFRASTRUCTURE: the checker of the GPU engine's config-5 checksum. The oracle
engine (oracle/engine_ref.py, the restated Engine::step) drives the oracle forward
(oracle/kanso_oracle_model.cpp) over the weights kanso_model_init_random draws on the
device, restated bit for bit on the host (oracle/model_ref.device_init_weights):
SmolLM2-360M shape, 32 layers, F32 KV pool of config5_total_blocks blocks of 16,
the 64-request trace of kanso_infer_amd.workloads.config5_workload, budget 512,
max_running 64, greedy. The same trace and settings as bench.py's config-5 run.

    python tests/golden/make_config5_checksum.py [--threads 8] [--layers 32]

Takes about an hour on 8 host cores. --layers / --requests make smaller runs for
a quick look (their output goes to a different file name).
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

import engine_ref  # noqa: E402
import oracle  # noqa: E402
from kanso_infer_amd import workloads  # noqa: E402
from kanso_infer_amd.engine import synthetic_prompt  # noqa: E402
from model_ref import OracleModel, device_init_weights  # noqa: E402

SMOLLM2 = dict(hidden=960, num_heads=15, num_kv_heads=5, head_dim=64, num_layers=32,
               intermediate=2560, vocab=49152)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--requests", type=int, default=64)
    args = ap.parse_args()
    cfg = dict(SMOLLM2, num_layers=args.layers)
    t0 = time.time()
    w = device_init_weights(cfg, workloads.CONFIG5_WEIGHT_SEED, workloads.CONFIG5_STD)
    reqs = workloads.config5_workload(num_requests=args.requests)
    total_blocks = workloads.config5_total_blocks(reqs)
    om = OracleModel(cfg, w, total_blocks, workloads.BLOCK_SIZE, nthreads=args.threads)
    eng = engine_ref.Engine(om.forward, workloads.CONFIG5_MAX_RUNNING, total_blocks, workloads.BLOCK_SIZE,
                            workloads.CONFIG5_BUDGET, reset_block=om.reset_block)
    print(f"weights + pool ready in {time.time() - t0:.0f} s, {total_blocks} blocks", file=sys.stderr, flush=True)
    trace = [(synthetic_prompt(i, r.prompt_len), r.gen_len, r.arrival_step) for i, r in enumerate(reqs)]
    state = dict(steps=0, t=time.time())

    def on_step(e, outs):
        state["steps"] += 1
        if state["steps"] % 25 == 0:
            print(f"step {state['steps']}: {time.time() - state['t']:.0f} s", file=sys.stderr, flush=True)

    tokens = engine_ref.run_workload(eng, trace, on_step=on_step)
    suffix = "" if (args.layers, args.requests) == (32, 64) else f"_{args.layers}l_{args.requests}r"
    out = ROOT / "tests" / "golden"
    np.save(out / f"config5_oracle_tokens{suffix}.npy", np.asarray(tokens, np.uint32))
    info = dict(checksum=f"{oracle.fnv1a_64(tokens):016x}", generated_tokens=len(tokens), steps=state["steps"],
                layers=args.layers, requests=args.requests, total_blocks=total_blocks,
                budget=workloads.CONFIG5_BUDGET, max_running=workloads.CONFIG5_MAX_RUNNING,
                weight_seed=workloads.CONFIG5_WEIGHT_SEED, std=workloads.CONFIG5_STD,
                trace_seed=workloads.CONFIG5_SEED, seconds=round(time.time() - t0, 1))
    (out / f"config5_oracle{suffix}.json").write_text(json.dumps(info, indent=1) + "\n")
    print(json.dumps(info))


if __name__ == "__main__":
    main()
