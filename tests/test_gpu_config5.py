"""Config 5 end to end against the oracle: the GPU engine's greedy token stream over
the full trace (kanso_infer_amd.workloads.config5_workload), on the weights
kanso_model_init_random draws, must equal the oracle engine's stream committed by
tests/golden/make_config5_checksum.py (FNV-1a checksum and every token,
src/bench.rs:497-519)."""
import json
from pathlib import Path

import numpy as np
import pytest

from kanso_infer_amd import workloads
from kanso_infer_amd.engine import Engine, Model, ModelConfig, fnv1a_64, run_benchmark_workload

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def run_config5(ctx, layers: int, requests: int):
    cfg = ModelConfig.smollm2_360m(max_position=4096, num_hidden_layers=layers)
    model = Model(ctx, cfg)
    model.init_random(seed=workloads.CONFIG5_WEIGHT_SEED, std=workloads.CONFIG5_STD)
    reqs = workloads.config5_workload(num_requests=requests)
    total = workloads.config5_total_blocks(reqs)
    model.alloc_kv(total, workloads.BLOCK_SIZE, workloads.CONFIG5_BUDGET, workloads.CONFIG5_MAX_RUNNING + 1)
    eng = Engine(model, workloads.CONFIG5_MAX_RUNNING, total, workloads.BLOCK_SIZE, workloads.CONFIG5_BUDGET)
    rep = run_benchmark_workload(eng, reqs)
    eng.close()
    model.close()
    return rep


def check(rep, name):
    if not (GOLDEN / f"{name}.json").exists():
        pytest.skip(f"{name}.json not generated (tests/golden/make_config5_checksum.py)")
    info = json.loads((GOLDEN / f"{name}.json").read_text())
    want = np.load(GOLDEN / f"{name.replace('config5_oracle', 'config5_oracle_tokens')}.npy")
    got = np.asarray(rep["generated"], np.uint32)
    if not np.array_equal(got, want):
        n = min(got.size, want.size)
        first = int(np.argmax(got[:n] != want[:n])) if (got[:n] != want[:n]).any() else n
        pytest.fail(f"token streams differ at token {first} of {want.size} (gpu {got.size} tokens)")
    assert f"{fnv1a_64(got):016x}" == info["checksum"]
    assert rep["steps"] == info["steps"]


def test_config5_two_layers(ctx):
    """2 of the 32 layers, the first 4 requests of the trace."""
    check(run_config5(ctx, 2, 4), "config5_oracle_2l_4r")


def test_config5_full(ctx):
    """The headline workload itself: 32 layers, 64 Poisson requests, budget 512."""
    check(run_config5(ctx, 32, 64), "config5_oracle")
