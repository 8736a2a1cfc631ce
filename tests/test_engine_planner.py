"""The C++ scheduler of libkanso_hip.so (model-less mode, no GPU) against the
Python restatement in oracle/engine_ref.py: every step's outputs and flattened
batch must be identical. Also the reference's own scheduler tests
(tests/test_chunked_prefill.rs) restated."""
import numpy as np
import pytest

import engine_ref as R
from kanso_infer_amd.engine import Engine, dry_token

VOCAB = 50


def pair(max_running, total_blocks, block_size, budget, vocab=VOCAB):
    cpp = Engine(None, max_running, total_blocks, block_size, budget, dry_vocab=vocab)
    ref = R.Engine(R.dry_forward(vocab), max_running, total_blocks, block_size, budget)
    return cpp, ref


def assert_same_step(cpp, ref, tag=""):
    a = cpp.step()
    b = ref.step()
    assert [(o.request_id, o.token_id, o.is_finished) for o in a] == b, tag
    lp = cpp.last_plan()
    rp = ref.last_plan
    if rp is None:
        assert lp["tokens"].size == 0, tag
        return a
    assert lp["tokens"].tolist() == rp.tokens, tag
    assert lp["positions"].tolist() == rp.positions, tag
    assert lp["slot_mapping"].tolist() == rp.slot_mapping, tag
    assert lp["context_lens"].tolist() == rp.context_lens, tag
    assert lp["query_lens"].tolist() == rp.query_lens, tag
    assert lp["table_lens"].tolist() == [len(t) for t in rp.block_tables], tag
    assert lp["tables"].tolist() == [b for t in rp.block_tables for b in t], tag
    assert lp["sample_rows"].tolist() == rp.sample_rows, tag
    return a


def test_dry_token_matches():
    for rid, pos, v in [(1, 0, 50), (7, 1234, 49152), (123456, 99, 7)]:
        assert dry_token(rid, pos, v) == R.dry_token(rid, pos, v)


def test_chunked_prefill_budget_enforcement():
    # tests/test_chunked_prefill.rs:5-51: budget 4, block 4 -> chunks 4 / 4 / 2
    cpp, ref = pair(2, 30, 4, 4)
    for e in (cpp, ref):
        e.add_request(list(range(10)), 2)
    for n_out, fin in [(0, None), (0, None), (1, False), (1, True)]:
        out = assert_same_step(cpp, ref)
        assert len(out) == n_out
        if n_out:
            assert out[0].is_finished == fin
    assert not cpp.has_unfinished_requests()


def test_co_scheduling_decode_never_stalls():
    # tests/test_chunked_prefill.rs:53-99
    cpp, ref = pair(2, 30, 4, 5)
    for e in (cpp, ref):
        e.add_request([1, 2], 4)
    assert len(assert_same_step(cpp, ref)) == 1
    for e in (cpp, ref):
        e.add_request([10, 11, 12, 13, 14, 15, 16, 17], 2)
    out = assert_same_step(cpp, ref)
    assert [o.request_id for o in out] == [1]
    out = assert_same_step(cpp, ref)
    assert sorted(o.request_id for o in out) == [1, 2]


def test_prefix_cache_reused_before_first_chunk():
    # tests/test_chunked_prefill.rs:101-133
    cpp, ref = pair(2, 30, 4, 16)
    prefix = [1, 2, 3, 4, 5, 6, 7, 8]
    for e in (cpp, ref):
        e.add_request(prefix, 1)
    while cpp.has_unfinished_requests():
        assert_same_step(cpp, ref)
    for e in (cpp, ref):
        e.add_request(prefix + [9, 10], 1)
    out = assert_same_step(cpp, ref)
    assert [o.request_id for o in out] == [2]
    plan = cpp.last_plan()
    assert plan["query_lens"].tolist() == [2]  # only tokens 9, 10 were prefilled
    assert cpp.stats()["prefix_hits"] == 1


def test_long_prompt_chunking_keeps_decode_every_step():
    # tests/test_chunked_prefill.rs:135-200 (the step structure; timing is not a CPU property)
    cpp, ref = pair(4, 600, 16, 256)
    for e in (cpp, ref):
        e.add_request([1, 2, 3, 4], 30)
    assert_same_step(cpp, ref)
    assert_same_step(cpp, ref)
    for e in (cpp, ref):
        e.add_request([i % 45 for i in range(2048)], 2)
    last = 2
    emitted_huge = 0
    step = 2
    while cpp.has_unfinished_requests() and step < 50:
        out = assert_same_step(cpp, ref)
        step += 1
        if any(o.request_id == 1 for o in out):
            assert step - last == 1
            last = step
        emitted_huge += any(o.request_id == 2 for o in out)
    assert emitted_huge >= 1


def random_workload(rng, n, max_prompt, max_gen, arrivals, shared):
    reqs = []
    for i in range(n):
        plen = int(rng.integers(1, max_prompt + 1))
        if shared:
            prompt = [(i % 3 * 10 + p) % 30 for p in range(plen)]  # bench.rs:470-474 pattern
        else:
            prompt = rng.integers(0, VOCAB, plen).tolist()
        reqs.append((prompt, int(rng.integers(1, max_gen + 1)), int(rng.integers(0, arrivals + 1))))
    return reqs


@pytest.mark.parametrize("seed", range(20))
def test_random_workloads_match(seed):
    rng = np.random.default_rng(seed)
    if seed >= 12:
        # oversubscribed pool: recompute preemption on almost every step
        _run_pair(seed, rng, total_blocks=int(rng.integers(14, 24)), block_size=4,
                  budget=int(rng.choice([8, 64])), max_running=8,
                  reqs=random_workload(rng, 10, 12, 24, 4, shared=bool(seed % 2)))
        return
    # small pools force recompute preemption; shared prompts exercise the prefix cache
    total_blocks = int(rng.choice([20, 24, 64, 400]))
    block_size = int(rng.choice([4, 16]))
    budget = int(rng.choice([8, 32, 512]))
    max_running = int(rng.choice([2, 4, 64]))
    # every request must fit the pool alone, or the reference itself never finishes it
    max_prompt = max(4, min(int(rng.choice([20, 90])), total_blocks * block_size // 2 - 24 - block_size))
    reqs = random_workload(rng, int(rng.integers(4, 24)), max_prompt, 24, 10,
                           shared=bool(seed % 2))
    _run_pair(seed, rng, total_blocks, block_size, budget, max_running, reqs)


def _run_pair(seed, rng, total_blocks, block_size, budget, max_running, reqs):
    cpp, ref = pair(max_running, total_blocks, block_size, budget)
    order = sorted(range(len(reqs)), key=lambda i: reqs[i][2])
    nxt = step = 0
    while step < 3000:
        while nxt < len(order) and reqs[order[nxt]][2] <= step:
            p, g, _ = reqs[order[nxt]]
            stops = [p[0]] if (order[nxt] % 5 == 4) else []
            assert cpp.add_request(p, g, stops) == ref.add_request(p, g, stops)
            nxt += 1
        if nxt >= len(order) and not cpp.has_unfinished_requests():
            break
        assert_same_step(cpp, ref, tag=f"seed {seed} step {step}")
        st = cpp.stats()
        assert st["waiting"] == ref.waiting_count()
        assert st["running"] == ref.running_count()
        assert st["free_blocks"] == ref.block_pool.free_blocks_count()
        step += 1
    assert not ref.has_unfinished_requests()
    assert cpp.stats()["prefix_hits"] == ref.prefix_cache_hits
    return ref


def test_cancel_and_drain():
    cpp, ref = pair(4, 64, 4, 16)
    ids = [cpp.add_request([1, 2, 3, 4, 5], 10) for _ in range(3)]
    for _ in range(3):
        ref.add_request([1, 2, 3, 4, 5], 10)
    assert_same_step(cpp, ref)
    free_before = cpp.free_blocks_count()
    assert cpp.cancel_request(ids[1]) and ref.cancel_request(ids[1])
    assert cpp.free_blocks_count() == ref.block_pool.free_blocks_count() > free_before
    assert not cpp.cancel_request(999)
    while cpp.has_unfinished_requests():
        assert_same_step(cpp, ref)
    assert cpp.drain_finished() == ref.drain_finished() == 2


def test_continuous_batching_staggered_arrival():
    """tests/test_continuous_batching.rs:1-40: max_running 2, 20 blocks of 4, no
    budget (Engine::new, src/engine.rs:36-43). A request arriving mid-generation is
    admitted beside the running one, and every block returns to the pool."""
    cpp, ref = pair(2, 20, 4, (1 << 31) - 1)
    id1 = cpp.add_request([1, 2], 3)
    ref.add_request([1, 2], 3)
    assert cpp.stats()["waiting"] == 1 and cpp.stats()["running"] == 0
    out1 = assert_same_step(cpp, ref)
    assert len(out1) == 1 and out1[0].request_id == id1
    assert cpp.stats()["running"] == 1
    cpp.add_request([3, 4], 2)
    ref.add_request([3, 4], 2)
    assert cpp.stats()["waiting"] == 1
    out2 = assert_same_step(cpp, ref)
    assert len(out2) == 2 and cpp.stats()["running"] == 2
    steps = 0
    while cpp.has_unfinished_requests() and steps < 10:
        assert_same_step(cpp, ref)
        steps += 1
    assert not cpp.has_unfinished_requests()
    st = cpp.stats()
    assert st["running"] == 0 and st["waiting"] == 0
    assert cpp.free_blocks_count() == 20 == ref.block_pool.free_blocks_count()


def test_empty_prompt_rejected():
    """An empty prompt is refused at admission (the reference's server refuses it,
    src/server/routes.rs:109): the engine stays usable for the other requests."""
    from kanso_infer_amd import EngineError
    cpp, ref = pair(4, 16, 4, 8)
    with pytest.raises(EngineError, match="empty prompt"):
        cpp.add_request([], 4)
    cpp.add_request([1, 2, 3], 3)
    ref.add_request([1, 2, 3], 3)
    while cpp.has_unfinished_requests():
        assert_same_step(cpp, ref, "after a refused request")
