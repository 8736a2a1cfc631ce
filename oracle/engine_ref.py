"""Python restatement of kanso-infer's continuous-batching scheduler: BlockPool,
BlockTable, PrefixCache, Sequence and Engine::step (Sarathi token-budget planning,
admission with prefix-cache lookup, chunked prefill, recompute preemption, commit
and retirement).

TEST INFRASTRUCTURE ONLY: the checker the C++ engine of libkanso_hip.so is
compared against, plan by plan and token by token. The product never imports it.

Sources restated (kanso-infer tree):
  BlockPool            src/kv_cache/block_pool.rs:1-68
  BlockTable           src/kv_cache/block_table.rs:1-63
  PrefixCache          src/kv_cache/prefix_cache.rs:1-116
  allocate_zeroed      src/kv_cache/mod.rs:25-35
  Sequence             src/scheduler/sequence.rs:1-74
  Engine::step         src/engine.rs:213-505
  ensure_blocks / preempt_lowest_priority_after / preempt
                       src/engine.rs:533-601
  cancel_request / drain_finished   src/engine.rs:511-531
  fnv1a_64             src/bench.rs:20-29
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

WAITING, RUNNING, PREEMPTED, FINISHED = 0, 1, 2, 3


class BlockPool:
    """src/kv_cache/block_pool.rs: LIFO free list starting (0..n).rev(), ref counts."""

    def __init__(self, total_blocks: int):
        self.free_blocks = list(range(total_blocks - 1, -1, -1))
        self.ref_counts = [0] * total_blocks
        self.total_blocks = total_blocks

    def free_blocks_count(self) -> int:
        return len(self.free_blocks)

    def allocate(self):
        if not self.free_blocks:
            return None
        b = self.free_blocks.pop()
        self.ref_counts[b] = 1
        return b

    def claim_block(self, block: int) -> bool:
        if block < self.total_blocks:
            if self.ref_counts[block] > 0:
                self.ref_counts[block] += 1
                return True
            if block in self.free_blocks:
                self.free_blocks.remove(block)
                self.ref_counts[block] = 1
                return True
        return False

    def free(self, block: int) -> None:
        if block < self.total_blocks and self.ref_counts[block] > 0:
            self.ref_counts[block] -= 1
            if self.ref_counts[block] == 0:
                self.free_blocks.append(block)


@dataclass
class BlockTable:
    """src/kv_cache/block_table.rs."""
    blocks: list = field(default_factory=list)
    num_tokens: int = 0


class PrefixCache:
    """src/kv_cache/prefix_cache.rs: block-aligned token prefixes -> physical blocks,
    a reverse index for invalidation and LRU eviction past max_entries."""

    def __init__(self, block_size: int, max_entries: int = 64):
        self.block_size = block_size
        self.max_entries = max(max_entries, 1)
        self.cached = {}
        self.block_to_keys = {}
        self.last_used = {}
        self.tick = 0

    def insert_prefix(self, tokens, blocks) -> None:
        n = len(tokens) // self.block_size
        for b in range(1, n + 1):
            key = tuple(tokens[:b * self.block_size])
            bp = list(blocks[:b])
            self.tick += 1
            old = self.cached.get(key)
            self.cached[key] = bp
            if old is not None:
                for blk in old:
                    if blk not in bp:
                        self._detach(key, blk)
            for blk in bp:
                keys = self.block_to_keys.setdefault(blk, [])
                if key not in keys:
                    keys.append(key)
            self.last_used[key] = self.tick
        while len(self.cached) > self.max_entries:
            if not self.last_used:
                break
            oldest = min(self.last_used.items(), key=lambda kv: kv[1])[0]
            self._remove_entry(oldest)

    def invalidate_block(self, block: int) -> int:
        keys = self.block_to_keys.pop(block, [])
        for key in keys:
            self._remove_entry(key)
        return len(keys)

    def find_longest_prefix(self, tokens):
        n = len(tokens) // self.block_size
        for b in range(n, 0, -1):
            key = tuple(tokens[:b * self.block_size])
            if key in self.cached:
                self.tick += 1
                self.last_used[key] = self.tick
                return b * self.block_size, list(self.cached[key])
        return 0, []

    def _remove_entry(self, key) -> None:
        blocks = self.cached.pop(key, None)
        if blocks is not None:
            for blk in blocks:
                self._detach(key, blk)
        self.last_used.pop(key, None)

    def _detach(self, key, block) -> None:
        keys = self.block_to_keys.get(block)
        if keys is not None:
            if key in keys:
                keys[:] = [k for k in keys if k != key]
            if not keys:
                del self.block_to_keys[block]


@dataclass
class Sequence:
    """src/scheduler/sequence.rs."""
    id: int
    prompt_tokens: list
    max_tokens: int
    generated_tokens: list = field(default_factory=list)
    block_table: BlockTable = field(default_factory=BlockTable)
    status: int = WAITING
    prefilled_tokens: int = 0
    stop_token_ids: list = field(default_factory=list)

    def is_finished(self) -> bool:
        return self.status == FINISHED

    def is_done_after(self, token: int) -> bool:
        return len(self.generated_tokens) >= self.max_tokens or token in self.stop_token_ids


@dataclass
class StepPlan:
    """The flattened batch of one step, as Engine::step hands it to forward_batch."""
    tokens: list
    positions: list
    slot_mapping: list
    block_tables: list
    context_lens: list
    query_lens: list
    sample_rows: list
    request_ids: list


# forward(plan) -> next token per planned sequence (len == len(plan.query_lens))
Forward = Callable[[StepPlan], list]


class Engine:
    def __init__(self, forward: Forward, max_running: int, total_blocks: int, block_size: int,
                 token_budget: int, reset_block: Callable[[int], None] | None = None):
        self.forward = forward
        self.reset_block = reset_block or (lambda b: None)
        self.block_pool = BlockPool(total_blocks)
        self.prefix_cache = PrefixCache(block_size)
        self.sequences: list[Sequence] = []
        self.max_running = max_running
        self.block_size = block_size
        self.token_budget = token_budget
        self.current_step = 0
        self.next_request_id = 1
        self.prefix_matched_tokens = 0
        self.total_prompt_tokens_admitted = 0
        self.prefix_cache_hits = 0
        self.prefix_cache_lookups = 0
        self.last_plan: StepPlan | None = None

    def add_request(self, prompt, max_tokens, stop_token_ids=()) -> int:
        rid = self.next_request_id
        self.next_request_id += 1
        self.sequences.append(Sequence(rid, list(prompt), max_tokens,
                                       stop_token_ids=list(stop_token_ids)))
        return rid

    def waiting_count(self) -> int:
        return sum(s.status == WAITING for s in self.sequences)

    def running_count(self) -> int:
        return sum(s.status == RUNNING for s in self.sequences)

    def has_unfinished_requests(self) -> bool:
        return any(not s.is_finished() for s in self.sequences)

    def drain_finished(self) -> int:
        before = len(self.sequences)
        self.sequences = [s for s in self.sequences if not s.is_finished()]
        return before - len(self.sequences)

    def cancel_request(self, rid: int) -> bool:
        for s in self.sequences:
            if s.id == rid:
                for b in s.block_table.blocks:
                    self.block_pool.free(b)
                s.status = FINISHED
                self.drain_finished()
                return True
        return False

    # ---- block management (src/engine.rs:533-601)

    def _allocate_zeroed(self):
        b = self.block_pool.allocate()
        if b is not None:
            self.reset_block(b)
        return b

    def _decode_needs_block(self, idx) -> bool:
        t = self.sequences[idx].block_table
        return t.num_tokens + 1 > len(t.blocks) * self.block_size

    def _ensure_blocks(self, idx, want, planned) -> bool:
        while self.block_pool.free_blocks_count() < want:
            if not self._preempt_lowest_priority_after(idx, planned):
                return False
        seq = self.sequences[idx]
        for _ in range(want):
            blk = self._allocate_zeroed()
            if blk is None:
                return False
            self.prefix_cache.invalidate_block(blk)
            seq.block_table.blocks.append(blk)
        return True

    def _preempt_lowest_priority_after(self, idx, planned) -> bool:
        for j in range(len(self.sequences) - 1, idx, -1):
            s = self.sequences[j]
            if not planned[j] and s.status == RUNNING and not s.is_finished():
                self._preempt(j)
                return True
        return False

    def _preempt(self, idx) -> None:
        seq = self.sequences[idx]
        for b in seq.block_table.blocks:
            self.block_pool.free(b)
        emitted = len(seq.generated_tokens)
        seq.prompt_tokens.extend(seq.generated_tokens)
        seq.generated_tokens = []
        seq.max_tokens = max(seq.max_tokens - emitted, 0)
        seq.block_table = BlockTable()
        seq.prefilled_tokens = 0
        seq.status = WAITING

    # ---- one step (src/engine.rs:213-505)

    def step(self):
        self.current_step += 1
        outputs = []
        finished = []
        budget = self.token_budget
        planned = []  # (idx, start_pos, tokens, is_prefill)
        flags = [False] * len(self.sequences)

        # 1. decode rows first, in sequence order
        for idx, seq in enumerate(self.sequences):
            if (seq.status != RUNNING or seq.is_finished()
                    or seq.prefilled_tokens < len(seq.prompt_tokens)):
                continue
            if budget == 0:
                break
            if self._decode_needs_block(idx) and not self._ensure_blocks(idx, 1, flags):
                continue
            pos = len(seq.prompt_tokens) + len(seq.generated_tokens) - 1
            planned.append((idx, pos, [seq.generated_tokens[-1]], False))
            flags[idx] = True
            budget -= 1

        # 2. admission with prefix-cache lookup
        available = max(self.max_running - self.running_count(), 0)
        admitted = 0
        for seq in self.sequences:
            if (seq.status == WAITING and admitted < available
                    and (self.block_pool.free_blocks_count() > 0 or seq.prefilled_tokens > 0)):
                if seq.prefilled_tokens == 0 and not seq.generated_tokens:
                    self.prefix_cache_lookups += 1
                    self.total_prompt_tokens_admitted += len(seq.prompt_tokens)
                    matched, blocks = self.prefix_cache.find_longest_prefix(seq.prompt_tokens)
                    if matched > 0:
                        claimed = []
                        ok = True
                        for b in blocks:
                            if self.block_pool.claim_block(b):
                                claimed.append(b)
                            else:
                                ok = False
                                break
                        if ok:
                            seq.block_table.blocks.extend(blocks)
                            eff = matched - 1 if matched == len(seq.prompt_tokens) else matched
                            seq.block_table.num_tokens = eff
                            seq.prefilled_tokens = eff
                            self.prefix_cache_hits += 1
                            self.prefix_matched_tokens += matched
                        else:
                            for b in claimed:
                                self.block_pool.free(b)
                seq.status = RUNNING
                admitted += 1

        # 3. prefill chunks with the remaining budget
        for idx in range(len(self.sequences)):
            seq = self.sequences[idx]
            if (seq.status != RUNNING or seq.is_finished()
                    or seq.prefilled_tokens >= len(seq.prompt_tokens)):
                continue
            if budget == 0:
                continue
            needed = len(seq.prompt_tokens) - seq.prefilled_tokens
            chunk = min(needed, budget)
            if chunk == 0:
                continue
            start = seq.prefilled_tokens
            end = start + chunk
            need_blocks = -(-(end + int(end == len(seq.prompt_tokens))) // self.block_size)
            cur = len(seq.block_table.blocks)
            if need_blocks > cur and not self._ensure_blocks(idx, need_blocks - cur, flags):
                continue
            seq = self.sequences[idx]
            planned.append((idx, start, list(seq.prompt_tokens[start:end]), True))
            flags[idx] = True
            budget -= chunk

        # 4. one batched forward
        self.last_plan = None
        next_tokens = None
        if planned:
            plan = StepPlan([], [], [], [], [], [], [], [])
            for row, (idx, start, toks, is_prefill) in enumerate(planned):
                table = self.sequences[idx].block_table.blocks
                for i, tok in enumerate(toks):
                    pos = start + i
                    bi = pos // self.block_size
                    if bi >= len(table):
                        raise RuntimeError(f"Position {pos} requires block index {bi} but block "
                                           f"table only has {len(table)} blocks")
                    plan.tokens.append(tok)
                    plan.positions.append(pos)
                    plan.slot_mapping.append(table[bi] * self.block_size + pos % self.block_size)
                plan.block_tables.append(list(table))
                plan.context_lens.append(start + len(toks))
                plan.query_lens.append(len(toks))
                plan.request_ids.append(self.sequences[idx].id)
                if not is_prefill or start + len(toks) == len(self.sequences[idx].prompt_tokens):
                    plan.sample_rows.append(row)
            self.last_plan = plan
            next_tokens = self.forward(plan)

        # 5. commit in plan order
        for row, (idx, start, toks, is_prefill) in enumerate(planned):
            seq = self.sequences[idx]
            if is_prefill:
                end = start + len(toks)
                seq.prefilled_tokens = end
                seq.block_table.num_tokens = end
                if end != len(seq.prompt_tokens):
                    continue
            tok = int(next_tokens[row])
            seq.generated_tokens.append(tok)
            seq.block_table.num_tokens += 1
            done = seq.is_done_after(tok)
            if done:
                seq.status = FINISHED
                finished.append(idx)
            outputs.append((seq.id, tok, done))

        for (idx, start, toks, is_prefill) in planned:
            seq = self.sequences[idx]
            if is_prefill and seq.prefilled_tokens == len(seq.prompt_tokens):
                self.prefix_cache.insert_prefix(seq.prompt_tokens, seq.block_table.blocks)

        # 6. retirement
        for idx in finished:
            for b in self.sequences[idx].block_table.blocks:
                self.block_pool.free(b)
        return outputs


def fnv1a_64(tokens) -> int:
    h = 0xcbf29ce484222325
    for t in tokens:
        h = ((h ^ (int(t) & 0xffffffff)) * 0x100000001b3) & 0xffffffffffffffff
    return h


def dry_token(request_id: int, position: int, vocab: int) -> int:
    """Deterministic stand-in for a model's greedy token (host-only planner tests):
    the same formula the C++ engine's model-less mode uses."""
    return (request_id * 2654435761 + position * 40503 + 12345) % 4294967296 % vocab


def dry_forward(vocab: int) -> Forward:
    """The model-less engine's forward: the stand-in token of every planned row."""
    return lambda plan: [dry_token(rid, ctx, vocab)
                         for rid, ctx in zip(plan.request_ids, plan.context_lens)]


def run_workload(engine: Engine, requests, on_step=None):
    """execute_engine_run (src/bench.rs:447-537): requests arrive at their step in
    arrival order, one engine step per loop, generated tokens in emit order.
    `requests` is a list of (prompt_tokens, gen_len, arrival_step)."""
    order = sorted(range(len(requests)), key=lambda i: requests[i][2])
    nxt, step_idx, generated = 0, 0, []
    while True:
        while nxt < len(order) and requests[order[nxt]][2] <= step_idx:
            prompt, gen_len, _ = requests[order[nxt]]
            engine.add_request(prompt, gen_len)
            nxt += 1
        if nxt >= len(order) and not engine.has_unfinished_requests():
            break
        outs = engine.step()
        if on_step is not None:
            on_step(engine, outs)
        generated.extend(t for _, t, _ in outs)
        step_idx += 1
    return generated
