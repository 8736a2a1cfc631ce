"""Seeded synthetic inputs for the benchmark configurations of this path.

Each generator returns plain numpy arrays (host) describing one attention call:
query rows, per-sequence query lengths / context lengths, and block tables over a
paged pool. Pools themselves are filled by the caller (on the device for the
benchmark, on the host for small parity cases), so a multi-GB pool never has to
exist in host memory.

Seeds are 0x5EED0057 + config index (the reference's MOCK_SEED, src/model.rs:201,
reused as a base so every run of a config sees the same inputs).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

MOCK_SEED = 0x5EED0057

SMOLLM2 = dict(num_heads=15, num_kv_heads=5, head_dim=64)   # src/config.rs:71-90
GRANITE = dict(num_heads=16, num_kv_heads=4, head_dim=64)   # src/config.rs:92-111
BLOCK_SIZE = 16


@dataclass
class AttnBatch:
    """One ragged attention call in plan order (decodes first, then prefill chunks)."""
    q_lens: np.ndarray            # [S] query rows per sequence
    context_lens: np.ndarray      # [S] keys each sequence attends (start + q_len)
    block_tables: np.ndarray      # [S, max_blocks] u32, padded by repeating the last needed block
    num_blocks: int               # physical blocks in the pool
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int = BLOCK_SIZE
    scale: float = 0.125
    label: str = ""
    extra: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return int(self.q_lens.size)

    @property
    def total_q(self) -> int:
        return int(self.q_lens.sum())

    @property
    def cu_seqlens(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)

    @property
    def max_blocks(self) -> int:
        return int(self.block_tables.shape[1])

    def kv_bytes_per_token_head(self, kv_dtype: int) -> float:
        """Bytes of K plus V per (token, KV head) for a pool kind."""
        d = self.head_dim
        if kv_dtype == 0:
            return 2 * d * 4
        if kv_dtype in (1, 3):  # INT8, FP8: one f32 scale per row
            return 2 * (d + 4)
        return 2 * (d + 2 * d // 32)

    def algorithmic_bytes(self, kv_dtype: int = 0) -> int:
        """K/V once per sequence + block-table entries + Q + O + cu_seqlens + context_lens."""
        ctx = self.context_lens.astype(np.int64)
        kv = int((ctx * self.num_kv_heads).sum() * self.kv_bytes_per_token_head(kv_dtype))
        tables = int(((ctx + self.block_size - 1) // self.block_size).sum() * 4)
        qo = 2 * self.total_q * self.num_heads * self.head_dim * 4
        return kv + tables + qo + (self.num_seqs + 1) * 4 + self.num_seqs * 4


def _scatter_tables(rng, context_lens, block_size, num_blocks):
    """Distinct random physical blocks per sequence (a random scatter over the pool),
    padded with the sequence's last needed block (src/model.rs:102-104)."""
    need = np.maximum((context_lens + block_size - 1) // block_size, 1)
    total = int(need.sum())
    if total > num_blocks:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {total}")
    ids = rng.choice(num_blocks, size=total, replace=False).astype(np.uint32)
    mb = int(need.max())
    tables = np.zeros((len(context_lens), mb), dtype=np.uint32)
    off = 0
    for s, n in enumerate(need):
        row = ids[off:off + n]
        off += n
        tables[s, :n] = row
        tables[s, n:] = row[-1]
    return tables


def config1_decode(seed_offset: int = 0, num_seqs: int = 8) -> AttnBatch:
    """Config 1: decode-only, SmolLM2 attention shape, S=8, ctx ~ U{64..1024}, tables a
    random permutation of free block ids (the pool holds exactly the needed blocks)."""
    rng = np.random.default_rng(MOCK_SEED + 1 + seed_offset)
    ctx = rng.integers(64, 1024, size=num_seqs, endpoint=True).astype(np.int64)
    need = (ctx + BLOCK_SIZE - 1) // BLOCK_SIZE
    num_blocks = int(need.sum())
    tables = _scatter_tables(rng, ctx, BLOCK_SIZE, num_blocks)
    return AttnBatch(np.ones(num_seqs, np.int64), ctx, tables, num_blocks, label="config1",
                     **SMOLLM2)


def config2_mixed(num_decodes: int = 48, num_chunks: int = 4, budget: int = 512,
                  num_blocks: int = 65536, seed_offset: int = 0,
                  decode_ctx=(128, 4096), chunk_len=(32, 256), chunk_prior=(0, 2048)) -> AttnBatch:
    """Config 2: a Sarathi step under a token budget. Decodes (ctx ~ U{128..4096}) are
    planned first and cost one token each; then prefill chunks (q_len ~ U{32..256},
    prior context ~ U{0..2048}) take min(q_len, remaining budget) in order
    (src/engine.rs:228-266, 321-362). Tables are a random scatter over the pool."""
    rng = np.random.default_rng(MOCK_SEED + 2 + seed_offset)
    dctx = rng.integers(decode_ctx[0], decode_ctx[1], size=num_decodes, endpoint=True)
    clen = rng.integers(chunk_len[0], chunk_len[1], size=num_chunks, endpoint=True)
    cprior = rng.integers(chunk_prior[0], chunk_prior[1], size=num_chunks, endpoint=True)
    remaining = budget - num_decodes
    q_lens, ctx = [1] * num_decodes, list(dctx)
    for n, prior in zip(clen, cprior):
        take = int(min(n, remaining))
        if take == 0:
            continue
        remaining -= take
        q_lens.append(take)
        ctx.append(int(prior) + take)
    q_lens = np.asarray(q_lens, np.int64)
    ctx = np.asarray(ctx, np.int64)
    tables = _scatter_tables(rng, ctx, BLOCK_SIZE, num_blocks)
    return AttnBatch(q_lens, ctx, tables, num_blocks,
                     label=f"config2 {num_decodes} decodes + {int((q_lens > 1).sum())} chunks",
                     **SMOLLM2)


def config3_quant_decode(num_seqs: int = 32, num_blocks: int | None = None,
                         seed_offset: int = 0) -> AttnBatch:
    """Config 3: Granite-dense attention shape, 32 decode queries with context
    log-uniform in [256, 8192]."""
    rng = np.random.default_rng(MOCK_SEED + 3 + seed_offset)
    ctx = np.exp(rng.uniform(np.log(256), np.log(8192), size=num_seqs)).astype(np.int64)
    need = (ctx + BLOCK_SIZE - 1) // BLOCK_SIZE
    nb = int(need.sum()) if num_blocks is None else num_blocks
    tables = _scatter_tables(rng, ctx, BLOCK_SIZE, nb)
    return AttnBatch(np.ones(num_seqs, np.int64), ctx, tables, nb, label="config3", **GRANITE)


def small_mixed(seed: int, num_decodes: int = 5, num_chunks: int = 2, num_heads: int = 15,
                num_kv_heads: int = 5, head_dim: int = 64, block_size: int = 16,
                max_ctx: int = 600, chunk_max: int = 40) -> AttnBatch:
    """A small ragged batch for parity tests that the oracle finishes in well under a second."""
    rng = np.random.default_rng(MOCK_SEED + 100 + seed)
    q_lens = [1] * num_decodes + list(rng.integers(2, chunk_max, size=num_chunks, endpoint=True))
    prior = list(rng.integers(1, max_ctx, size=num_decodes, endpoint=True)) + list(
        rng.integers(0, max_ctx, size=num_chunks, endpoint=True))
    q_lens = np.asarray(q_lens, np.int64)
    ctx = np.asarray([p if q == 1 else p + q for p, q in zip(prior, q_lens)], np.int64)
    need = (ctx + block_size - 1) // block_size
    nb = int(need.sum()) + 7
    tables = _scatter_tables(rng, ctx, block_size, nb)
    return AttnBatch(q_lens, ctx, tables, nb, num_heads=num_heads, num_kv_heads=num_kv_heads,
                     head_dim=head_dim, block_size=block_size,
                     scale=1.0 / float(np.sqrt(head_dim)), label=f"small_mixed[{seed}]")


# Config 5: the engine run's request trace and its model / pool settings
# (create_engine_for_model_profile, src/bench.rs:598-614).
CONFIG5_SEED = 0x5EED0005
CONFIG5_WEIGHT_SEED = 0x5EED0057
CONFIG5_STD = 0.02
CONFIG5_BUDGET = 512
CONFIG5_MAX_RUNNING = 64


def config5_workload(seed: int = CONFIG5_SEED, num_requests: int = 64, rate: float = 40.0,
                     step_secs: float = 0.005) -> list:
    """Config 5 requests: prompt lengths log-uniform [16, 2048], generation lengths
    uniform [32, 512], Poisson arrivals at `rate` requests/s mapped to steps of
    `step_secs` (the reference's sweep constants, src/bench/traffic.rs:5-9, 153-160),
    synthetic prompts (req*10 + p) % 30 (src/bench.rs:470-474). numpy PCG64 seeded."""
    from .engine import generate_poisson_schedule, schedule_to_trace
    rng = np.random.default_rng(seed)
    plen = np.rint(np.exp(rng.uniform(np.log(16), np.log(2048), num_requests))).astype(int)
    glen = rng.integers(32, 513, num_requests)
    sched = generate_poisson_schedule(num_requests, rate, seed + 1)
    return schedule_to_trace(sched, plen, glen, step_secs)


def config5_total_blocks(requests: list, block_size: int = BLOCK_SIZE) -> int:
    """Pool size of the config-5 engine: one sequence's worst case plus a block, per
    request (src/bench.rs:598-614), at least 128."""
    max_tokens = max(r.prompt_len + r.gen_len for r in requests)
    blocks_per_seq = -(-max_tokens // block_size) + 1
    return max(blocks_per_seq * len(requests), 128)
