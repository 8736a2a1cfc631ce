"""CPU model of the parity tests: random-init Q8_0 weights (numpy, seeded), per-layer
F32 KV pools, and the batched forward of oracle_forward_batch behind the
engine_ref.Engine forward interface.

TEST INFRASTRUCTURE ONLY (the checker of the GPU decoder and engine)."""
from __future__ import annotations

import numpy as np

import oracle


def random_weights(cfg: dict, seed: int, std: float = 0.02) -> dict:
    """Every matrix N(0, std^2) quantized by the Q8_0 rule (src/quant/q8_0.rs:13-32);
    norms = 1 plus a small seeded perturbation so the norm weights are exercised."""
    rng = np.random.default_rng(seed)
    h, D, I, V = cfg["hidden"], cfg["head_dim"], cfg["intermediate"], cfg["vocab"]
    H, KV = cfg["num_heads"], cfg["num_kv_heads"]

    def mat(rows, cols):
        return oracle.quantize_row_q8_0((rng.standard_normal((rows, cols)) * std).astype(np.float32))

    def norm():
        return (1.0 + 0.05 * rng.standard_normal(h)).astype(np.float32)

    w = {"embed": mat(V, h), "final_norm": norm(), "layers": []}
    if not cfg.get("tied", True):
        w["lm_head"] = mat(V, h)
    for _ in range(cfg["num_layers"]):
        w["layers"].append({
            "attn_norm": norm(), "ffn_norm": norm(),
            "wq": mat(H * D, h), "wk": mat(KV * D, h), "wv": mat(KV * D, h), "wo": mat(h, H * D),
            "w_gate": mat(I, h), "w_up": mat(I, h), "w_down": mat(h, I)})
    return w


def device_init_weights(cfg: dict, seed: int, std: float = 0.02) -> dict:
    """The weights kanso_model_init_random draws on the device, restated on the host
    (bit for bit): matrix j (1 = embedding, 2 = untied lm_head, then per layer Q, K,
    V, O, gate, up, down) uses stream seed seed * 0x100000001b3 + j *
    0x9e3779b97f4a7c15 mod 2^64; norms are 1."""
    h, D, I, V = cfg["hidden"], cfg["head_dim"], cfg["intermediate"], cfg["vocab"]
    H, KV = cfg["num_heads"], cfg["num_kv_heads"]
    M = 2**64 - 1
    j = 0

    def mat(rows, cols):
        nonlocal j
        j += 1
        return oracle.init_random_q8_0((seed * 0x100000001b3 + j * 0x9e3779b97f4a7c15) & M,
                                       rows, cols, std)

    ones = np.ones(h, np.float32)
    w = {"embed": mat(V, h), "final_norm": ones, "layers": []}
    if not cfg.get("tied", True):
        w["lm_head"] = mat(V, h)
    for _ in range(cfg["num_layers"]):
        L = {"attn_norm": ones, "ffn_norm": ones}
        for name, rows, cols in (("wq", H * D, h), ("wk", KV * D, h), ("wv", KV * D, h),
                                 ("wo", h, H * D), ("w_gate", I, h), ("w_up", I, h),
                                 ("w_down", h, I)):
            L[name] = mat(rows, cols)
        w["layers"].append(L)
    return w


class OracleModel:
    """kv_dtype: the pool kind (oracle.KV_*): F32, or a 1-byte pool whose rows are
    quantized by oracle_kv_append (Engine::new_with_budget_and_kv, src/engine.rs:62-100)."""

    def __init__(self, cfg: dict, weights: dict, num_blocks: int, block_size: int, nthreads=8,
                 kv_dtype: int = oracle.KV_F32):
        self.cfg, self.weights = dict(cfg, kv_dtype=kv_dtype), weights
        self.kv_dtype = kv_dtype
        self.num_blocks, self.block_size = num_blocks, block_size
        pools = [oracle.kv_pool_arrays(kv_dtype, num_blocks, block_size, cfg["num_kv_heads"],
                                       cfg["head_dim"]) for _ in range(cfg["num_layers"])]
        self.k = [p[0] for p in pools]
        self.v = [p[1] for p in pools]
        self.ks = [p[2] for p in pools]
        self.vs = [p[3] for p in pools]
        self.nthreads = nthreads
        self.last_logits = None

    def reset_block(self, block: int) -> None:
        """allocate_zeroed's erase (src/kv_cache/mod.rs:25-35) across every layer."""
        rows = self.block_size * self.cfg["num_kv_heads"]
        w = rows * self.cfg["head_dim"]
        for a in self.k + self.v:
            a[block * w:(block + 1) * w] = 0
        if self.kv_dtype != oracle.KV_F32:
            # scales of an empty row: 1.0 (INT8 / FP8, quantized_storage.rs:35-40), 0 (Q8_0)
            per = rows if self.kv_dtype in (oracle.KV_INT8, oracle.KV_FP8) else w // 32
            empty = 1.0 if self.kv_dtype in (oracle.KV_INT8, oracle.KV_FP8) else 0
            for a in self.ks + self.vs:
                a[block * per:(block + 1) * per] = empty

    def logits(self, plan, all_rows: bool = False) -> np.ndarray:
        """[S, vocab] of each sequence's last row, or with all_rows [T, vocab] of every
        new token (forward_batch_all_rows, src/model.rs:1382-1410)."""
        bs = self.block_size
        ctx = np.asarray(plan.context_lens, np.int64)
        max_blocks = int(max(1, ((ctx + bs - 1) // bs).max()))
        tables = np.zeros((len(ctx), max_blocks), np.uint32)
        for s, t in enumerate(plan.block_tables):  # PaddedDecodeTables (model.rs:84-105)
            need = max(1, -(-int(ctx[s]) // bs))
            for b in range(max_blocks):
                tables[s, b] = t[min(b, need - 1)]
        cu = np.concatenate([[0], np.cumsum(plan.query_lens)]).astype(np.int32)
        return oracle.forward_batch(self.cfg, self.weights, self.k, self.v, self.num_blocks, bs,
                                    plan.tokens, plan.positions, plan.slot_mapping, tables,
                                    max_blocks, cu, ctx, nthreads=self.nthreads, all_rows=all_rows,
                                    k_scales=self.ks, v_scales=self.vs)

    def forward(self, plan) -> list:
        """engine_ref forward: greedy_token (src/sampler.rs:7-17) of each sequence."""
        lg = self.logits(plan)
        self.last_logits = lg
        return [oracle.greedy(row) for row in lg]
