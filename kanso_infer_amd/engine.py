"""Host mirror of kanso-infer's engine over the C ABI: Model (the device-resident
decoder), Engine (the C++ continuous-batching scheduler) and the benchmark loop.

Mirrors, with the reference's names and meaning:
  Model / ModelConfig          src/model.rs:177-194, src/config.rs (SmolLM2-360M shape)
  Engine.new_with_budget, add_request, step, has_unfinished_requests,
  waiting_count, running_count, free_blocks_count, drain_finished,
  cancel_request, prefix_cache_hit_rate
                               src/engine.rs:35-601
  StepOutput                   src/engine.rs:11-16
  fnv1a_64                     src/bench.rs:20-29
  TraceEntry, run_benchmark_workload (execute_engine_run)
                               src/bench.rs:31-63, 447-614
  generate_poisson_schedule, schedule_to_trace
                               src/bench/traffic.rs:17-33, 84-104

Errors raise EngineError; nothing falls back to the CPU.
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from . import EngineError, Context, _check, _stream
from . import _capi
from ._capi import ModelConfigC, SeqPlanC, StepOutputC

__all__ = ["ModelConfig", "Model", "Engine", "StepOutput", "TraceEntry", "fnv1a_64",
           "run_benchmark_workload", "generate_poisson_schedule", "schedule_to_trace",
           "synthetic_prompt"]


@dataclass
class ModelConfig:
    """The decoder shape (ModelConfig, src/config.rs); head_dim is hidden / heads."""
    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    num_hidden_layers: int
    intermediate_size: int
    vocab_size: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_position: int = 8192
    tied_embeddings: bool = True
    # Granite multipliers (src/weights.rs:395-406); 0 = absent
    embedding_scale: float = 0.0
    attention_scale: float = 0.0
    residual_scale: float = 0.0
    logit_scale: float = 0.0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def smollm2_360m(cls, **overrides) -> "ModelConfig":
        """SmolLM2-360M: 32 layers, hidden 960, GQA 15:5, SwiGLU 2560, vocab 49152,
        tied embeddings."""
        base = dict(hidden_size=960, num_attention_heads=15, num_key_value_heads=5,
                    num_hidden_layers=32, intermediate_size=2560, vocab_size=49152)
        base.update(overrides)
        return cls(**base)

    def to_c(self) -> ModelConfigC:
        return ModelConfigC(self.hidden_size, self.num_attention_heads, self.num_key_value_heads,
                            self.head_dim, self.num_hidden_layers, self.intermediate_size,
                            self.vocab_size, self.rms_norm_eps, self.rope_theta,
                            self.max_position, int(self.tied_embeddings), self.embedding_scale,
                            self.attention_scale, self.residual_scale, self.logit_scale)

    def kv_cache_bytes_per_token_f32(self) -> int:
        """K and V of every layer for one token (src/config.rs kv_cache_bytes_per_token_f32)."""
        return 2 * self.num_hidden_layers * self.num_key_value_heads * self.head_dim * 4

    def weight_bytes_q8_0(self) -> int:
        """Q8_0 storage bytes of every projection plus the (tied) embedding table."""
        h, d = self.hidden_size, self.head_dim
        per_layer = ((self.num_attention_heads * d) * h + 2 * (self.num_key_value_heads * d) * h
                     + h * (self.num_attention_heads * d) + 3 * self.intermediate_size * h)
        tables = self.vocab_size * h * (1 if self.tied_embeddings else 2)
        return (per_layer * self.num_hidden_layers + tables) // 32 * 34


def quantize_q8_0_rows(ctx: Context, x: np.ndarray) -> np.ndarray:
    """f32 [rows, in] -> GGUF Q8_0 rows ([rows][in/32] x 34 B) with the device
    quantizer (kanso_quantize_q8_0, BlockQ8_0::from_f32_slice rounding)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.size == 0 or a.shape[-1] % 32:
        raise EngineError(-2, f"Q8_0 rows need a multiple of 32 columns (shape {a.shape})")
    xd = torch.from_numpy(a.ravel()).to("cuda:0")
    out = torch.empty(a.size // 32 * 34, dtype=torch.uint8, device="cuda:0")
    _check(ctx._lib.kanso_quantize_q8_0(ctx.handle, xd.data_ptr(), a.size, out.data_ptr(),
                                        _stream(None)))
    return out.cpu().numpy()


class Model:
    """The device decoder (kanso_model): packed Q8_0 projections, F32 paged KV pool."""

    def __init__(self, ctx: Context, config: ModelConfig):
        self.ctx, self.config = ctx, config
        self._lib = ctx._lib
        h = C.c_void_p()
        cfg = config.to_c()
        _check(self._lib.kanso_model_create(ctx.handle, C.byref(cfg), C.byref(h)))
        self.handle = h

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.kanso_model_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def set_weight(self, kind: int, layer: int, data: np.ndarray) -> None:
        """GGUF Q8_0 bytes of a matrix, or an f32 norm vector (host array)."""
        a = np.ascontiguousarray(data)
        _check(self._lib.kanso_model_set_weight(self.handle, kind, layer,
                                                a.ctypes.data_as(C.c_void_p), a.nbytes))

    def set_weight_q4_k(self, kind: int, layer: int, data: np.ndarray) -> None:
        """GGUF Q4_K bytes of a projection matrix, kept in that format."""
        a = np.ascontiguousarray(data)
        _check(self._lib.kanso_model_set_weight_q4_k(self.handle, kind, layer,
                                                     a.ctypes.data_as(C.c_void_p), a.nbytes))

    def load_weights(self, weights: dict) -> None:
        """weights: {"embed", "lm_head"?, "final_norm", "layers": [{"attn_norm",
        "ffn_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down", "fmt"?}]};
        a layer's optional "fmt" maps matrix names to their GGUF type (8 = Q8_0, the
        default; 12 = Q4_K)."""
        self.set_weight(_capi.KANSO_W_EMBED, 0, weights["embed"])
        if not self.config.tied_embeddings:
            self.set_weight(_capi.KANSO_W_LM_HEAD, 0, weights["lm_head"])
        self.set_weight(_capi.KANSO_W_FINAL_NORM, 0, weights["final_norm"])
        kinds = {"attn_norm": _capi.KANSO_W_ATTN_NORM, "ffn_norm": _capi.KANSO_W_FFN_NORM,
                 "wq": _capi.KANSO_W_Q, "wk": _capi.KANSO_W_K, "wv": _capi.KANSO_W_V,
                 "wo": _capi.KANSO_W_O, "w_gate": _capi.KANSO_W_GATE,
                 "w_up": _capi.KANSO_W_UP, "w_down": _capi.KANSO_W_DOWN}
        for li, layer in enumerate(weights["layers"]):
            fmt = layer.get("fmt", {})
            for name, kind in kinds.items():
                if fmt.get(name, 8) == 12:
                    self.set_weight_q4_k(kind, li, layer[name])
                else:
                    self.set_weight(kind, li, layer[name])

    @classmethod
    def from_gguf(cls, ctx: Context, path, max_position: int = 8192) -> "Model":
        """A model with the shape and weights of a llama GGUF file
        (ModelWeights::load_from_gguf, src/weights.rs:328-486)."""
        from . import gguf
        g = gguf.GGUFFile(path)
        cfg = gguf.model_config(g, max_position=max_position)
        model = cls(ctx, cfg)
        model.load_weights(gguf.load_weights(g, cfg, lambda a: quantize_q8_0_rows(ctx, a)))
        return model

    def init_random(self, seed: int = 0x5EED0057, std: float = 0.02) -> None:
        _check(self._lib.kanso_model_init_random(self.handle, seed, std))

    def get_weight(self, kind: int, layer: int = 0) -> np.ndarray:
        """One weight back on the host: GGUF Q8_0 bytes of a matrix (uint8), or an f32
        norm vector."""
        c = self.config
        if kind in (_capi.KANSO_W_FINAL_NORM, _capi.KANSO_W_ATTN_NORM, _capi.KANSO_W_FFN_NORM):
            out = np.empty(c.hidden_size, np.float32)
        else:
            hd = c.head_dim
            rows, cols = {
                _capi.KANSO_W_EMBED: (c.vocab_size, c.hidden_size),
                _capi.KANSO_W_LM_HEAD: (c.vocab_size, c.hidden_size),
                _capi.KANSO_W_Q: (c.num_attention_heads * hd, c.hidden_size),
                _capi.KANSO_W_K: (c.num_key_value_heads * hd, c.hidden_size),
                _capi.KANSO_W_V: (c.num_key_value_heads * hd, c.hidden_size),
                _capi.KANSO_W_O: (c.hidden_size, c.num_attention_heads * hd),
                _capi.KANSO_W_GATE: (c.intermediate_size, c.hidden_size),
                _capi.KANSO_W_UP: (c.intermediate_size, c.hidden_size),
                _capi.KANSO_W_DOWN: (c.hidden_size, c.intermediate_size),
            }[kind]
            out = np.empty(rows * cols // 32 * 34, np.uint8)
        _check(self._lib.kanso_model_get_weight(self.handle, kind, layer,
                                                out.ctypes.data_as(C.c_void_p), out.nbytes))
        return out

    def alloc_kv(self, num_blocks: int, block_size: int, max_tokens: int, max_seqs: int,
                 kv_dtype: int = 0) -> None:
        """The paged KV pool; kv_dtype (KANSO_KV_*) as Engine::new_with_budget_and_kv's
        kv_mode (src/engine.rs:62-100): 0 = F32, else a 1-byte pool."""
        _check(self._lib.kanso_model_alloc_kv_quant(self.handle, num_blocks, block_size,
                                                    max_tokens, max_seqs, kv_dtype))

    def kv_pool(self, layer: int) -> tuple[int, int]:
        k, v = C.c_void_p(), C.c_void_p()
        _check(self._lib.kanso_model_kv_pool(self.handle, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def read_kv_rows(self, layer: int, slots) -> tuple[np.ndarray, np.ndarray]:
        """Host copies of the K / V pool rows of `slots` ([n, kv_heads * head_dim])."""
        sl = np.ascontiguousarray(slots, dtype=np.uint64)
        width = self.config.num_key_value_heads * self.config.head_dim
        k = np.zeros((sl.size, width), np.float32)
        v = np.zeros_like(k)
        _check(self._lib.kanso_model_read_kv_rows(self.handle, layer, sl.ctypes.data_as(C.c_void_p),
                                                  sl.size, k.ctypes.data_as(C.c_void_p),
                                                  v.ctypes.data_as(C.c_void_p)))
        return k, v

    def forward(self, plan: np.ndarray, token_arena: np.ndarray, table_arena: np.ndarray,
                logits: torch.Tensor | None = None) -> np.ndarray:
        """One batched forward of a compact plan ([S, 5] u32 rows of start_pos, q_len,
        table_offset, table_len, token_offset); returns the greedy token per sequence."""
        plan = np.ascontiguousarray(plan, dtype=np.uint32)
        toks = np.ascontiguousarray(token_arena, dtype=np.uint32)
        tabs = np.ascontiguousarray(table_arena, dtype=np.uint32)
        S = plan.shape[0]
        out = np.zeros(S, np.uint32)
        _check(self._lib.kanso_model_forward(
            self.handle, plan.ctypes.data_as(C.c_void_p), S, toks.ctypes.data_as(C.c_void_p),
            toks.size, tabs.ctypes.data_as(C.c_void_p), tabs.size,
            None if logits is None else logits.data_ptr(), out.ctypes.data_as(C.c_void_p),
            _stream(None)))
        return out

    def forward_all_rows(self, plan: np.ndarray, token_arena: np.ndarray, table_arena: np.ndarray,
                         logits: torch.Tensor | None = None) -> np.ndarray:
        """Model::forward_batch_all_rows (src/model.rs:1382-1410): the same forward,
        returning the greedy token of every new token (plan order, T entries) and,
        when `logits` is given, writing [T, vocab] into it."""
        plan = np.ascontiguousarray(plan, dtype=np.uint32)
        toks = np.ascontiguousarray(token_arena, dtype=np.uint32)
        tabs = np.ascontiguousarray(table_arena, dtype=np.uint32)
        S = plan.shape[0]
        T = int(plan[:, 1].sum())
        out = np.zeros(T, np.uint32)
        _check(self._lib.kanso_model_forward_all_rows(
            self.handle, plan.ctypes.data_as(C.c_void_p), S, toks.ctypes.data_as(C.c_void_p),
            toks.size, tabs.ctypes.data_as(C.c_void_p), tabs.size,
            None if logits is None else logits.data_ptr(), out.ctypes.data_as(C.c_void_p),
            _stream(None)))
        return out


@dataclass
class StepOutput:
    """src/engine.rs:11-16."""
    request_id: int
    token_id: int
    is_finished: bool


class Engine:
    """Engine::new_with_budget (src/engine.rs:45-125) over the C++ scheduler.
    model=None gives the scheduler alone, committing kanso_engine_dry_token
    stand-in tokens (tests of the planner without a GPU)."""

    def __init__(self, model: Model | None, max_running: int, total_blocks: int,
                 block_size: int = 16, token_budget: int = 512, dry_vocab: int = 0):
        self._lib = _capi.load()
        self.model = model
        h = C.c_void_p()
        _check(self._lib.kanso_engine_create(None if model is None else model.handle, max_running,
                                             total_blocks, block_size, token_budget, dry_vocab,
                                             C.byref(h)))
        self.handle = h
        self.block_size = block_size
        self.token_budget = token_budget
        self._out = (StepOutputC * max(max_running + 1, token_budget + 1))()

    new_with_budget = classmethod(lambda cls, *a, **k: cls(*a, **k))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.kanso_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def add_request(self, prompt_tokens, max_tokens: int, stop_token_ids=()) -> int:
        p = np.ascontiguousarray(prompt_tokens, dtype=np.uint32)
        s = np.ascontiguousarray(stop_token_ids, dtype=np.uint32)
        rid = C.c_uint64(0)
        _check(self._lib.kanso_engine_add_request(self.handle, p.ctypes.data_as(C.c_void_p), p.size,
                                                  max_tokens, s.ctypes.data_as(C.c_void_p), s.size,
                                                  C.byref(rid)))
        return rid.value

    def step(self) -> list[StepOutput]:
        n = C.c_uint32(0)
        _check(self._lib.kanso_engine_step(self.handle, self._out, len(self._out), C.byref(n)))
        return [StepOutput(self._out[i].request_id, self._out[i].token_id,
                           bool(self._out[i].is_finished)) for i in range(n.value)]

    def _stats(self) -> list[int]:
        st = (C.c_uint64 * 10)()
        _check(self._lib.kanso_engine_stats(self.handle, st))
        return list(st)

    def waiting_count(self) -> int:
        return self._stats()[0]

    def running_count(self) -> int:
        return self._stats()[1]

    def free_blocks_count(self) -> int:
        return self._stats()[2]

    def has_unfinished_requests(self) -> bool:
        return self._stats()[3] > 0

    def prefix_cache_hit_rate(self) -> float:
        st = self._stats()
        return 0.0 if st[8] == 0 else min(st[7] / st[8], 1.0)

    def stats(self) -> dict:
        st = self._stats()
        keys = ("waiting", "running", "free_blocks", "unfinished", "sequences", "prefix_hits",
                "prefix_lookups", "prefix_matched_tokens", "prompt_tokens_admitted", "steps")
        return dict(zip(keys, st))

    def drain_finished(self) -> int:
        n = C.c_uint32(0)
        _check(self._lib.kanso_engine_drain_finished(self.handle, C.byref(n)))
        return n.value

    def cancel_request(self, request_id: int) -> bool:
        f = C.c_uint32(0)
        _check(self._lib.kanso_engine_cancel(self.handle, request_id, C.byref(f)))
        return bool(f.value)

    def last_plan(self) -> dict:
        """The last step's flattened batch (src/engine.rs:376-402)."""
        sizes = (C.c_uint32 * 4)()
        _check(self._lib.kanso_engine_last_plan(self.handle, sizes, *([None] * 8)))
        T, S, NT, NR = list(sizes)
        arr = {k: np.zeros(n, dt) for k, n, dt in (
            ("tokens", T, np.uint32), ("positions", T, np.uint32), ("slot_mapping", T, np.uint64),
            ("context_lens", S, np.uint32), ("query_lens", S, np.uint32),
            ("table_lens", S, np.uint32), ("tables", NT, np.uint32),
            ("sample_rows", NR, np.uint32))}
        _check(self._lib.kanso_engine_last_plan(
            self.handle, sizes, *[arr[k].ctypes.data_as(C.c_void_p) for k in (
                "tokens", "positions", "slot_mapping", "context_lens", "query_lens",
                "table_lens", "tables", "sample_rows")]))
        return arr


def dry_token(request_id: int, position: int, vocab: int) -> int:
    return int(_capi.load().kanso_engine_dry_token(request_id, position, vocab))


def fnv1a_64(tokens) -> int:
    """Order-sensitive FNV-1a over u32 tokens widened to u64 (src/bench.rs:20-29)."""
    h = 0xcbf29ce484222325
    for t in tokens:
        h = ((h ^ (int(t) & 0xffffffff)) * 0x100000001b3) & 0xffffffffffffffff
    return h


@dataclass
class TraceEntry:
    """src/bench.rs:31-40."""
    prompt_len: int
    gen_len: int
    arrival_step: int = 0
    prompt_tokens: list | None = None


def synthetic_prompt(req_idx: int, prompt_len: int) -> list:
    """The benchmark's synthetic prompt: token p is (req_idx * 10 + p) % 30
    (src/bench.rs:470-474)."""
    return [(req_idx * 10 + p) % 30 for p in range(prompt_len)]


def generate_poisson_schedule(num_requests: int, rate_lambda: float, seed: int) -> list:
    """Arrival times with exponential gaps -ln(U)/lambda (src/bench/traffic.rs:17-33).
    The reference draws U from rand's StdRng; this build uses numpy's PCG64 with the
    same seed, so the schedule has the same law but not the same values."""
    if num_requests == 0 or rate_lambda <= 0:
        return []
    rng = np.random.default_rng(seed)
    t, out = 0.0, []
    for _ in range(num_requests):
        u = min(max(1.0 - rng.random(), np.finfo(np.float64).tiny), 1.0)
        t += -np.log(u) / rate_lambda
        out.append(t)
    return out


def schedule_to_trace(schedule, prompt_lens, gen_lens, step_duration_secs: float) -> list:
    """Arrival times to arrival steps, floor(t / step) (src/bench/traffic.rs:84-104),
    with per-request prompt / generation lengths."""
    step = step_duration_secs if step_duration_secs > 0 else 0.001
    return [TraceEntry(int(p), int(g), int(np.floor(t / step)))
            for t, p, g in zip(schedule, prompt_lens, gen_lens)]


def run_benchmark_workload(engine: Engine, requests: list, on_step=None) -> dict:
    """execute_engine_run (src/bench.rs:447-537): requests are added at their arrival
    step (stable order by arrival), one engine step per loop until every request has
    finished; the checksum is fnv1a_64 of the generated tokens in emit order."""
    order = sorted(range(len(requests)), key=lambda i: requests[i].arrival_step)
    nxt = step_idx = decode_steps = 0
    generated = []
    prefill_s = decode_s = 0.0
    t0 = time.perf_counter()
    while True:
        while nxt < len(order) and requests[order[nxt]].arrival_step <= step_idx:
            ri = order[nxt]
            e = requests[ri]
            prompt = e.prompt_tokens if e.prompt_tokens is not None else synthetic_prompt(ri, e.prompt_len)
            engine.add_request(prompt, e.gen_len)
            nxt += 1
        if nxt >= len(order) and not engine.has_unfinished_requests():
            break
        st = engine.stats()
        prefilling = st["waiting"] > 0 or _any_prefilling(engine)
        s0 = time.perf_counter()
        outs = engine.step()
        dt = time.perf_counter() - s0
        if prefilling:
            prefill_s += dt
        if outs:
            decode_steps += 1
            decode_s += dt
        if on_step is not None:
            on_step(engine, outs)
        generated.extend(o.token_id for o in outs)
        step_idx += 1
    total = time.perf_counter() - t0
    return {
        "total_tokens": len(generated),
        "total_duration_secs": total,
        "num_requests": len(requests),
        "total_tokens_per_sec": len(generated) / total if total > 0 else 0.0,
        "steps": step_idx,
        "decode_steps": decode_steps,
        "decode_ms_per_step": 1000.0 * decode_s / max(decode_steps, 1),
        "prefill_secs": prefill_s,
        "checksum": fnv1a_64(generated),
        "generated": generated,
        "prefix_hit_rate": engine.prefix_cache_hit_rate(),
    }


def _any_prefilling(engine: Engine) -> bool:
    # The reference tests "a running sequence is still prefilling" per sequence; the
    # last plan's prefill rows say the same thing for the step about to run.
    plan = engine.last_plan()
    return bool((plan["query_lens"] > 1).any()) if plan["query_lens"].size else False
