"""numpy front end of the CPU oracle (oracle/libkanso_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker. The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libkanso_oracle.so"

KV_F32, KV_INT8, KV_Q8_0, KV_FP8 = 0, 1, 2, 3

_lib: C.CDLL | None = None


class PagedParams(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("num_seqs", "num_heads", "num_kv_heads", "head_dim",
                                          "block_size", "max_num_blocks_per_seq")] + [
        ("scale", C.c_float)]


class RaggedParams(C.Structure):
    _fields_ = PagedParams._fields_ + [(n, C.c_uint32) for n in (
        "total_q", "kv_dtype", "num_blocks", "max_q_len", "pool_layout")]


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        _lib = C.CDLL(str(LIB_PATH))
        V, U, I, F = C.c_void_p, C.c_uint32, C.c_int, C.c_float
        sig = {
            "oracle_paged_attention": (None, [V, V, V, V, V, C.POINTER(PagedParams), V]),
            "oracle_ragged_attention": (I, [V, V, V, V, V, V, V, V, C.POINTER(RaggedParams), V, I]),
            "oracle_pack_step": (I, [V, U, V, V, U, V, V, V, V, V, V, V, V]),
            "oracle_quantize_head_int8": (F, [V, U, V]),
            "oracle_quantize_head_fp8": (F, [V, U, V]),
            "oracle_stream_triad": (C.c_double, [C.c_uint64, I, I]),
            "oracle_f32_to_e4m3": (C.c_uint8, [F]),
            "oracle_e4m3_to_f32": (F, [C.c_uint8]),
            "oracle_quantize_q8_0_block": (F, [V, V]),
            "oracle_f32_to_f16": (C.c_uint16, [F]),
            "oracle_f16_to_f32": (F, [C.c_uint16]),
            "oracle_kv_append": (I, [U, V, V, V, U, U, U, U, U, V, V, V, V]),
            "oracle_gemv_q8_0": (None, [V, V, V, U, U, U, I]),
            "oracle_gemv_q8_0_f32d": (None, [V, V, V, U, U, U]),
            "oracle_dequant_q4_k": (None, [V, V]),
            "oracle_dequant_q4_k_f32d": (None, [V, V]),
            "oracle_get_scale_min_k4": (None, [U, V, V, V]),
            "oracle_gemv_q4_k": (None, [V, V, V, U, U, U, I]),
            "oracle_gemv_q4_k_f32d": (None, [V, V, V, U, U, U]),
            "oracle_quantize_row_q8_0": (None, [V, U, V]),
            "oracle_quantize_row_q4_k": (None, [V, U, V]),
            "oracle_dequant_row_q8_0": (None, [V, U, V]),
            "oracle_rmsnorm": (None, [V, V, V, U, U, F]),
            "oracle_rope_table": (None, [U, U, F, V, V]),
            "oracle_rope_apply": (None, [V, U, U, U, V, V, V]),
            "oracle_silu_mul": (None, [V, V, V, U]),
            "oracle_greedy": (U, [V, U]),
            "oracle_fnv1a_64": (C.c_uint64, [V, C.c_size_t]),
            "oracle_splitmix64": (C.c_uint64, [C.c_uint64]),
            "oracle_randn_scale": (F, [F]),
            "oracle_init_random_q8_0": (I, [C.c_uint64, U, U, F, V]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def splitmix64(x: int) -> int:
    return int(lib().oracle_splitmix64(x & (2**64 - 1)))


def init_random_q8_0(stream_seed: int, rows: int, cols: int, std: float) -> np.ndarray:
    """kanso_model_init_random's matrix (GGUF Q8_0 bytes, uint8) for one stream seed."""
    out = np.empty(rows * cols // 32 * 34, np.uint8)
    c = lib().oracle_randn_scale(std)
    if lib().oracle_init_random_q8_0(stream_seed & (2**64 - 1), rows, cols, c, _p(out)) != 0:
        raise ValueError("cols must be a multiple of 32")
    return out


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def paged_attention(q, k_cache, v_cache, block_tables, context_lens, num_seqs, num_heads,
                    num_kv_heads, head_dim, block_size, max_num_blocks_per_seq, scale):
    """cpu_paged_attention (src/metal/paged_attention.rs:84-178)."""
    q, k, v = _f32(q), _f32(k_cache), _f32(v_cache)
    t, l = _u32(block_tables), _u32(context_lens)
    p = PagedParams(num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                    max_num_blocks_per_seq, scale)
    out = np.zeros(num_seqs * num_heads * head_dim, dtype=np.float32)
    lib().oracle_paged_attention(_p(q), _p(k), _p(v), _p(t), _p(l), C.byref(p), _p(out))
    return out


def ragged_attention(q, k_pool, v_pool, block_tables, cu_seqlens, context_lens, *, num_heads,
                     num_kv_heads, head_dim, block_size, scale, kv_dtype=KV_F32, k_scales=None,
                     v_scales=None, num_blocks, nthreads=1):
    """Mixed-batch attention (src/model.rs:1689-1714 semantics, decode arithmetic)."""
    q = _f32(q)
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
    lens = _u32(context_lens)
    S = cu.size - 1
    tables = _u32(block_tables)
    max_blocks = tables.size // S
    T = int(cu[-1])
    kp = np.ascontiguousarray(k_pool)
    vp = np.ascontiguousarray(v_pool)
    ks = None if k_scales is None else np.ascontiguousarray(k_scales)
    vs = None if v_scales is None else np.ascontiguousarray(v_scales)
    p = RaggedParams(S, num_heads, num_kv_heads, head_dim, block_size, max_blocks, scale, T,
                     kv_dtype, num_blocks, 0)
    out = np.zeros(T * num_heads * head_dim, dtype=np.float32)
    rc = lib().oracle_ragged_attention(_p(q), _p(kp), _p(vp), _p(ks), _p(vs), _p(tables), _p(cu),
                                       _p(lens), C.byref(p), _p(out), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_ragged_attention rejected the batch")
    return out


def pack_step(plan, token_arena, table_arena, block_size):
    """Engine::step packing + PaddedDecodeTables (dict of numpy arrays)."""
    plan = _u32(plan).reshape(-1, 5)
    S = plan.shape[0]
    T = int(plan[:, 1].sum())
    ctx = plan[:, 0].astype(np.int64) + plan[:, 1]
    mb = int(max(1, ((ctx + block_size - 1) // block_size).max(initial=1)))
    out = dict(cu_seqlens=np.zeros(S + 1, np.int32), seq_of_query=np.zeros(T, np.int32),
               positions=np.zeros(T, np.int32), slot_mapping=np.zeros(T, np.int64),
               tokens=np.zeros(T, np.uint32), block_tables=np.zeros(S * mb, np.uint32),
               context_lens=np.zeros(S, np.uint32))
    mbo = C.c_uint32(0)
    ta, tb = _u32(token_arena), _u32(table_arena)
    rc = lib().oracle_pack_step(_p(plan), S, _p(ta), _p(tb), block_size, _p(out["cu_seqlens"]),
                                _p(out["seq_of_query"]), _p(out["positions"]),
                                _p(out["slot_mapping"]), _p(out["tokens"]),
                                _p(out["block_tables"]), _p(out["context_lens"]), C.byref(mbo))
    if rc != 0:
        raise ValueError("oracle_pack_step: block table too short")
    out["max_blocks"] = mbo.value
    return out


def quantize_head_int8(x):
    x = _f32(x)
    q = np.zeros(x.size, dtype=np.int8)
    s = lib().oracle_quantize_head_int8(_p(x), x.size, _p(q))
    return q, np.float32(s)


def quantize_head_fp8(x):
    x = _f32(x)
    q = np.zeros(x.size, dtype=np.uint8)
    s = lib().oracle_quantize_head_fp8(_p(x), x.size, _p(q))
    return q, np.float32(s)


def f32_to_e4m3(x: float) -> int:
    return int(lib().oracle_f32_to_e4m3(C.c_float(float(x))))


def e4m3_to_f32(b: int) -> float:
    return float(lib().oracle_e4m3_to_f32(C.c_uint8(int(b))))


def quantize_q8_0_block(x):
    x = _f32(x)
    assert x.size == 32
    q = np.zeros(32, dtype=np.int8)
    d = lib().oracle_quantize_q8_0_block(_p(x), _p(q))
    return q, np.float32(d)


def f32_to_f16_bits(x: float) -> int:
    return int(lib().oracle_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(int(h)))


def kv_pool_arrays(kv_dtype, num_blocks, block_size, num_kv_heads, head_dim):
    """Zeroed (k_pool, v_pool, k_scales, v_scales) host arrays for a pool kind."""
    rows = num_blocks * block_size * num_kv_heads
    if kv_dtype == KV_F32:
        return (np.zeros(rows * head_dim, np.float32), np.zeros(rows * head_dim, np.float32),
                None, None)
    if kv_dtype in (KV_INT8, KV_FP8):
        return (np.zeros(rows * head_dim, np.int8), np.zeros(rows * head_dim, np.int8),
                np.ones(rows, np.float32), np.ones(rows, np.float32))
    return (np.zeros(rows * head_dim, np.int8), np.zeros(rows * head_dim, np.int8),
            np.zeros(rows * head_dim // 32, np.uint16), np.zeros(rows * head_dim // 32, np.uint16))


def kv_append(kv_dtype, k, v, slot_mapping, num_blocks, block_size, num_kv_heads, head_dim,
              k_pool, v_pool, k_scales=None, v_scales=None):
    """write_kv_slots on host arrays (modified in place)."""
    k, v = _f32(k), _f32(v)
    sm = np.ascontiguousarray(np.asarray(slot_mapping, dtype=np.int64))
    rc = lib().oracle_kv_append(kv_dtype, _p(k), _p(v), _p(sm), sm.size, num_blocks, block_size,
                                num_kv_heads, head_dim, _p(k_pool), _p(v_pool), _p(k_scales),
                                _p(v_scales))
    if rc != 0:
        raise ValueError("oracle_kv_append: slot out of bounds")


def quantize_row_q8_0(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    lib().oracle_quantize_row_q8_0(_p(x), x.size, _p(out))
    return out


def dequant_q8_0_rows(blocks: np.ndarray, cols: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = b.size // 34 * 32
    out = np.zeros(n, np.float32)
    lib().oracle_dequant_row_q8_0(_p(b), n, _p(out))
    return out.reshape(-1, cols)


def quantize_row_q4_k(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size // 256 * 144, dtype=np.uint8)
    lib().oracle_quantize_row_q4_k(_p(x), x.size, _p(out))
    return out


def gemv_q8_0(w: np.ndarray, x, rows, cols, nthreads=1):
    x = _f32(x)
    batch = x.size // cols
    y = np.zeros(batch * rows, dtype=np.float32)
    lib().oracle_gemv_q8_0(_p(np.ascontiguousarray(w)), _p(x), _p(y), rows, cols, batch, nthreads)
    return y


def gemv_q8_0_f32d(w: np.ndarray, x, rows, cols):
    x = _f32(x)
    batch = x.size // cols
    y = np.zeros(batch * rows, dtype=np.float32)
    lib().oracle_gemv_q8_0_f32d(_p(np.ascontiguousarray(w)), _p(x), _p(y), rows, cols, batch)
    return y


def gemv_q4_k(w: np.ndarray, x, rows, cols, nthreads=1):
    x = _f32(x)
    batch = x.size // cols
    y = np.zeros(batch * rows, dtype=np.float32)
    lib().oracle_gemv_q4_k(_p(np.ascontiguousarray(w)), _p(x), _p(y), rows, cols, batch, nthreads)
    return y


def gemv_q4_k_f32d(w: np.ndarray, x, rows, cols):
    x = _f32(x)
    batch = x.size // cols
    y = np.zeros(batch * rows, dtype=np.float32)
    lib().oracle_gemv_q4_k_f32d(_p(np.ascontiguousarray(w)), _p(x), _p(y), rows, cols, batch)
    return y


def dequant_q4_k(block: np.ndarray, f32d: bool = False) -> np.ndarray:
    out = np.zeros(256, dtype=np.float32)
    fn = lib().oracle_dequant_q4_k_f32d if f32d else lib().oracle_dequant_q4_k
    fn(_p(np.ascontiguousarray(block)), _p(out))
    return out


def get_scale_min_k4(j: int, scales12) -> tuple[int, int]:
    s = np.ascontiguousarray(np.asarray(scales12, dtype=np.uint8))
    sc, m = C.c_uint8(0), C.c_uint8(0)
    lib().oracle_get_scale_min_k4(j, _p(s), C.byref(sc), C.byref(m))
    return sc.value, m.value


def rmsnorm(x, w, eps=1e-5):
    x, w = _f32(x), _f32(w)
    n = w.size
    y = np.zeros_like(x)
    lib().oracle_rmsnorm(_p(x), _p(w), _p(y), x.size // n, n, eps)
    return y


def rope_table(length, head_dim, theta=10000.0):
    half = head_dim // 2
    c = np.zeros(length * half, np.float32)
    s = np.zeros(length * half, np.float32)
    lib().oracle_rope_table(length, head_dim, theta, _p(c), _p(s))
    return c.reshape(length, half), s.reshape(length, half)


def rope_apply(x, positions, heads, head_dim, cos_t, sin_t):
    x = _f32(x).copy()
    pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int32))
    lib().oracle_rope_apply(_p(x), pos.size, heads, head_dim, _p(pos), _p(_f32(cos_t)),
                            _p(_f32(sin_t)))
    return x


def silu_mul(gate, up):
    g, u = _f32(gate), _f32(up)
    y = np.zeros_like(g)
    lib().oracle_silu_mul(_p(g), _p(u), _p(y), g.size)
    return y


def greedy(logits) -> int:
    x = _f32(logits)
    return int(lib().oracle_greedy(_p(x), x.size))


def fnv1a_64(tokens) -> int:
    t = _u32(tokens)
    return int(lib().oracle_fnv1a_64(_p(t), t.size))


def available() -> bool:
    return LIB_PATH.exists() or os.environ.get("KANSO_ORACLE_BUILD") == "1"


# ---------------------------------------------------------------- batched forward


class ModelConfigC(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "num_heads", "num_kv_heads", "head_dim",
                                          "num_layers", "intermediate", "vocab")] + [
        ("eps", C.c_float), ("rope_theta", C.c_float), ("weight_format", C.c_uint32),
        ("kv_dtype", C.c_uint32), ("embedding_scale", C.c_float), ("attention_scale", C.c_float),
        ("residual_scale", C.c_float), ("logit_scale", C.c_float)]


class ModelWeightsC(C.Structure):
    _fields_ = [("embed", C.c_void_p), ("lm_head", C.c_void_p), ("final_norm", C.c_void_p)] + [
        (n, C.POINTER(C.c_void_p)) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down",
                                             "attn_norm", "ffn_norm")] + [
        ("formats", C.c_void_p)]


def forward_batch(cfg: dict, weights: dict, k_pools, v_pools, num_blocks, block_size, tokens,
                  positions, slot_mapping, block_tables, max_blocks, cu_seqlens, context_lens,
                  nthreads=8, all_rows=False, k_scales=None, v_scales=None) -> np.ndarray:
    """oracle_forward_batch_rows: logits [S, vocab] of each sequence's last row, or with
    all_rows [T, vocab] of every new token (forward_batch_all_rows). k_pools / v_pools
    are per-layer float32 arrays updated in place (write_kv_slots)."""
    L = cfg["num_layers"]
    c = ModelConfigC(cfg["hidden"], cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"], L,
                     cfg["intermediate"], cfg["vocab"], cfg.get("eps", 1e-5),
                     cfg.get("rope_theta", 10000.0), cfg.get("weight_format", 0),
                     cfg.get("kv_dtype", KV_F32), cfg.get("embedding_scale", 0.0),
                     cfg.get("attention_scale", 0.0), cfg.get("residual_scale", 0.0),
                     cfg.get("logit_scale", 0.0))
    keep = []

    def arr(name):
        a = (C.c_void_p * L)(*[_p(np.ascontiguousarray(layer[name])).value
                                for layer in weights["layers"]])
        keep.append(a)
        return C.cast(a, C.POINTER(C.c_void_p))

    lm = weights.get("lm_head", weights["embed"])
    names = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
    fmts = np.array([[layer.get("fmt", {}).get(n, 8) for n in names] for layer in weights["layers"]],
                    np.uint32)
    keep.append(fmts)
    w = ModelWeightsC(_p(weights["embed"]), _p(lm), _p(weights["final_norm"]),
                      *[arr(n) for n in (*names, "attn_norm", "ffn_norm")], _p(fmts))
    kp = (C.c_void_p * L)(*[_p(k).value for k in k_pools])
    vp = (C.c_void_p * L)(*[_p(v).value for v in v_pools])
    quant = cfg.get("kv_dtype", KV_F32) != KV_F32
    ksp = (C.c_void_p * L)(*[_p(k).value for k in k_scales]) if quant else None
    vsp = (C.c_void_p * L)(*[_p(v).value for v in v_scales]) if quant else None
    tokens = _u32(tokens)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    tables = _u32(block_tables)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    ctx = _u32(context_lens)
    S = ctx.size
    logits = np.zeros((tokens.size if all_rows else S, cfg["vocab"]), np.float32)
    fn = lib().oracle_forward_batch_rows
    fn.restype = C.c_int
    rc = fn(C.byref(c), C.byref(w), _p(tokens), _p(positions), _p(slots), C.c_uint32(tokens.size),
            C.cast(kp, C.POINTER(C.c_void_p)), C.cast(vp, C.POINTER(C.c_void_p)),
            C.cast(ksp, C.POINTER(C.c_void_p)) if quant else None,
            C.cast(vsp, C.POINTER(C.c_void_p)) if quant else None,
            C.c_uint32(num_blocks), C.c_uint32(block_size), _p(tables), C.c_uint32(max_blocks),
            _p(cu), _p(ctx), C.c_uint32(S), C.c_int(1 if all_rows else 0), _p(logits),
            C.c_int(nthreads))
    if rc != 0:
        raise RuntimeError("oracle_forward_batch rejected the batch")
    return logits


def stream_triad_gbps(n: int = 1 << 26, nthreads: int = 1, reps: int = 5) -> float:
    """Host STREAM-triad bandwidth in GB/s (n doubles per array)."""
    return float(lib().oracle_stream_triad(n, nthreads, reps))
