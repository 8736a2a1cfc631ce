"""Independent float64 numpy formulations used to pin the oracle.

These are written from the mathematics of the operation (gather the context
through the table, softmax over masked scores, weighted sum of V), vectorised,
in float64 — not a transcription of the oracle's f32 loops — so that an indexing
slip, a dropped term or a wrong mask in the oracle shows up as a mismatch far
above float32 rounding.
"""
from __future__ import annotations

import numpy as np


def gather_context(pool: np.ndarray, table_row: np.ndarray, ctx: int, block_size: int,
                   num_kv_heads: int, head_dim: int) -> np.ndarray:
    """[ctx, Hkv, D] rows of sequence's context from a [blocks, bs, Hkv, D] pool."""
    p = pool.reshape(-1, block_size, num_kv_heads, head_dim)
    t = np.arange(ctx)
    return p[table_row[t // block_size], t % block_size]


def attention_f64(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, tables: np.ndarray,
                  cu_seqlens: np.ndarray, context_lens: np.ndarray, num_heads: int,
                  num_kv_heads: int, head_dim: int, block_size: int, scale: float) -> np.ndarray:
    """Ragged causal GQA attention in float64: row i of a sequence with q_len rows and
    context c attends keys 0..=c-q_len+i."""
    S = cu_seqlens.size - 1
    T = int(cu_seqlens[-1])
    G = num_heads // num_kv_heads
    qv = q.reshape(T, num_heads, head_dim).astype(np.float64)
    out = np.zeros((T, num_heads, head_dim))
    tables = tables.reshape(S, -1)
    for s in range(S):
        r0, r1 = int(cu_seqlens[s]), int(cu_seqlens[s + 1])
        ql, c = r1 - r0, int(context_lens[s])
        if c == 0:
            continue
        K = gather_context(k_pool, tables[s], c, block_size, num_kv_heads, head_dim).astype(np.float64)
        V = gather_context(v_pool, tables[s], c, block_size, num_kv_heads, head_dim).astype(np.float64)
        # scores [ql, H, c]
        kh = np.repeat(K, G, axis=1)  # [c, H, D], head h reads kv head h // G
        vh = np.repeat(V, G, axis=1)
        sc = np.einsum("qhd,chd->qhc", qv[r0:r1], kh) * scale
        limit = (c - ql + np.arange(ql))[:, None, None]
        sc = np.where(np.arange(c)[None, None, :] <= limit, sc, -np.inf)
        sc -= sc.max(axis=2, keepdims=True)
        w = np.exp(sc)
        w /= w.sum(axis=2, keepdims=True)
        out[r0:r1] = np.einsum("qhc,chd->qhd", w, vh)
    return out.reshape(-1)


def round_half_away(x: np.ndarray) -> np.ndarray:
    """Rust f32::round on float64 values (exact for any f32 input)."""
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def quantize_int8_f64(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """quantize_head_slice INT8 from its definition; divisions rounded to f32 exactly as
    IEEE single precision does (numpy float32 division is correctly rounded)."""
    x = x.astype(np.float32)
    amax = np.float32(np.abs(x).max()) if x.size else np.float32(0)
    scale = np.float32(amax / np.float32(127.0)) if amax > 0 else np.float32(1.0)
    inv = np.float32(np.float32(1.0) / scale)
    prod = (x * inv).astype(np.float32).astype(np.float64)
    q = np.clip(round_half_away(prod), -127, 127).astype(np.int8)
    return q, scale


def quantize_q8_0_f64(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    x = x.astype(np.float32)
    amax = np.float32(np.abs(x).max())
    d = np.float32(amax / np.float32(127.0))
    idv = np.float32(np.float32(1.0) / d) if d != 0 else np.float32(0.0)
    prod = (x * idv).astype(np.float32).astype(np.float64)
    q = np.clip(round_half_away(prod), -128, 127).astype(np.int8)
    return q, d


def scale_min_k4_table(scales12) -> list[tuple[int, int]]:
    """The 8 (scale, min) pairs of a Q4_K scale array, decoded bit by bit from the
    llama.cpp / GGUF packing description: sub-blocks 0..3 keep 6-bit scale and min in
    the low bits of bytes 0..3 and 4..7; sub-blocks 4..7 take their low 4 bits from
    the nibbles of bytes 8..11 and their high 2 bits from the top bits of bytes 0..7."""
    b = [int(v) for v in scales12]
    out = []
    for j in range(8):
        if j < 4:
            out.append((b[j] % 64, b[j + 4] % 64))
        else:
            lo_sc, lo_m = b[j + 4] % 16, b[j + 4] // 16
            hi_sc, hi_m = b[j - 4] // 64, b[j] // 64
            out.append((lo_sc + 16 * hi_sc, lo_m + 16 * hi_m))
    return out


def dequant_q4k_f64(d: float, dmin: float, scales12, qs128) -> np.ndarray:
    """Q4_K super-block from the format description: element 64c + l (l < 32) is the low
    nibble of qs[32c + l] in sub-block 2c, element 64c + 32 + l the high nibble in
    sub-block 2c + 1; value = d * sc * nibble - dmin * m."""
    pairs = scale_min_k4_table(scales12)
    qs = np.asarray(qs128, dtype=np.int64)
    out = np.zeros(256)
    for c in range(4):
        sc1, m1 = pairs[2 * c]
        sc2, m2 = pairs[2 * c + 1]
        lo = qs[32 * c:32 * c + 32] & 0xF
        hi = qs[32 * c:32 * c + 32] >> 4
        out[64 * c:64 * c + 32] = d * sc1 * lo - dmin * m1
        out[64 * c + 32:64 * c + 64] = d * sc2 * hi - dmin * m2
    return out


def q8_0_gguf_to_dense(w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Dense float64 weights of GGUF block_q8_0 bytes (numpy float16 decodes d)."""
    blk = w.reshape(rows, cols // 32, 34)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)  # [rows, nb, 1]
    qs = blk[:, :, 2:].view(np.int8).astype(np.float64)
    return (qs * d).reshape(rows, cols)


def q4k_gguf_to_dense(w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    blk = w.reshape(rows, cols // 256, 144)
    out = np.zeros((rows, cols))
    for r in range(rows):
        for b in range(cols // 256):
            raw = blk[r, b]
            d = float(raw[0:2].copy().view(np.float16)[0])
            dmin = float(raw[2:4].copy().view(np.float16)[0])
            out[r, b * 256:(b + 1) * 256] = dequant_q4k_f64(d, dmin, raw[4:16], raw[16:144])
    return out
