"""kanso_infer_amd — MI355X (gfx950) implementation of kanso-infer's ragged
continuous-batching attention path.

The compute lives in libkanso_hip.so (hand-written HIP, C ABI in
include/kanso_hip.h). This module is the thin host layer over it: device buffers
and streams are torch tensors / streams (plumbing only), and every call goes
through the C ABI. It mirrors the reference's own entry points for the path:

  PagedAttentionParams, paged_attention_num_partitions,
  validate_paged_attention_params, gpu_paged_attention_v2
      <- src/metal/paged_attention.rs:12-81, 328-382
  ragged_paged_attention   <- the mixed-batch attention of src/model.rs:1689-1714
  pack_step                <- Engine::step packing, src/engine.rs:376-402
  kv_append / kv_reset_blocks <- KvStorageKind::write_kv_slots / reset_block
  gemv_q8_0 / gemv_q4_k    <- LinearWeight::forward on Q8_0 / Q4_K weights
  q8_0_pack, gemm_q8_0, gemm_q8_0_residual, embed_q8_0, qkv_rope_append,
  qkv_rope_append_quant, gate_up_swiglu, lm_head_argmax
                           <- the layer body of Model::forward_batch_rows
                              (src/model.rs:1569-1739) on packed Q8_0 weights

Errors are raised as EngineError (src/error.rs:4-11), never swallowed: there is
no CPU fallback, and a missing library is an error.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _capi
from ._capi import (KANSO_KV_F32, KANSO_KV_FP8, KANSO_KV_INT8, KANSO_KV_Q8_0, PackedStepC,
                    PagedAttentionParamsC, RaggedAttentionParamsC, SeqPlanC)

__all__ = [
    "EngineError", "Context", "PagedAttentionParams", "paged_attention_num_partitions",
    "validate_paged_attention_params", "gpu_paged_attention_v2", "paged_attention_v2",
    "ragged_paged_attention", "ragged_work", "pack_step", "kv_append", "kv_reset_blocks", "gemv_q8_0",
    "gemv_q4_k", "KANSO_KV_F32", "KANSO_KV_INT8", "KANSO_KV_Q8_0", "KANSO_KV_FP8", "ragged_partition_size", "ragged_chunk_partition_size", "q8_0_packed_bytes",
    "q8_0_pack", "gemm_q8_0", "gemm_q8_0_residual", "embed_q8_0", "qkv_rope_append",
    "qkv_rope_append_quant",
    "gate_up_swiglu", "lm_head_argmax",
]


class EngineError(RuntimeError):
    """Error of the path (the reference's EngineError::Metal / ::Model, src/error.rs:4-11)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def _check(rc: int) -> None:
    if rc != _capi.KANSO_OK:
        msg = _capi.load().kanso_last_error().decode(errors="replace")
        raise EngineError(rc, msg)


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise EngineError(_capi.KANSO_E_INVALID_ARG, "buffers must be device tensors")
    if not t.is_contiguous():
        raise EngineError(_capi.KANSO_E_INVALID_ARG, "buffers must be contiguous")
    return t.data_ptr()


def _stream(stream: torch.cuda.Stream | None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class Context:
    """A kanso_ctx on one device: owns split-K scratch and the device status word."""

    def __init__(self, device: int = 0):
        self._lib = _capi.load()
        torch.cuda.set_device(device)
        h = C.c_void_p()
        _check(self._lib.kanso_create(device, C.byref(h)))
        self.handle = h
        self.device = device

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.kanso_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter teardown order varies
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def check_device_status(self, stream: torch.cuda.Stream | None = None) -> int:
        """Synchronises and raises EngineError if a kernel flagged bad input."""
        flags = C.c_uint32(0)
        _check(self._lib.kanso_check_device_status(self.handle, _stream(stream), C.byref(flags)))
        return flags.value

    def set_profiling(self, enabled: bool) -> None:
        _check(self._lib.kanso_set_profiling(self.handle, int(enabled)))

    def kernel_time(self, name: str) -> tuple[float, int]:
        """(total ms, launches) of a library kernel timed with HIP events."""
        ms = C.c_double(0.0)
        n = C.c_uint64(0)
        _check(self._lib.kanso_get_kernel_time(self.handle, name.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value


# ---------------------------------------------------------------- params mirror


@dataclass
class PagedAttentionParams:
    """src/metal/paged_attention.rs:12-22 (same fields, same order)."""
    num_seqs: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    max_num_blocks_per_seq: int
    scale: float

    def to_c(self) -> PagedAttentionParamsC:
        return PagedAttentionParamsC(self.num_seqs, self.num_heads, self.num_kv_heads,
                                     self.head_dim, self.block_size,
                                     self.max_num_blocks_per_seq, self.scale)


def paged_attention_num_partitions(params: PagedAttentionParams) -> int:
    """src/metal/paged_attention.rs:27-32."""
    p = params.to_c()
    return int(_capi.load().kanso_paged_attention_num_partitions(C.byref(p)))


def validate_paged_attention_params(params: PagedAttentionParams) -> None:
    """src/metal/paged_attention.rs:39-81; raises EngineError on an unrepresentable shape."""
    p = params.to_c()
    _check(_capi.load().kanso_validate_paged_attention_params(C.byref(p)))


# ---------------------------------------------------------------- attention


def paged_attention_v2(ctx: Context, params: PagedAttentionParams, q: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                       context_lens: torch.Tensor, out: torch.Tensor,
                       stream: torch.cuda.Stream | None = None) -> None:
    """Device-buffer decode attention (encode_paged_attention_v2, paged_attention.rs:193-293)."""
    p = params.to_c()
    _check(ctx._lib.kanso_paged_attention_v2(
        ctx.handle, C.byref(p), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
        _ptr(context_lens), _ptr(out), _stream(stream)))


def gpu_paged_attention_v2(ctx: Context, q, k_cache, v_cache, block_tables, context_lens,
                           params: PagedAttentionParams) -> np.ndarray:
    """Host-array wrapper (gpu_paged_attention_v2, paged_attention.rs:328-382): rejects a
    context longer than the table capacity and an empty context before any upload,
    copies to the device, runs, and returns the [seqs, heads, head_dim] output."""
    capacity = params.max_num_blocks_per_seq * params.block_size
    lens = np.asarray(context_lens, dtype=np.uint32)
    for length in lens:
        if length > capacity:
            raise EngineError(_capi.KANSO_E_OUT_OF_BOUNDS,
                              f"paged attention: context_len {length} exceeds block table "
                              f"capacity {capacity}")
    if (lens == 0).any():
        raise EngineError(_capi.KANSO_E_INVALID_SHAPE,
                          "paged attention: context_len must be non-zero "
                          "(empty context merges to NaN)")
    validate_paged_attention_params(params)
    dev = torch.device("cuda", ctx.device)

    def up(a, dt):
        return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=dt))).to(dev)

    q_d = up(q, np.float32)
    k_d = up(k_cache, np.float32)
    v_d = up(v_cache, np.float32)
    t_d = up(np.asarray(block_tables, dtype=np.uint32).view(np.int32), np.int32)
    l_d = up(lens.view(np.int32), np.int32)
    out = torch.empty(params.num_seqs * params.num_heads * params.head_dim, dtype=torch.float32,
                      device=dev)
    paged_attention_v2(ctx, params, q_d, k_d, v_d, t_d, l_d, out)
    ctx.check_device_status()
    return out.cpu().numpy()


def ragged_paged_attention(ctx: Context, *, q: torch.Tensor, k_pool: torch.Tensor,
                           v_pool: torch.Tensor, block_tables: torch.Tensor,
                           cu_seqlens: torch.Tensor | None, context_lens: torch.Tensor,
                           out: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int,
                           block_size: int, scale: float, kv_dtype: int = KANSO_KV_F32,
                           k_scales: torch.Tensor | None = None,
                           v_scales: torch.Tensor | None = None, num_blocks: int = 0,
                           max_q_len: int = 0, pool_layout: int = 0, partition_size: int = 0,
                           chunk_partition_size: int = 0, work: torch.Tensor | None = None,
                           work_chunk_items: int = 0,
                           stream: torch.cuda.Stream | None = None) -> None:
    """Mixed prefill + decode attention over the paged pool (kanso_ragged_paged_attention).
    cu_seqlens None: a decode batch, one query row per sequence. work: a device copy of
    ragged_work's list, work_chunk_items its chunk items (kanso_ragged_paged_attention_work)."""
    num_seqs = cu_seqlens.numel() - 1 if cu_seqlens is not None else context_lens.numel()
    max_blocks = block_tables.numel() // max(num_seqs, 1)
    total_q = q.numel() // (num_heads * head_dim)
    p = RaggedAttentionParamsC(num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_blocks,
                               scale, total_q, kv_dtype, num_blocks, max_q_len, pool_layout,
                               partition_size, chunk_partition_size)
    args = (ctx.handle, C.byref(p), _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(k_scales),
            _ptr(v_scales), _ptr(block_tables), _ptr(cu_seqlens), _ptr(context_lens), _ptr(out))
    if work is None:
        _check(ctx._lib.kanso_ragged_paged_attention(*args, _stream(stream)))
    else:
        _check(ctx._lib.kanso_ragged_paged_attention_work(
            *args, _ptr(work), work.numel() // _capi.KANSO_RAGGED_WORK_ITEM_WORDS, work_chunk_items,
            _stream(stream)))


def ragged_work(*, q_lens, context_lens, block_tables, num_heads: int, num_kv_heads: int,
                head_dim: int, block_size: int, partition_size: int, kv_dtype: int = KANSO_KV_F32,
                num_blocks: int = 0, max_q_len: int = 0, pool_layout: int = 0,
                chunk_partition_size: int = 0) -> tuple[np.ndarray, int] | None:
    """The work list of a planned batch (kanso_ragged_build_work) from host lengths and
    the host copy of the [S, max_blocks] block table, and the number of chunk items
    at its end; None when the batch cannot take one (kanso_ragged_work_items == 0).
    Host-only."""
    lib = _capi.load()
    ql = np.ascontiguousarray(np.asarray(q_lens, dtype=np.uint32))
    cl = np.ascontiguousarray(np.asarray(context_lens, dtype=np.uint32))
    tabs = np.ascontiguousarray(np.asarray(block_tables, dtype=np.uint32).reshape(ql.size, -1))
    p = RaggedAttentionParamsC(ql.size, num_heads, num_kv_heads, head_dim, block_size, tabs.shape[1],
                               1.0, int(ql.sum()), kv_dtype, num_blocks, max_q_len, pool_layout,
                               partition_size, chunk_partition_size)
    nc = C.c_uint32(0)
    n = int(lib.kanso_ragged_work_items(C.byref(p), ql.ctypes.data_as(C.c_void_p),
                                        cl.ctypes.data_as(C.c_void_p), C.byref(nc)))
    if n == 0:
        return None
    out = np.zeros(n * _capi.KANSO_RAGGED_WORK_ITEM_WORDS, np.uint32)
    _check(lib.kanso_ragged_build_work(C.byref(p), ql.ctypes.data_as(C.c_void_p),
                                       cl.ctypes.data_as(C.c_void_p), tabs.ctypes.data_as(C.c_void_p),
                                       out.ctypes.data_as(C.c_void_p), n))
    return out, int(nc.value)


def _lengths_call(fn, q_lens, context_lens, num_heads, num_kv_heads, head_dim, block_size,
                  max_blocks, kv_dtype, num_blocks, ctx) -> int:
    ql = np.ascontiguousarray(np.asarray(q_lens, dtype=np.uint32))
    cl = np.ascontiguousarray(np.asarray(context_lens, dtype=np.uint32))
    p = RaggedAttentionParamsC(ql.size, num_heads, num_kv_heads, head_dim, block_size, max_blocks,
                               1.0, int(ql.sum()), kv_dtype, num_blocks, int(ql.max(initial=0)), 0, 0, 0)
    return int(fn(ctx.handle, C.byref(p), ql.ctypes.data_as(C.c_void_p),
                  cl.ctypes.data_as(C.c_void_p)))


def ragged_partition_size(ctx: Context, *, q_lens, context_lens, num_heads: int,
                          num_kv_heads: int, head_dim: int, block_size: int, max_blocks: int,
                          kv_dtype: int = KANSO_KV_F32, num_blocks: int = 0) -> int:
    """The split-K partition for ragged_paged_attention from the step's host-side
    query / context lengths (kanso_ragged_partition_size); 0 = the library's choice."""
    return _lengths_call(ctx._lib.kanso_ragged_partition_size, q_lens, context_lens, num_heads,
                         num_kv_heads, head_dim, block_size, max_blocks, kv_dtype, num_blocks, ctx)


def ragged_chunk_partition_size(ctx: Context, *, q_lens, context_lens, num_heads: int,
                                num_kv_heads: int, head_dim: int, block_size: int,
                                max_blocks: int, kv_dtype: int = KANSO_KV_F32,
                                num_blocks: int = 0) -> int:
    """The chunk partition (kanso_ragged_chunk_partition_size): non-zero only for
    batches whose sequences all have more than one query row; 0 = automatic."""
    return _lengths_call(ctx._lib.kanso_ragged_chunk_partition_size, q_lens, context_lens,
                         num_heads, num_kv_heads, head_dim, block_size, max_blocks, kv_dtype,
                         num_blocks, ctx)


# ---------------------------------------------------------------- packing


@dataclass
class PackedStep:
    cu_seqlens: torch.Tensor
    seq_of_query: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    tokens: torch.Tensor
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    max_blocks: int
    total_q: int


def plan_shapes(plan: np.ndarray, block_size: int) -> tuple[int, int]:
    """(total_q, max_blocks) of a plan array with fields start_pos, q_len (host side,
    the same arithmetic as PaddedDecodeTables::new, src/model.rs:84-88)."""
    start = plan[:, 0].astype(np.int64)
    qlen = plan[:, 1].astype(np.int64)
    ctx = start + qlen
    max_blocks = int(max(1, ((ctx + block_size - 1) // block_size).max(initial=1)))
    return int(qlen.sum()), max_blocks


def pack_step(ctx: Context, plan: np.ndarray, token_arena: torch.Tensor, table_arena: torch.Tensor,
              block_size: int, stream: torch.cuda.Stream | None = None) -> PackedStep:
    """Packs one step on the device. `plan` is an int array [S, 5] of
    (start_pos, q_len, table_offset, table_len, token_offset) in plan order."""
    plan = np.ascontiguousarray(np.asarray(plan, dtype=np.uint32))
    S = plan.shape[0]
    total_q, max_blocks = plan_shapes(plan, block_size)
    dev = torch.device("cuda", ctx.device)
    plan_d = torch.from_numpy(plan.view(np.int32)).to(dev)
    out = PackedStep(
        cu_seqlens=torch.empty(S + 1, dtype=torch.int32, device=dev),
        seq_of_query=torch.empty(total_q, dtype=torch.int32, device=dev),
        positions=torch.empty(total_q, dtype=torch.int32, device=dev),
        slot_mapping=torch.empty(total_q, dtype=torch.int64, device=dev),
        tokens=torch.empty(total_q, dtype=torch.int32, device=dev),
        block_tables=torch.empty(S * max_blocks, dtype=torch.int32, device=dev),
        context_lens=torch.empty(S, dtype=torch.int32, device=dev),
        max_blocks=max_blocks, total_q=total_q)
    c = PackedStepC(out.cu_seqlens.data_ptr(), out.seq_of_query.data_ptr(),
                    out.positions.data_ptr(), out.slot_mapping.data_ptr(), out.tokens.data_ptr(),
                    out.block_tables.data_ptr(), out.context_lens.data_ptr())
    _check(ctx._lib.kanso_pack_step(ctx.handle, _ptr(plan_d), S, _ptr(token_arena),
                                    _ptr(table_arena), block_size, max_blocks, total_q,
                                    C.byref(c), _stream(stream)))
    out._plan_keepalive = plan_d  # the kernel reads it asynchronously
    return out


# ---------------------------------------------------------------- KV pool


def kv_append(ctx: Context, kv_dtype: int, k: torch.Tensor, v: torch.Tensor,
              slot_mapping: torch.Tensor, num_blocks: int, block_size: int, num_kv_heads: int,
              head_dim: int, k_pool: torch.Tensor, v_pool: torch.Tensor,
              k_scales: torch.Tensor | None = None, v_scales: torch.Tensor | None = None,
              stream: torch.cuda.Stream | None = None) -> None:
    """Fused append (+ quantize) of [T, Hkv, D] K/V rows into pool row slot_mapping[t]."""
    T = slot_mapping.numel()
    _check(ctx._lib.kanso_kv_append(ctx.handle, kv_dtype, _ptr(k), _ptr(v), _ptr(slot_mapping), T,
                                    num_blocks, block_size, num_kv_heads, head_dim, _ptr(k_pool),
                                    _ptr(v_pool), _ptr(k_scales), _ptr(v_scales), _stream(stream)))


def kv_reset_blocks(ctx: Context, kv_dtype: int, blocks: torch.Tensor, num_blocks: int,
                    block_size: int, num_kv_heads: int, head_dim: int, k_pool: torch.Tensor,
                    v_pool: torch.Tensor, k_scales: torch.Tensor | None = None,
                    v_scales: torch.Tensor | None = None,
                    stream: torch.cuda.Stream | None = None) -> None:
    """allocate_zeroed's erase (src/kv_cache/mod.rs:25-35) for a list of blocks."""
    _check(ctx._lib.kanso_kv_reset_blocks(ctx.handle, kv_dtype, _ptr(blocks), blocks.numel(),
                                          num_blocks, block_size, num_kv_heads, head_dim,
                                          _ptr(k_pool), _ptr(v_pool), _ptr(k_scales),
                                          _ptr(v_scales), _stream(stream)))


# ---------------------------------------------------------------- GEMV


def gemv_q8_0(ctx: Context, w: torch.Tensor, x: torch.Tensor, y: torch.Tensor, out_features: int,
              in_features: int, stream: torch.cuda.Stream | None = None) -> None:
    """y[b, out] = W x[b] with W as GGUF block_q8_0 bytes ([out, in/32] x 34 B)."""
    batch = x.numel() // in_features
    _check(ctx._lib.kanso_gemv_q8_0(ctx.handle, _ptr(w), _ptr(x), _ptr(y), out_features,
                                    in_features, batch, _stream(stream)))


def gemv_q4_k(ctx: Context, w: torch.Tensor, x: torch.Tensor, y: torch.Tensor, out_features: int,
              in_features: int, stream: torch.cuda.Stream | None = None) -> None:
    """y[b, out] = W x[b] with W as GGUF block_q4_K bytes ([out, in/256] x 144 B)."""
    batch = x.numel() // in_features
    _check(ctx._lib.kanso_gemv_q4_k(ctx.handle, _ptr(w), _ptr(x), _ptr(y), out_features,
                                    in_features, batch, _stream(stream)))


# ---------------------------------------------------------------- packed Q8_0 / decoder ops


def q8_0_packed_bytes(rows: int, in_features: int) -> int:
    """Bytes of a packed Q8_0 matrix (16-row groups rounded up to pairs)."""
    return int(_capi.load().kanso_q8_0_packed_bytes(rows, in_features))


def q8_0_pack(ctx: Context, gguf: torch.Tensor, rows: int, in_features: int, packed: torch.Tensor,
              group_stride: int = 1, group_offset: int = 0,
              stream: torch.cuda.Stream | None = None) -> None:
    """Re-lays GGUF block_q8_0 bytes into the packed layout (source group g ->
    destination group g * group_stride + group_offset)."""
    _check(ctx._lib.kanso_q8_0_pack(ctx.handle, _ptr(gguf), rows, in_features, _ptr(packed),
                                    group_stride, group_offset, _stream(stream)))


def pack_q8_0_matrix(ctx: Context, gguf: torch.Tensor, rows: int, in_features: int) -> torch.Tensor:
    """A freshly allocated packed copy of one GGUF Q8_0 matrix."""
    packed = torch.zeros(q8_0_packed_bytes(rows, in_features), dtype=torch.uint8,
                         device=gguf.device)
    q8_0_pack(ctx, gguf, rows, in_features, packed)
    return packed


def gemm_q8_0(ctx: Context, packed: torch.Tensor, x: torch.Tensor, y: torch.Tensor,
              out_features: int, in_features: int,
              stream: torch.cuda.Stream | None = None) -> None:
    """y[t, out] = W x[t] over a packed matrix."""
    T = x.numel() // in_features
    _check(ctx._lib.kanso_gemm_q8_0(ctx.handle, _ptr(packed), _ptr(x), _ptr(y), out_features,
                                    in_features, T, _stream(stream)))


def gemm_q8_0_residual(ctx: Context, packed: torch.Tensor, x: torch.Tensor, y: torch.Tensor,
                       out_features: int, in_features: int,
                       stream: torch.cuda.Stream | None = None) -> None:
    """y[t, out] += W x[t] (projection + residual add)."""
    T = x.numel() // in_features
    _check(ctx._lib.kanso_gemm_q8_0_residual(ctx.handle, _ptr(packed), _ptr(x), _ptr(y),
                                             out_features, in_features, T, _stream(stream)))


def embed_q8_0(ctx: Context, packed_table: torch.Tensor, vocab: int, hidden: int,
               tokens: torch.Tensor, out: torch.Tensor,
               stream: torch.cuda.Stream | None = None) -> None:
    """out[t] = dequantized row tokens[t] of a packed Q8_0 embedding table."""
    _check(ctx._lib.kanso_embed_q8_0(ctx.handle, _ptr(packed_table), vocab, hidden, _ptr(tokens),
                                     tokens.numel(), _ptr(out), _stream(stream)))


def qkv_rope_append(ctx: Context, packed_qkv: torch.Tensor, x: torch.Tensor, norm_w: torch.Tensor,
                    positions: torch.Tensor, slot_mapping: torch.Tensor, cos_t: torch.Tensor,
                    sin_t: torch.Tensor, q_out: torch.Tensor, k_pool: torch.Tensor,
                    v_pool: torch.Tensor, *, hidden: int, num_heads: int, num_kv_heads: int,
                    num_blocks: int, block_size: int, eps: float = 1e-5, head_dim: int = 64,
                    stream: torch.cuda.Stream | None = None) -> None:
    """RMSNorm + Q/K/V + RoPE; Q to q_out, K/V into pool row slot_mapping[t]."""
    T = x.numel() // hidden
    p = _capi.QkvParamsC(T, hidden, num_heads, num_kv_heads, head_dim,
                         cos_t.numel() // (head_dim // 2), eps, num_blocks, block_size)
    _check(ctx._lib.kanso_qkv_rope_append(
        ctx.handle, C.byref(p), _ptr(packed_qkv), _ptr(x), _ptr(norm_w), _ptr(positions),
        _ptr(slot_mapping), _ptr(cos_t), _ptr(sin_t), _ptr(q_out), _ptr(k_pool), _ptr(v_pool),
        _stream(stream)))


def qkv_rope_append_quant(ctx: Context, packed_qkv: torch.Tensor, x: torch.Tensor,
                          norm_w: torch.Tensor, positions: torch.Tensor, slot_mapping: torch.Tensor,
                          cos_t: torch.Tensor, sin_t: torch.Tensor, q_out: torch.Tensor,
                          kv_dtype: int, k_pool: torch.Tensor, v_pool: torch.Tensor,
                          k_scales: torch.Tensor, v_scales: torch.Tensor, *, hidden: int,
                          num_heads: int, num_kv_heads: int, num_blocks: int, block_size: int,
                          eps: float = 1e-5, head_dim: int = 64,
                          stream: torch.cuda.Stream | None = None) -> None:
    """qkv_rope_append into a 1-byte pool: K/V rows quantized (with their scales) into
    pool row slot_mapping[t] in the product's epilogue."""
    T = x.numel() // hidden
    p = _capi.QkvParamsC(T, hidden, num_heads, num_kv_heads, head_dim,
                         cos_t.numel() // (head_dim // 2), eps, num_blocks, block_size)
    _check(ctx._lib.kanso_qkv_rope_append_quant(
        ctx.handle, C.byref(p), _ptr(packed_qkv), _ptr(x), _ptr(norm_w), _ptr(positions),
        _ptr(slot_mapping), _ptr(cos_t), _ptr(sin_t), _ptr(q_out), kv_dtype, _ptr(k_pool),
        _ptr(v_pool), _ptr(k_scales), _ptr(v_scales), _stream(stream)))


def gate_up_swiglu(ctx: Context, packed_gate_up: torch.Tensor, x: torch.Tensor,
                   norm_w: torch.Tensor, h: torch.Tensor, *, hidden: int, intermediate: int,
                   eps: float = 1e-5, stream: torch.cuda.Stream | None = None) -> None:
    """h[t] = silu(gate(n)) * up(n) with n = RMSNorm(x[t]) * norm_w."""
    T = x.numel() // hidden
    _check(ctx._lib.kanso_gate_up_swiglu(ctx.handle, _ptr(packed_gate_up), _ptr(x), _ptr(norm_w),
                                         eps, T, hidden, intermediate, _ptr(h), _stream(stream)))


def lm_head_argmax(ctx: Context, packed: torch.Tensor, x: torch.Tensor, tokens: torch.Tensor, *,
                   hidden: int, vocab: int, rows: torch.Tensor | None = None,
                   norm_w: torch.Tensor | None = None, eps: float = 1e-5,
                   logits: torch.Tensor | None = None,
                   stream: torch.cuda.Stream | None = None) -> None:
    """tokens[i] = greedy argmax of lm_head(RMSNorm(x[rows[i]]))."""
    n = tokens.numel()
    _check(ctx._lib.kanso_lm_head_argmax(ctx.handle, _ptr(packed), _ptr(x), _ptr(rows),
                                         _ptr(norm_w), eps, n, hidden, vocab, _ptr(logits),
                                         _ptr(tokens), _stream(stream)))
