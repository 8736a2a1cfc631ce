"""Helpers shared by the GPU parity tests: upload host arrays, run the HIP path
through the C ABI, and compare with the oracle at the tolerance the path states."""
from __future__ import annotations

import numpy as np
import torch

import kanso_infer_amd as K
import oracle

# Attention / GEMV outputs: max-abs 2e-3 / rel 1e-3 in f32 accumulation.
ATOL, RTOL = 2e-3, 1e-3


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint8:
        a = a.view(np.uint8)
    return torch.from_numpy(a).to("cuda:0")


def host(t: torch.Tensor, dtype=None) -> np.ndarray:
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def assert_close(got: np.ndarray, want: np.ndarray, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside atol {atol} rtol {rtol}; "
                           f"max abs err {err.max():.3g}")


def fill_pool(batch, kv_dtype: int, seed: int):
    """Random N(0,1) K/V for every row of the pool, quantized by the oracle for
    INT8 / Q8_0. Returns host arrays (k_pool, v_pool, k_scales, v_scales)."""
    rng = np.random.default_rng(seed)
    rows = batch.num_blocks * batch.block_size
    width = batch.num_kv_heads * batch.head_dim
    k = rng.standard_normal((rows, width), dtype=np.float32)
    v = rng.standard_normal((rows, width), dtype=np.float32)
    if kv_dtype == oracle.KV_F32:
        return k.ravel(), v.ravel(), None, None
    kp, vp, ks, vs = oracle.kv_pool_arrays(kv_dtype, batch.num_blocks, batch.block_size,
                                           batch.num_kv_heads, batch.head_dim)
    oracle.kv_append(kv_dtype, k, v, np.arange(rows), batch.num_blocks, batch.block_size,
                     batch.num_kv_heads, batch.head_dim, kp, vp, ks, vs)
    return kp, vp, ks, vs


def run_ragged_gpu(ctx, batch, q, kp, vp, ks=None, vs=None, kv_dtype=0, partition_size=0,
                   chunk_partition_size=0, cu_seqlens=True):
    out = torch.empty(batch.total_q * batch.num_heads * batch.head_dim, dtype=torch.float32,
                      device="cuda:0")
    K.ragged_paged_attention(
        ctx, q=dev(q), k_pool=dev(kp), v_pool=dev(vp),
        k_scales=None if ks is None else dev(ks), v_scales=None if vs is None else dev(vs),
        block_tables=dev(batch.block_tables.ravel()), cu_seqlens=dev(batch.cu_seqlens) if cu_seqlens else None,
        context_lens=dev(batch.context_lens.astype(np.uint32)), out=out,
        num_heads=batch.num_heads, num_kv_heads=batch.num_kv_heads, head_dim=batch.head_dim,
        block_size=batch.block_size, scale=batch.scale, kv_dtype=kv_dtype,
        num_blocks=batch.num_blocks, max_q_len=int(batch.q_lens.max()),
        partition_size=partition_size, chunk_partition_size=chunk_partition_size)
    ctx.check_device_status()
    return host(out)


def run_ragged_oracle(batch, q, kp, vp, ks=None, vs=None, kv_dtype=0, nthreads=8):
    return oracle.ragged_attention(q, kp, vp, batch.block_tables, batch.cu_seqlens,
                                   batch.context_lens, num_heads=batch.num_heads,
                                   num_kv_heads=batch.num_kv_heads, head_dim=batch.head_dim,
                                   block_size=batch.block_size, scale=batch.scale,
                                   kv_dtype=kv_dtype, k_scales=ks, v_scales=vs,
                                   num_blocks=batch.num_blocks, nthreads=nthreads)
