"""kanso_ragged_paged_attention_noalloc (the entry point that allocates nothing: its
split-K scratch is a fixed device array) against kanso_ragged_paged_attention, the
allocating entry point with the same kernels: outputs equal bit for bit on two
calls in a row, the second with a smaller batch, and a call beyond the fixed
scratch rejected. Both are called through the C ABI (ctypes)."""
import ctypes as C

import numpy as np
import pytest
import torch

import kanso_infer_amd as K
from kanso_infer_amd import workloads
from kanso_infer_amd._capi import RaggedAttentionParamsC
from kanso_infer_amd import _capi

pytestmark = pytest.mark.gpu


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _call(ctx, fn, b, q, k, v, tables, cu, lens, out, partition=0):
    p = RaggedAttentionParamsC(b.num_seqs, b.num_heads, b.num_kv_heads, b.head_dim, b.block_size,
                               b.max_blocks, b.scale, b.total_q, K.KANSO_KV_F32, b.num_blocks,
                               int(b.q_lens.max()), 0, partition, 0)
    return fn(ctx.handle, C.byref(p), _ptr(q), _ptr(k), _ptr(v), None, None, _ptr(tables), _ptr(cu),
              _ptr(lens), _ptr(out), None)


def _batch(b, seed):
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rows = b.num_blocks * b.block_size * b.num_kv_heads * b.head_dim
    k = torch.randn(rows, generator=g, device=dev)
    v = torch.randn(rows, generator=g, device=dev)
    q = torch.randn(b.total_q * b.num_heads * b.head_dim, generator=g, device=dev)
    tables = torch.from_numpy(b.block_tables.ravel().view(np.int32)).to(dev)
    cu = torch.from_numpy(b.cu_seqlens).to(dev)
    lens = torch.from_numpy(b.context_lens.astype(np.int32)).to(dev)
    return q, k, v, tables, cu, lens


def test_noalloc_equals_allocating_entry(ctx):
    lib = _capi.load()
    # a mixed batch (prefill chunks on the matrix cores + decode rows), then a smaller
    # decode-only one: the second call reuses the scratch the first one left behind
    for b, seed in ((workloads.config2_mixed(num_blocks=10000, seed_offset=5), 1),
                    (workloads.small_mixed(3, num_chunks=0), 2)):
        q, k, v, tables, cu, lens = _batch(b, seed)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        assert _call(ctx, lib.kanso_ragged_paged_attention, b, q, k, v, tables, cu, lens, want) == 0
        torch.cuda.synchronize()
        assert _call(ctx, lib.kanso_ragged_paged_attention_noalloc, b, q, k, v, tables, cu, lens, got) == 0
        torch.cuda.synchronize()
        ctx.check_device_status()
        assert torch.equal(got, want), b.label


def test_noalloc_rejects_beyond_fixed_scratch(ctx):
    lib = _capi.load()
    # 512 rows x 15 heads x 128 partitions of 32 keys x 264 B = 259 MB > 64 MiB
    b = workloads.config2_mixed(num_blocks=10000, seed_offset=6)
    q, k, v, tables, cu, lens = _batch(b, 3)
    out = torch.empty_like(q)
    rc = _call(ctx, lib.kanso_ragged_paged_attention_noalloc, b, q, k, v, tables, cu, lens, out, partition=32)
    assert rc == _capi.KANSO_E_INVALID_SHAPE
    assert b"fixed" in lib.kanso_last_error()
