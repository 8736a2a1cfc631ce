"""The C-ABI library loads and exports every symbol include/kanso_hip.h declares
(no compute calls: this runs without a GPU)."""
import re

import numpy as np
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kanso_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kanso_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("kanso_paged_attention_v2", "kanso_ragged_paged_attention",
                     "kanso_pack_step", "kanso_kv_append", "kanso_gemv_q8_0", "kanso_gemv_q4_k"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from kanso_infer_amd import _capi
    if not _capi.LIB_PATH.exists():
        pytest.fail("libkanso_hip.so is not built (python -m kanso_infer_amd.build)")
    lib = _capi.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _capi.SIGNATURES, f"{name} has no ctypes signature"


def test_no_fallback_when_library_missing(monkeypatch, tmp_path):
    from kanso_infer_amd import _capi
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setenv("KANSO_HIP_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError):
        _capi.load()


def test_work_list_layout():
    """kanso_ragged_build_work on the host: one 64-word item per (row, partition) of
    every row outside the matrix-core chunk path, block ids first (the partition's
    table slice), then row, first key, end key and the row's key count; a row
    without keys or an FP8 pool gives no list."""
    import kanso_infer_amd as K
    q_lens = np.array([1, 1, 1], np.uint32)
    ctx = np.array([40, 100, 1], np.uint32)
    bs, P = 16, 32
    tables = np.arange(3 * 8, dtype=np.uint32).reshape(3, 8) + 1000
    geo = dict(num_heads=15, num_kv_heads=5, head_dim=64, block_size=bs, partition_size=P,
               num_blocks=4096)
    w, n_chunk = K.ragged_work(q_lens=q_lens, context_lens=ctx, block_tables=tables, **geo)
    assert n_chunk == 0
    items = w.reshape(-1, 64)
    want = []
    for s, c in enumerate(ctx):
        for t0 in range(0, int(c), P):
            t1 = min(t0 + P, int(c))
            blocks = list(tables[s, t0 // bs:(t1 - 1) // bs + 1])
            want.append((blocks, s, t0, t1, int(c)))
    assert items.shape[0] == len(want) == 2 + 4 + 1
    for it, (blocks, row, t0, t1, lim) in zip(items, want):
        assert list(it[:len(blocks)]) == blocks and not it[len(blocks):60].any()
        assert list(it[60:]) == [row, t0, t1, lim]
    assert K.ragged_work(q_lens=q_lens, context_lens=np.array([40, 0, 1], np.uint32),
                         block_tables=tables, **geo) is None
    assert K.ragged_work(q_lens=q_lens, context_lens=ctx, block_tables=tables, kv_dtype=K.KANSO_KV_FP8,
                         **geo) is None


def test_work_list_chunk_items():
    """A mixed batch: decode items first, then one chunk item per (64-row block,
    chunk partition) of the multi-row sequence: block ids of the partition, then
    first row, rows, key position of the first row, partition."""
    import kanso_infer_amd as K
    q_lens = np.array([1, 100, 1], np.uint32)   # a 100-row chunk between two decodes
    ctx = np.array([50, 700, 20], np.uint32)     # the chunk's rows sit at keys 600 .. 699
    bs, P, CP = 16, 32, 512
    tables = np.arange(3 * 48, dtype=np.uint32).reshape(3, 48) + 7
    w, n_chunk = K.ragged_work(q_lens=q_lens, context_lens=ctx, block_tables=tables, num_heads=15,
                               num_kv_heads=5, head_dim=64, block_size=bs, partition_size=P,
                               num_blocks=4096, max_q_len=100, chunk_partition_size=CP)
    items = w.reshape(-1, 64)
    n_dec = 2 + 1  # rows of 50 and 20 keys at 32-key partitions
    assert items.shape[0] == n_dec + n_chunk
    assert [list(it[60:]) for it in items[:n_dec]] == [[0, 0, 32, 50], [0, 32, 50, 50], [101, 0, 20, 20]]
    # chunk blocks: rows 0-63 (keys up to 600 + 63 + 1 = 664: partitions 0, 1) and rows 64-99
    # (keys up to 700: partitions 0, 1)
    want = [(1, 64, 600, 0), (65, 36, 664, 0), (1, 64, 600, 1), (65, 36, 664, 1)]  # partition-major
    assert [tuple(int(x) for x in it[60:]) for it in items[n_dec:]] == want
    first = items[n_dec]
    assert list(first[:32]) == list(tables[1, :32]) and not first[32:60].any()
    second = items[n_dec + 2]  # rows 0-63, keys 512 .. 663: blocks 32 .. 41
    assert list(second[:10]) == list(tables[1, 32:42]) and not second[10:60].any()
