"""Inputs of the deterministic-pattern cases in the reference's
tests/test_paged_attention_v2.rs (the reference compares its GPU kernel with
cpu_paged_attention at 1e-4 and stores no outputs). The outputs this build
computed for them with the oracle are frozen in tests/golden/paged_attention_v2_cases.npz
(written by tests/golden/make_golden.py)."""
from pathlib import Path

import numpy as np

GOLDEN_PATH = Path(__file__).resolve().parent / "golden" / "paged_attention_v2_cases.npz"


def _pattern(n, mod, center, step):
    i = np.arange(n)
    return (((i % mod).astype(np.float32) - np.float32(center)) * np.float32(step)).astype(np.float32)


def _case(num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_blocks, num_blocks,
          q_pat, k_pat, v_pat, tables, lens, scale=None):
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    total_kv = num_blocks * block_size * num_kv_heads * head_dim
    return dict(num_seqs=num_seqs, num_heads=num_heads, num_kv_heads=num_kv_heads,
                head_dim=head_dim, block_size=block_size, max_blocks=max_blocks,
                q=_pattern(num_seqs * num_heads * head_dim, *q_pat),
                k=_pattern(total_kv, *k_pat), v=_pattern(total_kv, *v_pat),
                tables=np.asarray(tables, np.uint32), lens=np.asarray(lens, np.uint32),
                scale=scale)


def contiguous_heads():  # :89-164
    return _case(1, 4, 4, 64, 16, 4, 8, (17, 8, 0.125), (19, 9, 0.1), (23, 11, 0.15),
                 [5, 2, 7, 0], [35])


def gqa_8_2():  # :166-240
    return _case(1, 8, 2, 32, 8, 4, 6, (13, 6, 0.1), (29, 14, 0.05), (31, 15, 0.05),
                 [3, 1, 4, 0], [20])


def multi_seq():  # :242-321 (tables padded with 0, as in the reference test)
    return _case(3, 4, 2, 32, 16, 4, 12, (11, 5, 0.1), (7, 3, 0.2), (13, 6, 0.1),
                 [1, 5, 0, 0, 0, 8, 2, 0, 10, 0, 0, 0], [25, 40, 8])


def multi_partition():  # :484-556, table (7b + 3) % 44, ctx 600 over 3 partitions
    return _case(1, 8, 2, 128, 16, 40, 44, (17, 8, 0.125), (19, 9, 0.1), (23, 11, 0.15),
                 [(7 * b + 3) % 44 for b in range(40)], [600])


def matrix(head_dim, group):  # :323-401
    return lambda: _case(2, 2 * group, 2, head_dim, 16, 4, 10, (17, 8, 0.125), (19, 9, 0.1),
                         (23, 11, 0.15), [5, 2, 7, 0, 3, 9, 1, 6], [37, 16])


REFERENCE_CASES = {
    "contiguous_heads": contiguous_heads,
    "gqa_8_2": gqa_8_2,
    "multi_seq": multi_seq,
    "multi_partition": multi_partition,
}
for _hd in (64, 128, 256):
    for _g in (1, 4, 5, 8):
        REFERENCE_CASES[f"matrix_hd{_hd}_g{_g}"] = matrix(_hd, _g)
