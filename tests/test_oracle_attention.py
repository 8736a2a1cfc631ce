"""Pins the oracle's attention (cpu_paged_attention restatement and the ragged
mixed-batch restatement) against the reference's known-answer test, an independent
float64 formulation, closed-form invariants and the committed golden fixtures."""
import numpy as np
import pytest

import oracle
from kanso_infer_amd import workloads
from refmath import attention_f64
from golden_cases import REFERENCE_CASES, GOLDEN_PATH


def run_paged(case):
    return oracle.paged_attention(case["q"], case["k"], case["v"], case["tables"], case["lens"],
                                  case["num_seqs"], case["num_heads"], case["num_kv_heads"],
                                  case["head_dim"], case["block_size"], case["max_blocks"],
                                  case["scale"])


def test_known_answer_hand_computed():
    # tests/test_paged_attention_v2.rs:10-87: q=[1,0,1,0], 3 tokens over physical
    # blocks [2, 1], block size 2 -> out = [2.7407, 5.4814, 13.5558, 0].
    bs, hd = 2, 4
    k = np.zeros(4 * bs * hd, np.float32)
    v = np.zeros_like(k)
    t0 = (2 * bs) * hd
    k[t0] = 1.0
    v[t0] = 10.0
    t1 = (2 * bs + 1) * hd
    k[t1 + 2] = 1.0
    v[t1 + 1] = 20.0
    t2 = bs * hd
    k[t2] = 1.0
    k[t2 + 2] = 1.0
    v[t2 + 2] = 30.0
    out = oracle.paged_attention([1, 0, 1, 0], k, v, [2, 1], [3], 1, 1, 1, hd, bs, 2, 0.5)
    assert abs(out[0] - 2.7407) < 1e-3
    assert abs(out[1] - 5.4814) < 1e-3
    assert abs(out[2] - 13.5558) < 1e-3
    assert out[3] == 0.0


@pytest.mark.parametrize("name", sorted(REFERENCE_CASES))
def test_reference_patterns_match_float64(name):
    """The deterministic-pattern inputs of tests/test_paged_attention_v2.rs against the
    float64 formulation (no outputs are stored in the reference for these)."""
    case = REFERENCE_CASES[name]()
    out = run_paged(case)
    S = case["num_seqs"]
    cu = np.arange(S + 1)
    ref = attention_f64(case["q"], case["k"], case["v"], case["tables"], cu, case["lens"],
                        case["num_heads"], case["num_kv_heads"], case["head_dim"],
                        case["block_size"], case["scale"])
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("name", sorted(REFERENCE_CASES))
def test_golden_fixture(name):
    """Regression: the oracle still produces the committed fixture bit for bit."""
    golden = np.load(GOLDEN_PATH)
    out = run_paged(REFERENCE_CASES[name]())
    np.testing.assert_array_equal(out, golden[name])


def test_constant_v_and_single_token():
    rng = np.random.default_rng(1)
    H, HKV, D, BS, MB = 6, 2, 32, 4, 5
    nb = 12
    k = rng.standard_normal(nb * BS * HKV * D).astype(np.float32)
    v = np.tile(np.arange(D, dtype=np.float32), nb * BS * HKV)  # every row = 0..D-1
    q = rng.standard_normal(2 * H * D).astype(np.float32)
    tables = np.array([3, 7, 1, 0, 9, 2, 2, 2, 2, 2], np.uint32)
    out = oracle.paged_attention(q, k, v, tables, [17, 1], 2, H, HKV, D, BS, MB, 0.3)
    np.testing.assert_allclose(out.reshape(2, H, D), np.broadcast_to(np.arange(D), (2, H, D)),
                               rtol=1e-5, atol=1e-5)
    # ctx = 1 -> out is V of token 0 exactly
    v2 = rng.standard_normal(v.size).astype(np.float32)
    out = oracle.paged_attention(q, k, v2, tables, [1, 1], 2, H, HKV, D, BS, MB, 0.3)
    v4 = v2.reshape(nb, BS, HKV, D)
    for h in range(H):
        np.testing.assert_array_equal(out.reshape(2, H, D)[0, h], v4[3, 0, h // (H // HKV)])


def test_block_permutation_invariance():
    """Moving physical blocks and rewriting the table leaves the output unchanged."""
    rng = np.random.default_rng(2)
    H, HKV, D, BS = 4, 2, 16, 8
    nb, ctx = 10, 37
    k = rng.standard_normal((nb, BS, HKV, D)).astype(np.float32)
    v = rng.standard_normal((nb, BS, HKV, D)).astype(np.float32)
    q = rng.standard_normal(H * D).astype(np.float32)
    table = np.array([4, 1, 8, 6, 0], np.uint32)
    out = oracle.paged_attention(q, k, v, table, [ctx], 1, H, HKV, D, BS, 5, 0.25)
    perm = rng.permutation(nb)
    k2, v2 = np.empty_like(k), np.empty_like(v)
    k2[perm] = k
    v2[perm] = v
    out2 = oracle.paged_attention(q, k2, v2, perm[table].astype(np.uint32), [ctx], 1, H, HKV, D,
                                  BS, 5, 0.25)
    np.testing.assert_array_equal(out, out2)


def test_ragged_chunk_equals_rowwise_decode():
    """A prefill chunk of q_len rows == q_len decode calls with context start+i+1
    (the offset causal mask, src/model.rs:1510-1527)."""
    b = workloads.small_mixed(3, num_decodes=2, num_chunks=2, head_dim=32, num_heads=8,
                              num_kv_heads=2)
    rng = np.random.default_rng(3)
    pool_elems = b.num_blocks * b.block_size * b.num_kv_heads * b.head_dim
    k = rng.standard_normal(pool_elems).astype(np.float32)
    v = rng.standard_normal(pool_elems).astype(np.float32)
    q = rng.standard_normal(b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    out = oracle.ragged_attention(q, k, v, b.block_tables, b.cu_seqlens, b.context_lens,
                                  num_heads=b.num_heads, num_kv_heads=b.num_kv_heads,
                                  head_dim=b.head_dim, block_size=b.block_size, scale=b.scale,
                                  num_blocks=b.num_blocks)
    cu = b.cu_seqlens
    row_elems = b.num_heads * b.head_dim
    for s in range(b.num_seqs):
        ql, c = int(b.q_lens[s]), int(b.context_lens[s])
        for i in range(ql):
            row = int(cu[s]) + i
            dec = oracle.paged_attention(q[row * row_elems:(row + 1) * row_elems], k, v,
                                         b.block_tables[s], [c - ql + i + 1], 1, b.num_heads,
                                         b.num_kv_heads, b.head_dim, b.block_size, b.max_blocks,
                                         b.scale)
            np.testing.assert_array_equal(out[row * row_elems:(row + 1) * row_elems], dec)


def test_ragged_matches_float64_and_threads_do_not_matter():
    b = workloads.small_mixed(4)
    rng = np.random.default_rng(4)
    pool_elems = b.num_blocks * b.block_size * b.num_kv_heads * b.head_dim
    k = rng.standard_normal(pool_elems).astype(np.float32)
    v = rng.standard_normal(pool_elems).astype(np.float32)
    q = rng.standard_normal(b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    kw = dict(num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
              block_size=b.block_size, scale=b.scale, num_blocks=b.num_blocks)
    out1 = oracle.ragged_attention(q, k, v, b.block_tables, b.cu_seqlens, b.context_lens, **kw)
    out4 = oracle.ragged_attention(q, k, v, b.block_tables, b.cu_seqlens, b.context_lens,
                                   nthreads=4, **kw)
    np.testing.assert_array_equal(out1, out4)
    ref = attention_f64(q, k, v, b.block_tables, b.cu_seqlens, b.context_lens, b.num_heads,
                        b.num_kv_heads, b.head_dim, b.block_size, b.scale)
    np.testing.assert_allclose(out1, ref, rtol=1e-5, atol=1e-5)


def test_quantized_pool_equals_f32_pool_of_dequantized_values():
    """Attention over an INT8 / Q8_0 pool equals attention over the F32 pool holding
    the dequantized values (dequantization is the only difference)."""
    b = workloads.small_mixed(5, head_dim=64, num_heads=16, num_kv_heads=4)
    rng = np.random.default_rng(5)
    rows = b.num_blocks * b.block_size
    k = rng.standard_normal((rows, b.num_kv_heads * b.head_dim)).astype(np.float32)
    v = rng.standard_normal((rows, b.num_kv_heads * b.head_dim)).astype(np.float32)
    q = rng.standard_normal(b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    kw = dict(num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
              block_size=b.block_size, scale=b.scale, num_blocks=b.num_blocks)
    for kv in (oracle.KV_INT8, oracle.KV_Q8_0):
        kp, vp, ks, vs = oracle.kv_pool_arrays(kv, b.num_blocks, b.block_size, b.num_kv_heads,
                                               b.head_dim)
        oracle.kv_append(kv, k, v, np.arange(rows), b.num_blocks, b.block_size, b.num_kv_heads,
                         b.head_dim, kp, vp, ks, vs)
        # dequantize by hand
        if kv == oracle.KV_INT8:
            kd = (kp.astype(np.float32).reshape(-1, b.head_dim) * ks[:, None]).ravel()
            vd = (vp.astype(np.float32).reshape(-1, b.head_dim) * vs[:, None]).ravel()
        else:
            kd = (kp.astype(np.float32).reshape(-1, 32) *
                  ks.view(np.float16).astype(np.float32)[:, None]).ravel()
            vd = (vp.astype(np.float32).reshape(-1, 32) *
                  vs.view(np.float16).astype(np.float32)[:, None]).ravel()
        outq = oracle.ragged_attention(q, kp, vp, b.block_tables, b.cu_seqlens, b.context_lens,
                                       kv_dtype=kv, k_scales=ks, v_scales=vs, **kw)
        outf = oracle.ragged_attention(q, kd, vd, b.block_tables, b.cu_seqlens, b.context_lens,
                                       **kw)
        np.testing.assert_array_equal(outq, outf)


def test_rejects_empty_and_overlong():
    b = workloads.small_mixed(6)
    q = np.zeros(b.total_q * b.num_heads * b.head_dim, np.float32)
    pool = np.zeros(b.num_blocks * b.block_size * b.num_kv_heads * b.head_dim, np.float32)
    kw = dict(num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
              block_size=b.block_size, scale=b.scale, num_blocks=b.num_blocks)
    lens = b.context_lens.copy()
    lens[0] = 0
    with pytest.raises(ValueError):
        oracle.ragged_attention(q, pool, pool, b.block_tables, b.cu_seqlens, lens, **kw)
    lens = b.context_lens.copy()
    lens[-1] = 1  # fewer keys than the chunk's query rows
    with pytest.raises(ValueError):
        oracle.ragged_attention(q, pool, pool, b.block_tables, b.cu_seqlens, lens, **kw)
