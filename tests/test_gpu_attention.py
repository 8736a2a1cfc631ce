"""GPU parity of the ragged paged-attention kernels against the oracle (through the
C ABI), covering the reference's own GPU test matrix (tests/test_paged_attention_v2.rs)
and the ragged mixed batches of this path."""
import numpy as np
import pytest
import torch

import kanso_infer_amd as K
import oracle
from golden_cases import GOLDEN_PATH, REFERENCE_CASES
from gpu_helpers import (assert_close, dev, fill_pool, host, run_ragged_gpu,
                         run_ragged_oracle)
from kanso_infer_amd import workloads

pytestmark = pytest.mark.gpu


def params_of(c):
    return K.PagedAttentionParams(c["num_seqs"], c["num_heads"], c["num_kv_heads"],
                                  c["head_dim"], c["block_size"], c["max_blocks"], c["scale"])


def test_known_answer(ctx):
    bs, hd = 2, 4
    k = np.zeros(4 * bs * hd, np.float32)
    v = np.zeros_like(k)
    k[2 * bs * hd] = 1.0
    v[2 * bs * hd] = 10.0
    k[(2 * bs + 1) * hd + 2] = 1.0
    v[(2 * bs + 1) * hd + 1] = 20.0
    k[bs * hd] = 1.0
    k[bs * hd + 2] = 1.0
    v[bs * hd + 2] = 30.0
    p = K.PagedAttentionParams(1, 1, 1, hd, bs, 2, 0.5)
    out = K.gpu_paged_attention_v2(ctx, [1, 0, 1, 0], k, v, [2, 1], [3], p)
    assert abs(out[0] - 2.7407) < 1e-3
    assert abs(out[1] - 5.4814) < 1e-3
    assert abs(out[2] - 13.5558) < 1e-3
    assert abs(out[3]) < 1e-6


@pytest.mark.parametrize("name", sorted(REFERENCE_CASES))
def test_reference_matrix(ctx, name):
    c = REFERENCE_CASES[name]()
    out = K.gpu_paged_attention_v2(ctx, c["q"], c["k"], c["v"], c["tables"], c["lens"],
                                   params_of(c))
    golden = np.load(GOLDEN_PATH)[name]
    assert_close(out, golden, what=name)
    # the reference's own GPU-vs-CPU tolerance holds as well
    assert np.abs(out - golden).max() <= 1e-4, name


def test_flat_output_long_context(ctx):
    # tests/test_paged_attention_v2.rs:558-633: ctx 2048, out stays [seqs, heads, hd]
    hd, bs, ctx_len = 64, 16, 2048
    blocks = ctx_len // bs
    p = K.PagedAttentionParams(1, 4, 4, hd, bs, blocks, 1.0 / 8.0)
    nb = blocks + 4
    q = np.full(4 * hd, 0.1, np.float32)
    k = np.full(nb * bs * 4 * hd, 0.05, np.float32)
    v = np.full(nb * bs * 4 * hd, 0.02, np.float32)
    out = K.gpu_paged_attention_v2(ctx, q, k, v, np.arange(blocks), [ctx_len], p)
    assert out.shape == (4 * hd,)
    assert np.isfinite(out).all() and (out > 0).all()
    np.testing.assert_allclose(out, 0.02, rtol=1e-5)


def test_rejects_unrepresentable(ctx):
    p = K.PagedAttentionParams(1, 1, 1, 384, 16, 4, 1.0 / np.sqrt(384))
    with pytest.raises(K.EngineError):
        K.gpu_paged_attention_v2(ctx, np.full(384, 0.1), np.full(4 * 16 * 384, 0.1),
                                 np.full(4 * 16 * 384, 0.1), [0, 1, 2, 3], [8], p)
    p = K.PagedAttentionParams(1, 1, 1, 4, 2, 2, 0.5)
    with pytest.raises(K.EngineError):  # empty context
        K.gpu_paged_attention_v2(ctx, np.ones(4), np.zeros(16), np.zeros(16), [0, 1], [0], p)
    with pytest.raises(K.EngineError):  # context beyond table capacity
        K.gpu_paged_attention_v2(ctx, np.ones(4), np.zeros(16), np.zeros(16), [0, 1], [5], p)
    p = K.PagedAttentionParams(1, 9, 1, 64, 16, 4, 0.125)
    with pytest.raises(K.EngineError):  # GQA group above 8
        K.validate_paged_attention_params(p)


def test_device_flags_raise(ctx):
    """A context length the table cannot address is flagged on the device and raised."""
    hd, bs = 64, 16
    q = torch.zeros(2 * 4 * hd, device="cuda:0")
    pool = torch.zeros(8 * bs * 4 * hd, device="cuda:0")
    tables = dev(np.zeros(2 * 2, np.uint32))
    lens = dev(np.array([10, 40], np.uint32))  # 40 > capacity 32
    out = torch.empty_like(q)
    K.paged_attention_v2(ctx, K.PagedAttentionParams(2, 4, 4, hd, bs, 2, 0.125), q, pool, pool,
                         tables, lens, out)
    with pytest.raises(K.EngineError):
        ctx.check_device_status()
    ctx.check_device_status()  # cleared


def test_rows_without_keys_are_zero_in_mixed_batches(ctx):
    """A query row with no key (more query rows than context) is flagged and written as
    zeros (cpu_paged_attention's empty-context output), also when the batch has
    matrix-core chunk items, whose workgroups come first in the grid."""
    H, HKV, D, bs = 15, 5, 64, 16
    q_lens = np.array([20, 1, 3])
    ctx_lens = np.array([100, 50, 2])
    tables = np.array([[0, 1, 2, 3, 4, 5, 6], [7, 8, 9, 9, 9, 9, 9], [10, 10, 10, 10, 10, 10, 10]],
                      np.uint32)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    T = int(q_lens.sum())
    rng = np.random.default_rng(70)
    pool = dev(rng.standard_normal(16 * bs * HKV * D).astype(np.float32))
    q = dev(rng.standard_normal(T * H * D).astype(np.float32))
    out = torch.full((T * H * D,), float("nan"), device="cuda:0")
    K.ragged_paged_attention(ctx, q=q, k_pool=pool, v_pool=pool, block_tables=dev(tables.ravel()),
                             cu_seqlens=dev(cu), context_lens=dev(ctx_lens.astype(np.uint32)),
                             out=out, num_heads=H, num_kv_heads=HKV, head_dim=D, block_size=bs,
                             scale=0.125, num_blocks=16, max_q_len=20)
    with pytest.raises(K.EngineError):
        ctx.check_device_status()
    got = host(out).reshape(T, H * D)
    np.testing.assert_array_equal(got[21], np.zeros(H * D, np.float32))  # no key
    assert np.isfinite(got[:21]).all() and np.isfinite(got[22:]).all()


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_INT8, oracle.KV_Q8_0, oracle.KV_FP8])
def test_ragged_small(ctx, seed, kv_dtype):
    shapes = [dict(), dict(num_heads=16, num_kv_heads=4), dict(num_heads=8, num_kv_heads=1,
                                                              head_dim=128),
              dict(num_heads=4, num_kv_heads=4, head_dim=32, block_size=8)]
    b = workloads.small_mixed(seed, **shapes[seed])
    kp, vp, ks, vs = fill_pool(b, kv_dtype, seed)
    q = np.random.default_rng(seed + 50).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, ks, vs, kv_dtype)
    want = run_ragged_oracle(b, q, kp, vp, ks, vs, kv_dtype)
    assert_close(got, want, what=f"{b.label} kv {kv_dtype}")


@pytest.mark.parametrize("partition", [32, 64, 128, 512])
@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q8_0, oracle.KV_FP8])
def test_explicit_partition_size(ctx, partition, kv_dtype):
    """A caller-chosen split-K partition gives the oracle's result (decode and chunk rows)."""
    b = workloads.small_mixed(11)
    kp, vp, ks, vs = fill_pool(b, kv_dtype, 11)
    q = np.random.default_rng(61).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, ks, vs, kv_dtype, partition_size=partition)
    want = run_ragged_oracle(b, q, kp, vp, ks, vs, kv_dtype)
    assert_close(got, want, what=f"{b.label} P {partition} kv {kv_dtype}")


@pytest.mark.parametrize("chunks", [0, 4])
def test_max_sequences_per_call(ctx, chunks):
    """2048 sequences in one call (the LDS-resident per-call limit), all-decode and
    mixed with matrix-core chunks, against the oracle; 2049 is rejected."""
    rng = np.random.default_rng(90 + chunks)
    S = 2048
    q_lens = np.ones(S, np.int64)
    q_lens[:chunks] = rng.integers(3, 20, chunks)
    ctx_lens = rng.integers(1, 40, S).astype(np.int64) + np.where(q_lens > 1, q_lens, 0)
    nb = int(((ctx_lens + 15) // 16).sum()) + 8
    tables = workloads._scatter_tables(rng, ctx_lens, 16, nb)
    b = workloads.AttnBatch(q_lens, ctx_lens, tables, nb, label=f"S2048 chunks {chunks}",
                            **workloads.SMOLLM2)
    kp, vp, ks, vs = fill_pool(b, oracle.KV_F32, 91)
    q = rng.standard_normal(b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp)
    want = run_ragged_oracle(b, q, kp, vp)
    assert_close(got, want, what=b.label)
    over = workloads.AttnBatch(np.ones(S + 1, np.int64), np.ones(S + 1, np.int64),
                               np.zeros((S + 1, 1), np.uint32), 1, **workloads.SMOLLM2)
    with pytest.raises(K.EngineError):
        run_ragged_gpu(ctx, over, np.zeros(over.total_q * 15 * 64, np.float32),
                       np.zeros(16 * 5 * 64, np.float32), np.zeros(16 * 5 * 64, np.float32))


@pytest.mark.parametrize("bs", [1, 4, 32])
def test_block_size_extremes_with_longest_partition(ctx, bs):
    """Block sizes 1, 4 and 32 with the longest legal partitions (62 table entries,
    at most 992 keys) for decode and chunk rows, against the oracle."""
    b = workloads.small_mixed(20 + bs, block_size=bs, max_ctx=1500, chunk_max=70)
    kp, vp, ks, vs = fill_pool(b, oracle.KV_F32, 20 + bs)
    q = np.random.default_rng(63).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    longest = max(32, min(992, 62 * bs // 32 * 32))
    got = run_ragged_gpu(ctx, b, q, kp, vp, partition_size=longest, chunk_partition_size=longest)
    want = run_ragged_oracle(b, q, kp, vp)
    assert_close(got, want, what=f"{b.label} bs {bs} P {longest}")


def test_rejects_bad_partition_size(ctx):
    b = workloads.small_mixed(12)
    kp, vp, ks, vs = fill_pool(b, oracle.KV_F32, 12)
    q = np.zeros(b.total_q * b.num_heads * b.head_dim, np.float32)
    for bad in (48, 16, 1024, 100):
        with pytest.raises(K.EngineError):
            run_ragged_gpu(ctx, b, q, kp, vp, partition_size=bad)


@pytest.mark.parametrize("cp", [32, 64, 96, 160])
@pytest.mark.parametrize("P", [0, 64])
@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q8_0])
@pytest.mark.parametrize("decodes", [5, 0])
def test_explicit_chunk_partition_size(ctx, cp, P, kv_dtype, decodes):
    """A caller-chosen chunk partition (shorter or longer than the decode one) gives
    the oracle's result, with and without decode rows in the batch."""
    b = workloads.small_mixed(16, num_decodes=decodes, num_chunks=3, chunk_max=70)
    kp, vp, ks, vs = fill_pool(b, kv_dtype, 16)
    q = np.random.default_rng(62).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, ks, vs, kv_dtype, partition_size=P,
                         chunk_partition_size=cp)
    want = run_ragged_oracle(b, q, kp, vp, ks, vs, kv_dtype)
    assert_close(got, want, what=f"{b.label} P {P} CP {cp} kv {kv_dtype}")


def test_rejects_bad_chunk_partition_size(ctx):
    b = workloads.small_mixed(12)
    kp, vp, ks, vs = fill_pool(b, oracle.KV_F32, 12)
    q = np.zeros(b.total_q * b.num_heads * b.head_dim, np.float32)
    for bad in (48, 16, 1024, 100):
        with pytest.raises(K.EngineError):
            run_ragged_gpu(ctx, b, q, kp, vp, chunk_partition_size=bad)


@pytest.mark.parametrize("decodes", [0, 4])
def test_chunk_partition_from_host_lengths(ctx, decodes):
    """kanso_ragged_chunk_partition_size: 0 when the batch has a decode row, else a
    multiple of 32 in [64, 512]; the call with it gives the oracle's result."""
    b = workloads.small_mixed(17, num_decodes=decodes, num_chunks=4, chunk_max=90)
    args = dict(q_lens=b.q_lens, context_lens=b.context_lens, num_heads=b.num_heads,
                num_kv_heads=b.num_kv_heads, head_dim=b.head_dim, block_size=b.block_size,
                max_blocks=b.max_blocks, num_blocks=b.num_blocks)
    cp = K.ragged_chunk_partition_size(ctx, **args)
    if decodes:
        assert cp == 0
    else:
        assert 64 <= cp <= 512 and cp % 32 == 0
    P = K.ragged_partition_size(ctx, **args)
    kp, vp, ks, vs = fill_pool(b, oracle.KV_F32, 18)
    q = np.random.default_rng(19).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, partition_size=P, chunk_partition_size=cp)
    want = run_ragged_oracle(b, q, kp, vp)
    assert_close(got, want, what=f"{b.label} P {P} CP {cp}")


@pytest.mark.parametrize("variant", ["config1", "config2_small_pool", "config2_bench_pool",
                                     "config3_int8", "config3_q8_0", "config3_fp8"])
def test_baseline_shapes(ctx, variant):
    """The benchmark configurations at their real shapes (pools sized to what the tables use;
    config2_bench_pool: the 64k-block pool of 2.7 GB the headline is timed on)."""
    if variant == "config1":
        b, kv = workloads.config1_decode(), oracle.KV_F32
    elif variant == "config2_small_pool":
        b, kv = workloads.config2_mixed(num_blocks=10000), oracle.KV_F32
    elif variant == "config2_bench_pool":
        b, kv = workloads.config2_mixed(num_blocks=65536), oracle.KV_F32
    else:
        b = workloads.config3_quant_decode()
        kv = {"int8": oracle.KV_INT8, "q8_0": oracle.KV_Q8_0,
              "fp8": oracle.KV_FP8}[variant.split("_", 1)[1]]
    kp, vp, ks, vs = fill_pool(b, kv, 7)
    q = np.random.default_rng(8).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, ks, vs, kv)
    want = run_ragged_oracle(b, q, kp, vp, ks, vs, kv)
    assert_close(got, want, what=variant)


def test_ragged_equals_decode_entry(ctx):
    """The reference-compatible decode entry and the ragged entry agree on decode rows."""
    b = workloads.config1_decode(seed_offset=3)
    kp, vp, _, _ = fill_pool(b, oracle.KV_F32, 9)
    q = np.random.default_rng(10).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    ragged = run_ragged_gpu(ctx, b, q, kp, vp)
    p = K.PagedAttentionParams(b.num_seqs, b.num_heads, b.num_kv_heads, b.head_dim,
                               b.block_size, b.max_blocks, b.scale)
    out = torch.empty(q.size, device="cuda:0")
    K.paged_attention_v2(ctx, p, dev(q), dev(kp), dev(vp), dev(b.block_tables.ravel()),
                         dev(b.context_lens.astype(np.uint32)), out)
    ctx.check_device_status()
    np.testing.assert_array_equal(host(out), ragged)


def test_decode_batch_without_cu_seqlens(ctx):
    """A null cu_seqlens reads as one row per sequence: bit-identical to passing 0..=S;
    a batch with a multi-row sequence still needs it."""
    b = workloads.config1_decode(seed_offset=4)
    kp, vp, _, _ = fill_pool(b, oracle.KV_F32, 11)
    q = np.random.default_rng(12).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    np.testing.assert_array_equal(run_ragged_gpu(ctx, b, q, kp, vp, cu_seqlens=False),
                                  run_ragged_gpu(ctx, b, q, kp, vp))
    m = workloads.small_mixed(3)
    kp, vp, _, _ = fill_pool(m, oracle.KV_F32, 13)
    q = np.zeros(m.total_q * m.num_heads * m.head_dim, np.float32)
    with pytest.raises(K.EngineError, match="null buffer"):
        run_ragged_gpu(ctx, m, q, kp, vp, cu_seqlens=False)


def test_fp8_pool_decodes_every_finite_code(ctx):
    """Contexts of one token: the output is exactly that token's V row, so every
    finite E4M3 code (254 of 256) is decoded by the kernel and compared bit for bit."""
    codes = np.array([c for c in range(256) if c not in (0x7f, 0xff)], np.uint8)
    d, S, bs = 64, 4, 16
    vrows = np.zeros((S, d), np.uint8)
    vrows.ravel()[:codes.size] = codes
    b = workloads.AttnBatch(np.ones(S, np.int64), np.ones(S, np.int64),
                            np.arange(S, dtype=np.uint32)[:, None], S, num_heads=1,
                            num_kv_heads=1, head_dim=d, block_size=bs, scale=0.125)
    kp = np.zeros(S * bs * d, np.int8)
    vp = np.zeros(S * bs * d, np.int8)
    for s in range(S):  # token 0 of block s
        vp[s * bs * d:s * bs * d + d] = vrows[s].view(np.int8)
    ks = np.ones(S * bs, np.float32)
    vs = np.full(S * bs, 0.5, np.float32)
    q = np.random.default_rng(3).standard_normal(S * d).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, ks, vs, oracle.KV_FP8).reshape(S, d)
    dec = np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float32)
    np.testing.assert_array_equal(got, dec[vrows] * np.float32(0.5))


@pytest.mark.parametrize("variant", ["small_mixed", "config1", "config3_q8_0"])
def test_partition_from_host_lengths(ctx, variant):
    """kanso_ragged_partition_size: a multiple of 32 in [32, 512] from the batch's
    host-side lengths, and the call with it gives the oracle's result."""
    if variant == "small_mixed":
        b, kv = workloads.small_mixed(13), oracle.KV_F32
    elif variant == "config1":
        b, kv = workloads.config1_decode(), oracle.KV_F32
    else:
        b, kv = workloads.config3_quant_decode(), oracle.KV_Q8_0
    P = K.ragged_partition_size(ctx, q_lens=b.q_lens, context_lens=b.context_lens,
                                num_heads=b.num_heads, num_kv_heads=b.num_kv_heads,
                                head_dim=b.head_dim, block_size=b.block_size,
                                max_blocks=b.max_blocks, kv_dtype=kv, num_blocks=b.num_blocks)
    assert 32 <= P <= 512 and P % 32 == 0
    kp, vp, ks, vs = fill_pool(b, kv, 14)
    q = np.random.default_rng(15).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    got = run_ragged_gpu(ctx, b, q, kp, vp, ks, vs, kv, partition_size=P)
    want = run_ragged_oracle(b, q, kp, vp, ks, vs, kv)
    assert_close(got, want, what=f"{variant} P {P}")
    assert K.ragged_partition_size(ctx, q_lens=[], context_lens=[], num_heads=15, num_kv_heads=5,
                                   head_dim=64, block_size=16, max_blocks=4) == 0


@pytest.mark.parametrize("case", ["small_mixed", "decode_only", "config2_small_pool", "int8", "q8_0"])
def test_work_list_equals_table_path(ctx, case):
    """kanso_ragged_paged_attention_work with the host-built work list (decode and
    chunk items) gives the table-driven call's output bit for bit (same item
    arithmetic, only the way a wave finds its item differs), for mixed and
    decode-only batches and 1-byte pools."""
    kv = {"int8": oracle.KV_INT8, "q8_0": oracle.KV_Q8_0}.get(case, oracle.KV_F32)
    if case == "decode_only":
        b = workloads.config1_decode(seed_offset=6)
    elif case == "config2_small_pool":
        b = workloads.config2_mixed(num_blocks=10000, seed_offset=2)
    elif case in ("int8", "q8_0"):
        b = workloads.config3_quant_decode(seed_offset=1)
    else:
        b = workloads.small_mixed(7)
    kp, vp, ks, vs = fill_pool(b, kv, 21)
    q = np.random.default_rng(22).standard_normal(
        b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    geo = dict(num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
               block_size=b.block_size)
    P = K.ragged_partition_size(ctx, q_lens=b.q_lens, context_lens=b.context_lens,
                                max_blocks=b.max_blocks, kv_dtype=kv, num_blocks=b.num_blocks, **geo)
    work = K.ragged_work(q_lens=b.q_lens, context_lens=b.context_lens, block_tables=b.block_tables,
                         partition_size=P, kv_dtype=kv, num_blocks=b.num_blocks,
                         max_q_len=int(b.q_lens.max()), **geo)
    assert work is not None
    work, n_chunk = work
    assert (n_chunk > 0) == (case in ("small_mixed", "config2_small_pool"))

    def call(w):
        out = torch.empty(b.total_q * b.num_heads * b.head_dim, device="cuda:0")
        K.ragged_paged_attention(
            ctx, q=dev(q), k_pool=dev(kp), v_pool=dev(vp), k_scales=None if ks is None else dev(ks),
            v_scales=None if vs is None else dev(vs), block_tables=dev(b.block_tables.ravel()),
            cu_seqlens=dev(b.cu_seqlens), context_lens=dev(b.context_lens.astype(np.uint32)), out=out,
            scale=b.scale, kv_dtype=kv, num_blocks=b.num_blocks, max_q_len=int(b.q_lens.max()),
            partition_size=P, work=None if w is None else dev(w), work_chunk_items=n_chunk, **geo)
        ctx.check_device_status()
        return host(out)

    np.testing.assert_array_equal(call(work), call(None))
