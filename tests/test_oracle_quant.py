"""Pins the oracle's KV quantizers, f16 conversion, Q8_0 / Q4_K decode and GEMV."""
import numpy as np
import pytest

import oracle
from refmath import (dequant_q4k_f64, q4k_gguf_to_dense, q8_0_gguf_to_dense, quantize_int8_f64,
                     quantize_q8_0_f64, scale_min_k4_table)


def test_f16_matches_numpy_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 5.96e-8, 2.98e-8, 2.99e-8, 6.1e-5,
                  np.inf, -np.inf], np.float32),
        # exact ties between two f16 values
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -11) + np.float32(1.0)),
    ]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(x) for x in vals], np.uint16)
    np.testing.assert_array_equal(got, want)
    back = np.array([oracle.f16_bits_to_f32(h) for h in want], np.float32)
    np.testing.assert_array_equal(back, want.view(np.float16).astype(np.float32))


def test_int8_head_quantizer_bit_exact_and_bounds():
    rng = np.random.default_rng(1)
    for trial in range(300):
        n = [4, 32, 64, 128, 256][trial % 5]
        x = (rng.standard_normal(n) * rng.uniform(1e-3, 50)).astype(np.float32)
        if trial % 17 == 0:
            x[:] = 0.0
        q, s = oracle.quantize_head_int8(x)
        qw, sw = quantize_int8_f64(x)
        np.testing.assert_array_equal(q, qw)
        assert s == sw
        if np.abs(x).max() > 0:
            assert np.abs(q).max() == 127
            assert np.all(np.abs(q.astype(np.float32) * s - x) <= s * 0.5 + 1e-6 * np.abs(x))
        else:
            assert s == 1.0 and not q.any()


def test_int8_reconstruction_matches_reference_bound():
    # tests/test_quantized_kv_cache.rs:5-86: sin/cos KV, rel-L2 reconstruction <= 1%.
    i = np.arange(4 * 64, dtype=np.float32)
    for raw in (np.sin(i * np.float32(0.1)) * np.float32(2.5),
                np.cos(i * np.float32(0.15)) * np.float32(1.8)):
        recon = np.zeros_like(raw)
        for h in range(4):
            q, s = oracle.quantize_head_int8(raw[h * 64:(h + 1) * 64])
            recon[h * 64:(h + 1) * 64] = q.astype(np.float32) * s
        assert np.linalg.norm(recon - raw) / np.linalg.norm(raw) <= 0.01


def test_kv_bytes_per_token():
    # quantized_storage.rs:414-429: INT8 = 2*h*d + 8*h B/token; ratio 4d/(d+4).
    for h, d in ((8, 128), (4, 64), (5, 64)):
        kp, vp, ks, vs = oracle.kv_pool_arrays(oracle.KV_INT8, 1, 1, h, d)
        assert kp.nbytes + vp.nbytes + ks.nbytes + vs.nbytes == 2 * h * d + 8 * h
        f32 = 2 * h * d * 4
        assert abs(f32 / (2 * h * d + 8 * h) - 4 * d / (d + 4)) < 1e-9
    # Q8_0 KV (Granite, Hkv=4, D=64): 544 B per token
    kp, vp, ks, vs = oracle.kv_pool_arrays(oracle.KV_Q8_0, 1, 1, 4, 64)
    assert kp.nbytes + vp.nbytes + ks.nbytes + vs.nbytes == 544


def test_q8_0_block_quantizer():
    # tests/test_neon_simd_gemv.rs:46-69: x = i*0.1 - 3.2, |deq - x| < d.
    xs = (np.arange(64, dtype=np.float32) * np.float32(0.1) - np.float32(3.2)).astype(np.float32)
    for b in range(2):
        q, d = oracle.quantize_q8_0_block(xs[b * 32:(b + 1) * 32])
        assert d > 0
        assert np.all(np.abs(q.astype(np.float32) * d - xs[b * 32:(b + 1) * 32]) < d)
    rng = np.random.default_rng(2)
    for _ in range(300):
        x = (rng.standard_normal(32) * rng.uniform(1e-4, 30)).astype(np.float32)
        q, d = oracle.quantize_q8_0_block(x)
        qw, dw = quantize_q8_0_f64(x)
        np.testing.assert_array_equal(q, qw)
        assert d == dw
    q, d = oracle.quantize_q8_0_block(np.zeros(32, np.float32))
    assert d == 0.0 and not q.any()


def test_kv_append_layouts():
    """Rows land at slot = block*bs + offset with the reference's per-block layout."""
    rng = np.random.default_rng(3)
    nb, bs, h, d = 6, 4, 3, 64
    slots = np.array([5, 0, 23, 12], np.int64)
    k = rng.standard_normal((4, h * d)).astype(np.float32)
    v = rng.standard_normal((4, h * d)).astype(np.float32)
    kp, vp, _, _ = oracle.kv_pool_arrays(oracle.KV_F32, nb, bs, h, d)
    oracle.kv_append(oracle.KV_F32, k, v, slots, nb, bs, h, d, kp, vp)
    pool = kp.reshape(nb, bs, h, d)
    for t, s in enumerate(slots):
        np.testing.assert_array_equal(pool[s // bs, s % bs].ravel(), k[t])
    kq, vq, ks, vs = oracle.kv_pool_arrays(oracle.KV_INT8, nb, bs, h, d)
    oracle.kv_append(oracle.KV_INT8, k, v, slots, nb, bs, h, d, kq, vq, ks, vs)
    for t, s in enumerate(slots):
        for hh in range(h):
            q, sc = quantize_int8_f64(k[t, hh * d:(hh + 1) * d])
            r = s * h + hh  # scale_idx = offset*n_kv_heads + h within block
            np.testing.assert_array_equal(kq.reshape(-1, d)[r], q)
            assert ks[r] == sc
    untouched = np.setdiff1d(np.arange(nb * bs * h), (slots[:, None] * h + np.arange(h)).ravel())
    assert (ks[untouched] == 1.0).all()
    with pytest.raises(ValueError):
        oracle.kv_append(oracle.KV_F32, k[:1], v[:1], [nb * bs], nb, bs, h, d, kp, vp)


def test_get_scale_min_k4_decoding():
    scales = [12, 24, 35, 48, 15, 20, 25, 30, 40, 50, 10, 5]  # test_neon_simd_gemv.rs:79
    table = scale_min_k4_table(scales)
    for j in range(8):
        assert oracle.get_scale_min_k4(j, scales) == table[j]
    # spelled out for this array: j<4 low 6 bits; j>=4 nibble + top bits
    assert table[:4] == [(12, 15), (24, 20), (35, 25), (48, 30)]
    assert table[4:] == [(40 & 15, 40 >> 4), (50 & 15, 50 >> 4), (10 & 15, 10 >> 4), (5 & 15, 5 >> 4)]
    rng = np.random.default_rng(4)
    for _ in range(200):
        s = rng.integers(0, 256, 12)
        assert [oracle.get_scale_min_k4(j, s) for j in range(8)] == scale_min_k4_table(s)


def _q4k_block_f32d(d, dmin, scales, qs):
    return np.concatenate([np.array([d, dmin], np.float32).view(np.uint8),
                           np.asarray(scales, np.uint8), np.asarray(qs, np.uint8)])


def test_q4k_dequant_closed_form_and_layout():
    # all nibbles equal n: every value of sub-block j is d*sc_j*n - dmin*m_j
    scales = [10, 20, 30, 40, 15, 25, 35, 45, 5, 12, 18, 22]
    for n in (0, 7, 15):
        qs = np.full(128, n | (n << 4), np.uint8)
        out = oracle.dequant_q4_k(_q4k_block_f32d(0.05, 0.02, scales, qs), f32d=True)
        pairs = scale_min_k4_table(scales)
        for j in range(8):
            sc, m = pairs[j]
            want = np.float32(np.float32(0.05) * sc) * n - np.float32(np.float32(0.02) * m)
            np.testing.assert_allclose(out[32 * j:32 * j + 32], want, rtol=1e-6)
    rng = np.random.default_rng(5)
    for _ in range(50):
        sc = rng.integers(0, 256, 12)
        qs = rng.integers(0, 256, 128)
        d, dmin = rng.uniform(0.001, 0.1, 2)
        out = oracle.dequant_q4_k(_q4k_block_f32d(d, dmin, sc, qs), f32d=True)
        want = dequant_q4k_f64(float(np.float32(d)), float(np.float32(dmin)), sc, qs)
        np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)


def test_q8_0_gemv_closed_form():
    # src/bench/probes.rs:64-71: d = 0.01, qs = 1, x = 1 -> out = 0.01 * cols
    rows, cols = 16, 1024
    blk = np.concatenate([np.array([0.01], np.float32).view(np.uint8), np.ones(32, np.uint8)])
    w = np.tile(blk, rows * cols // 32)
    y = oracle.gemv_q8_0_f32d(w, np.ones(cols, np.float32), rows, cols)
    np.testing.assert_allclose(y, 0.01 * cols, rtol=1e-5)


def test_q8_0_gemv_reference_patterns_vs_float64():
    # test_neon_simd_gemv.rs:102-141 weights, with d rounded to f16 for the GGUF layout
    rows, cols = 64, 128
    bpr = cols // 32
    blocks = []
    for r in range(rows):
        for b in range(bpr):
            qs = np.array([((r * 31 + b * 17 + i * 5) % 255) - 128 for i in range(32)], np.int8)
            d = np.float16(0.01 + r * 0.001)
            blocks.append(np.concatenate([np.array([d]).view(np.uint8), qs.view(np.uint8)]))
    w = np.concatenate(blocks)
    x = (np.sin(np.arange(cols, dtype=np.float32) * np.float32(0.1)) * np.float32(1.2)).astype(np.float32)
    y = oracle.gemv_q8_0(w, x, rows, cols)
    want = q8_0_gguf_to_dense(w, rows, cols) @ x.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-4)


def test_q4k_gemv_reference_patterns_vs_float64():
    # test_neon_simd_gemv.rs:144-188 (rows 32, cols 256), GGUF f16 d / dmin
    rows, cols = 32, 256
    blocks = []
    for r in range(rows):
        qs = np.array([(r * 13 + i * 7) & 0xFF for i in range(128)], np.uint8)
        dd = np.array([0.02 + r * 0.001, 0.01], np.float16).view(np.uint8)
        blocks.append(np.concatenate([dd, np.array([10, 20, 30, 40, 15, 25, 35, 45, 5, 12, 18, 22],
                                                   np.uint8), qs]))
    w = np.concatenate(blocks)
    x = (np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.05)) * np.float32(2.0)).astype(np.float32)
    y = oracle.gemv_q4_k(w, x, rows, cols)
    want = q4k_gguf_to_dense(w, rows, cols) @ x.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-4)


def test_quantized_weights_round_trip_and_batch():
    rng = np.random.default_rng(6)
    rows, cols, batch = 40, 512, 3
    wf = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    w8 = oracle.quantize_row_q8_0(wf)
    dense8 = q8_0_gguf_to_dense(w8, rows, cols)
    assert np.abs(dense8 - wf).max() <= np.abs(wf).max() / 127 * 0.51 + 1e-4
    y8 = oracle.gemv_q8_0(w8, x, rows, cols, nthreads=2).reshape(batch, rows)
    np.testing.assert_allclose(y8, x.astype(np.float64) @ dense8.T, rtol=1e-4, atol=1e-4)
    w4 = oracle.quantize_row_q4_k(wf)
    dense4 = q4k_gguf_to_dense(w4, rows, cols)
    # 4-bit: error per element within one quantization step of its sub-block
    assert np.abs(dense4 - wf).max() < 0.02
    y4 = oracle.gemv_q4_k(w4, x, rows, cols, nthreads=2).reshape(batch, rows)
    np.testing.assert_allclose(y4, x.astype(np.float64) @ dense4.T, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- FP8 (E4M3FN) KV

def _e4m3_table():
    return np.array([oracle.e4m3_to_f32(b) for b in range(256)], np.float32)


def test_e4m3_decode_closed_form():
    # OCP E4M3FN: bias 7, 3 mantissa bits, subnormal step 2^-9, NaN = S.1111.111.
    dec = _e4m3_table()
    assert dec[0x00] == 0.0 and dec[0x01] == 2.0 ** -9 and dec[0x07] == 7 * 2.0 ** -9
    assert dec[0x08] == 2.0 ** -6 and dec[0x38] == 1.0 and dec[0x39] == 1.125
    assert dec[0x7e] == 448.0 and dec[0xfe] == -448.0 and dec[0xb8] == -1.0
    assert np.isnan(dec[0x7f]) and np.isnan(dec[0xff])
    assert dec[0x80] == 0.0 and np.signbit(dec[0x80])
    finite = dec[~np.isnan(dec)]
    assert finite.size == 254 and np.unique(finite[finite > 0]).size == 126


def test_e4m3_encode_is_round_to_nearest_even():
    """Pinned by brute force: the nearest of the 254 finite codes, ties to the even
    mantissa, for random values, every exact code and every midpoint between codes."""
    dec = _e4m3_table()
    for b in range(256):
        if not np.isnan(dec[b]):
            assert oracle.f32_to_e4m3(dec[b]) == b or (dec[b] == 0 and b in (0, 0x80))
    pos = np.array(sorted({float(dec[b]) for b in range(0x7f)}), np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(5)
    xs = np.concatenate([mids, -mids] + [rng.standard_normal(3000).astype(np.float32) * s
                                         for s in (1e-3, 0.05, 1.0, 20.0, 60.0)])
    fin = [b for b in range(256) if not np.isnan(dec[b])]
    fvals = dec[fin].astype(np.float64)
    for x in xs:
        d = np.abs(fvals - float(x))
        cands = [fin[i] for i in np.nonzero(d == d.min())[0]]
        cands = [c for c in cands if (c >> 7) == int(np.signbit(x))] or cands
        want = min(cands, key=lambda c: (c & 1, c))
        assert oracle.f32_to_e4m3(float(x)) == want, (x, cands)


def test_fp8_head_quantizer_scale_rule_and_reference_kat():
    # scale = 2^ceil(log2(amax / 64)), 1 for amax = 0 (quantized_storage.rs:470-486)
    for amax, want in ((64.0, 1.0), (64.0001, 2.0), (32.0, 0.5), (33.0, 1.0), (1.0, 2.0 ** -6),
                       (448.0, 8.0)):
        x = np.zeros(64, np.float32)
        x[7] = -amax
        q, s = oracle.quantize_head_fp8(x)
        assert s == np.float32(want)
        assert q[7] == oracle.f32_to_e4m3(np.float32(-amax) * np.float32(1.0 / want))
    q, s = oracle.quantize_head_fp8(np.zeros(64, np.float32))
    assert s == 1.0 and not q.any()
    # tests/test_quantized_kv_cache.rs:88-166 inputs (4 heads x 64): these values are
    # exact in E4M3 after scaling, so reconstruction is exact (the test asks <= 1%).
    i = np.arange(4 * 64)
    k = ((i % 16) * 0.5 - 3.5).astype(np.float32)
    k[k == 0] = 1.0
    v = ((i % 8) * 1.0 + 0.5).astype(np.float32)
    dec = _e4m3_table()
    for raw in (k, v):
        recon = np.zeros_like(raw)
        for h in range(4):
            q, s = oracle.quantize_head_fp8(raw[h * 64:(h + 1) * 64])
            recon[h * 64:(h + 1) * 64] = dec[q] * s
        np.testing.assert_array_equal(recon, raw)
    # random rows: within half a step of E4M3 (1/16 relative, or half of 2^-9 * scale)
    rng = np.random.default_rng(6)
    for _ in range(200):
        x = (rng.standard_normal(64) * rng.uniform(1e-3, 100)).astype(np.float32)
        q, s = oracle.quantize_head_fp8(x)
        assert np.abs(x).max() / s <= 64.0
        assert np.all(np.abs(dec[q] * s - x) <= np.abs(x) / 16 + s * 2.0 ** -10 + 1e-7)


def test_fp8_pool_layout_is_the_int8_layout():
    rng = np.random.default_rng(7)
    nb, bs, h, d = 4, 4, 2, 64
    slots = np.array([3, 9], np.int64)
    k = rng.standard_normal((2, h * d)).astype(np.float32)
    kq, vq, ks, vs = oracle.kv_pool_arrays(oracle.KV_FP8, nb, bs, h, d)
    assert kq.nbytes + vq.nbytes + ks.nbytes + vs.nbytes == (2 * h * d + 8 * h) * nb * bs
    oracle.kv_append(oracle.KV_FP8, k, k, slots, nb, bs, h, d, kq, vq, ks, vs)
    for t, s in enumerate(slots):
        for hh in range(h):
            q, sc = oracle.quantize_head_fp8(k[t, hh * d:(hh + 1) * d])
            r = s * h + hh
            np.testing.assert_array_equal(kq.reshape(-1, d)[r].view(np.uint8), q)
            assert ks[r] == sc


def test_fp8_pool_attention_is_f32_attention_over_the_dequantized_pool():
    from kanso_infer_amd import workloads
    b = workloads.small_mixed(1)
    rng = np.random.default_rng(8)
    rows, width = b.num_blocks * b.block_size, b.num_kv_heads * b.head_dim
    k = rng.standard_normal((rows, width), dtype=np.float32)
    v = rng.standard_normal((rows, width), dtype=np.float32)
    kp, vp, ks, vs = oracle.kv_pool_arrays(oracle.KV_FP8, b.num_blocks, b.block_size,
                                           b.num_kv_heads, b.head_dim)
    oracle.kv_append(oracle.KV_FP8, k, v, np.arange(rows), b.num_blocks, b.block_size,
                     b.num_kv_heads, b.head_dim, kp, vp, ks, vs)
    q = rng.standard_normal(b.total_q * b.num_heads * b.head_dim).astype(np.float32)
    args = dict(num_heads=b.num_heads, num_kv_heads=b.num_kv_heads, head_dim=b.head_dim,
                block_size=b.block_size, scale=b.scale, num_blocks=b.num_blocks)
    got = oracle.ragged_attention(q, kp, vp, b.block_tables, b.cu_seqlens, b.context_lens,
                                  kv_dtype=oracle.KV_FP8, k_scales=ks, v_scales=vs, **args)
    dec = _e4m3_table()
    kf = (dec[kp.view(np.uint8)].reshape(-1, b.head_dim) * ks[:, None]).ravel()
    vf = (dec[vp.view(np.uint8)].reshape(-1, b.head_dim) * vs[:, None]).ravel()
    want = oracle.ragged_attention(q, kf, vf, b.block_tables, b.cu_seqlens, b.context_lens, **args)
    np.testing.assert_array_equal(got, want)
