"""GGUF reader, hyperparameters and weight mapping (kanso_infer_amd/gguf.py) on files
written by tests/gguf_writer.py; CPU only."""
import numpy as np
import pytest

import oracle
from gguf_writer import (T_ARRAY, T_BOOL, T_F32, T_STRING, T_U32, T_U64, interleave_rows,
                         llama_file, write_gguf)
from kanso_infer_amd import gguf
from model_ref import random_weights

CFG = dict(hidden=128, num_heads=2, num_kv_heads=1, head_dim=64, num_layers=2,
           intermediate=256, vocab=300)


def host_quantize(a):
    return oracle.quantize_row_q8_0(np.ascontiguousarray(a, np.float32))


def test_reader_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    q = oracle.quantize_row_q8_0(rng.standard_normal((3, 64)).astype(np.float32))
    v = rng.standard_normal(7).astype(np.float32)
    h = rng.standard_normal((2, 32)).astype(np.float16)
    meta = [("a.u32", T_U32, 7), ("a.f32", T_F32, 0.25), ("a.s", T_STRING, "héllo"),
            ("a.b", T_BOOL, True), ("a.u64", T_U64, 1 << 40),
            ("a.arr", T_ARRAY, (T_STRING, ["x", "yz"]))]
    for align in (32, 64):
        p = tmp_path / f"t{align}.gguf"
        write_gguf(p, meta, [("q", 8, (64, 3), q.tobytes()), ("v", 0, (7,), v.tobytes()),
                             ("h", 1, (32, 2), h.tobytes())], alignment=align)
        g = gguf.GGUFFile(p)
        assert g.version == 3
        assert g.metadata["a.u32"] == 7 and g.metadata["a.f32"] == 0.25
        assert g.metadata["a.s"] == "héllo" and g.metadata["a.b"] is True
        assert g.metadata["a.u64"] == 1 << 40 and g.metadata["a.arr"] == ["x", "yz"]
        assert g.tensors["q"].shape == (64, 3) and g.tensors["q"].nbytes == 3 * 2 * 34
        assert g.tensors["q"].offset % align == 0
        np.testing.assert_array_equal(g.raw("q"), q)
        np.testing.assert_array_equal(g.f32("v"), v)
        np.testing.assert_array_equal(g.f32("h"), h.astype(np.float32).ravel())
        np.testing.assert_array_equal(g.q8_0_rows("h", host_quantize),
                                      host_quantize(h.astype(np.float32)))


def test_reader_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML" + bytes(60))
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(p)
    write_gguf(p, [], [("x", 0, (4,), bytes(16))], version=1)
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(p)
    write_gguf(p, [], [("x", 0, (4,), bytes(16))])
    p.write_bytes(p.read_bytes()[:-20])  # data cut short
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(p)
    write_gguf(p, [], [("w", 13, (256, 2), bytes(2 * 176))])  # Q5_K matrix: no loader
    g = gguf.GGUFFile(p)
    with pytest.raises(gguf.GGUFError):
        g.q8_0_rows("w", host_quantize)


def test_interleaved_permutation_closed_form():
    # src/weights.rs:231-252: per head, even dimensions first, then odd ones
    np.testing.assert_array_equal(gguf.interleaved_permutation(2, 4), [0, 2, 1, 3, 4, 6, 5, 7])
    p = gguf.interleaved_permutation(5, 64)
    assert sorted(p) == list(range(320)) and p[32] == 1 and p[64] == 64


def test_permutation_turns_interleaved_rope_into_rotate_half():
    """llama.cpp's RoPE rotates adjacent pairs (x_2i, x_2i+1); the model's rotate-half
    RoPE rotates (x_i, x_i+D/2) (src/model.rs:720-737). Reordering the projection rows
    by the permutation must make the two agree, which pins its direction."""
    D, theta = 64, 10000.0
    rng = np.random.default_rng(1)
    x = rng.standard_normal(D)
    inv = theta ** (-np.arange(D // 2) * 2.0 / D)
    for pos in (0, 1, 17, 1000):
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        inter = x.copy()
        inter[0::2], inter[1::2] = x[0::2] * c - x[1::2] * s, x[0::2] * s + x[1::2] * c
        perm = gguf.interleaved_permutation(1, D)
        y = x[perm]
        rot = np.concatenate([y[:D // 2] * c - y[D // 2:] * s, y[:D // 2] * s + y[D // 2:] * c])
        np.testing.assert_allclose(inter[perm], rot, rtol=0, atol=1e-12)


def test_model_config_and_weights(tmp_path):
    w = random_weights(CFG, seed=2)
    p = tmp_path / "m.gguf"
    llama_file(p, CFG, w)
    g = gguf.GGUFFile(p)
    cfg = gguf.model_config(g)
    assert (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads) == (128, 2, 1)
    assert (cfg.num_hidden_layers, cfg.intermediate_size, cfg.vocab_size) == (2, 256, 300)
    assert cfg.tied_embeddings and cfg.rms_norm_eps == np.float32(1e-5)
    got = gguf.load_weights(g, cfg, host_quantize)
    np.testing.assert_array_equal(got["embed"], w["embed"])
    np.testing.assert_array_equal(got["final_norm"], w["final_norm"])
    for a, b in zip(got["layers"], w["layers"]):
        for k in b:  # Q / K come back in rotate-half order, byte for byte
            np.testing.assert_array_equal(np.asarray(a[k]).ravel(), np.asarray(b[k]).ravel())


def test_model_config_rejections(tmp_path):
    w = random_weights(CFG, seed=3)
    p = tmp_path / "m.gguf"
    llama_file(p, CFG, w, arch="mamba")
    with pytest.raises(gguf.GGUFError):
        gguf.model_config(gguf.GGUFFile(p))
    llama_file(p, CFG, w, arch="granite", extra_meta=[("granite.residual_scale", T_F32, 0.2)])
    c = gguf.model_config(gguf.GGUFFile(p))  # Granite multipliers load (absent ones stay 0)
    assert c.residual_scale == np.float32(0.2) and c.embedding_scale == 0.0 and c.logit_scale == 0.0
    llama_file(p, CFG, w, arch="granite")  # no multipliers: the llama decoder
    assert gguf.model_config(gguf.GGUFFile(p)).num_hidden_layers == 2
    odd = dict(CFG, num_heads=4)  # head_dim 32
    llama_file(p, odd, random_weights(dict(odd, head_dim=32), seed=4))
    with pytest.raises(gguf.GGUFError):
        gguf.model_config(gguf.GGUFFile(p))


def test_dequant_q4_k_matches_oracle():
    """The loader's numpy Q4_K decode equals the oracle's restatement of
    BlockQ4_K::dequantize (src/quant/q4_k.rs:16-55) bit for bit."""
    import oracle
    x = np.random.default_rng(5).standard_normal((6, 512)).astype(np.float32)
    q = oracle.quantize_row_q4_k(x)
    want = np.concatenate([oracle.dequant_q4_k(q[i:i + 144]) for i in range(0, q.size, 144)])
    np.testing.assert_array_equal(gguf.dequant_q4_k(q), want)


def _pack_q6_k(q, scales, d):
    """One block_q6_K from 256 6-bit values (0..63), 16 int8 scales and d, by the public
    bit layout: for half h and l < 32, ql[64 h + l] holds the low nibbles of elements
    32 0 + l (low) and 64 + l (high) of that half, ql[64 h + 32 + l] those of 32 + l
    and 96 + l; qh[32 h + l] holds the top bit pairs of elements l, 32 + l, 64 + l and
    96 + l at bits 0-1, 2-3, 4-5, 6-7."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        e = q[128 * h:128 * (h + 1)]
        for l in range(32):
            ql[64 * h + l] = (e[l] & 15) | ((e[64 + l] & 15) << 4)
            ql[64 * h + 32 + l] = (e[32 + l] & 15) | ((e[96 + l] & 15) << 4)
            qh[32 * h + l] = ((e[l] >> 4) | ((e[32 + l] >> 4) << 2) | ((e[64 + l] >> 4) << 4)
                              | ((e[96 + l] >> 4) << 6))
    return np.concatenate([ql, qh, np.asarray(scales, np.int8).view(np.uint8),
                           np.array([d], np.float16).view(np.uint8)])


def test_dequant_q6_k_closed_form():
    """w = d * scale[j / 16] * (q - 32) for every element j of a block packed by the
    bit layout; parity with candle's Q6_K decode is unpinned beyond this (candle is
    not available), and only the loader's Q8_0 re-quantization consumes it."""
    rng = np.random.default_rng(9)
    for _ in range(4):
        q = rng.integers(0, 64, 256)
        scales = rng.integers(-128, 128, 16)
        d = np.float16(rng.uniform(0.001, 0.1))
        got = gguf.dequant_q6_k(_pack_q6_k(q, scales, d))
        want = np.float32(d) * scales[np.arange(256) // 16].astype(np.float32) * (q - 32).astype(np.float32)
        np.testing.assert_array_equal(got, want)


def test_q4_k_matrices_kept_and_mixed_groups_requantized(tmp_path):
    """Q4_K projections stay Q4_K bytes (Q / K rows reordered whole); a Q4_K gate whose
    up is Q8_0 is decoded and quantized again to Q8_0 (the pair shares one product)."""
    import oracle
    cfg = dict(CFG, hidden=256, intermediate=512, num_heads=4)
    w = random_weights(cfg, seed=6)
    p = tmp_path / "k.gguf"
    q4 = ("blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight",
          "blk.0.ffn_down.weight", "blk.1.ffn_gate.weight")
    llama_file(p, cfg, w, q4k=q4)
    g = gguf.GGUFFile(p)
    got = gguf.load_weights(g, gguf.model_config(g), host_quantize)
    L0, L1 = got["layers"]
    assert L0["fmt"] == dict(wq=12, wk=12, wv=12, wo=8, w_gate=8, w_up=8, w_down=12)
    assert L1["fmt"]["w_gate"] == 8 and L1["fmt"]["w_up"] == 8
    # Q4_K rows: the file's rows in rotate-half order
    want_q = oracle.quantize_row_q4_k(oracle.dequant_q8_0_rows(w["layers"][0]["wq"], 256))
    np.testing.assert_array_equal(np.asarray(L0["wq"]).ravel(), want_q)
    # the mixed gate: Q4_K decoded, then Q8_0
    gate_q4 = oracle.quantize_row_q4_k(oracle.dequant_q8_0_rows(w["layers"][1]["w_gate"], 256))
    np.testing.assert_array_equal(np.asarray(L1["w_gate"]).ravel(),
                                  host_quantize(gguf.dequant_q4_k(gate_q4).reshape(512, 256)).ravel())
