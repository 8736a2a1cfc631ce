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
    write_gguf(p, [], [("w", 12, (256, 2), bytes(2 * 144))])  # Q4_K matrix
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
    with pytest.raises(gguf.GGUFError):
        gguf.model_config(gguf.GGUFFile(p))
    llama_file(p, CFG, w, arch="granite")  # no multipliers: the llama decoder
    assert gguf.model_config(gguf.GGUFFile(p)).num_hidden_layers == 2
    odd = dict(CFG, num_heads=4)  # head_dim 32
    llama_file(p, odd, random_weights(dict(odd, head_dim=32), seed=4))
    with pytest.raises(gguf.GGUFError):
        gguf.model_config(gguf.GGUFFile(p))
