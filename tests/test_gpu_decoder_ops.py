"""GPU parity of the packed-Q8_0 matrix products and the fused decoder-layer
operations, each against the oracle's restatement of the reference op sequence
(src/model.rs:1569-1739) on the same seeded inputs."""
import numpy as np
import pytest
import torch

import kanso_infer_amd as K
import oracle
from gpu_helpers import assert_close, dev, host

pytestmark = pytest.mark.gpu


def q8_weights(rows, cols, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    return oracle.quantize_row_q8_0(wf)


def unpack_host(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """GGUF bytes rebuilt from the packed layout description (qs[kq][row][8] then
    d[16] per 544 B tile), independently of the device kernel."""
    nb = cols // 32
    tiles = packed.reshape(-1, nb, 544)
    out = np.zeros((rows, nb, 34), np.uint8)
    for r in range(rows):
        g, rr = divmod(r, 16)
        t = tiles[g]
        out[r, :, 0:2] = t[:, 512 + 2 * rr: 514 + 2 * rr]
        for kq in range(4):
            out[r, :, 2 + 8 * kq: 10 + 8 * kq] = t[:, 128 * kq + 8 * rr: 128 * kq + 8 * rr + 8]
    return out.ravel()


@pytest.mark.parametrize("rows,cols", [(960, 960), (320, 960), (100, 64), (17, 2560)])
def test_pack_is_a_relayout(ctx, rows, cols):
    w = q8_weights(rows, cols, rows + cols)
    packed = K.pack_q8_0_matrix(ctx, dev(w), rows, cols)
    got = host(packed)
    assert got.size == K.q8_0_packed_bytes(rows, cols)
    assert np.array_equal(unpack_host(got, rows, cols), w)
    # rows past the matrix are zero
    nb = cols // 32
    groups = got.size // (nb * 544)
    full = unpack_host(got, groups * 16, cols).reshape(groups * 16, -1)
    assert not full[rows:].any()


SHAPES = [("q", 960, 960), ("kv", 320, 960), ("gate_up", 2560, 960), ("down", 960, 2560),
          ("odd", 48, 96)]


@pytest.mark.parametrize("T", [1, 3, 16, 17, 32, 33, 64, 100, 512])
@pytest.mark.parametrize("name,rows,cols", SHAPES)
def test_gemm_packed(ctx, name, rows, cols, T):
    w = q8_weights(rows, cols, rows * 3 + cols)
    packed = K.pack_q8_0_matrix(ctx, dev(w), rows, cols)
    x = np.random.default_rng(T).standard_normal((T, cols)).astype(np.float32)
    y = torch.empty(T * rows, dtype=torch.float32, device="cuda:0")
    K.gemm_q8_0(ctx, packed, dev(x), y, rows, cols)
    want = oracle.gemv_q8_0(w, x, rows, cols, nthreads=8)
    assert_close(host(y), want, what=f"gemm {name} T{T}")


@pytest.mark.parametrize("T", [1, 40, 300])
def test_gemv_gguf_any_batch(ctx, T):
    rows, cols = 960, 2560
    w = q8_weights(rows, cols, 5)
    x = np.random.default_rng(T).standard_normal((T, cols)).astype(np.float32)
    y = torch.empty(T * rows, dtype=torch.float32, device="cuda:0")
    K.gemv_q8_0(ctx, dev(w), dev(x), y, rows, cols)
    assert_close(host(y), oracle.gemv_q8_0(w, x, rows, cols, nthreads=8), what=f"gguf T{T}")


@pytest.mark.parametrize("cols", [960, 2560])
@pytest.mark.parametrize("rows", [960, 5120])
def test_batch_invariance(ctx, rows, cols):
    """A token's output does not depend on the rest of the batch: every batch size
    (16- and 64-token tiles alike) assigns k-blocks to the same waves and sums them
    in the same order."""
    sizes = (1, 7, 16, 17, 32, 33, 40, 64, 200, 256, 257, 300, 512, 700)
    w = q8_weights(rows, cols, 9)
    packed = K.pack_q8_0_matrix(ctx, dev(w), rows, cols)
    x = np.random.default_rng(1).standard_normal((max(sizes), cols)).astype(np.float32)
    outs = []
    for T in sizes:
        y = torch.empty(T * rows, dtype=torch.float32, device="cuda:0")
        K.gemm_q8_0(ctx, packed, dev(x[:T]), y, rows, cols)
        outs.append(host(y).reshape(T, rows)[0])
    for T, o in zip(sizes[1:], outs[1:]):
        assert np.array_equal(o, outs[0]), T
    # every token of the largest batch (its 64-token tiles, the partial last one
    # included) against the same tokens 16 at a time
    y = torch.empty(max(sizes) * rows, dtype=torch.float32, device="cuda:0")
    K.gemm_q8_0(ctx, packed, dev(x), y, rows, cols)
    full = host(y).reshape(-1, rows)
    for t0 in range(0, max(sizes), 16):
        n = min(16, max(sizes) - t0)
        yc = torch.empty(n * rows, dtype=torch.float32, device="cuda:0")
        K.gemm_q8_0(ctx, packed, dev(x[t0:t0 + n]), yc, rows, cols)
        assert np.array_equal(full[t0:t0 + n], host(yc).reshape(n, rows)), t0


@pytest.mark.parametrize("T", [257, 300, 512])
def test_batch_invariance_rmsnorm(ctx, T):
    """The RMSNorm prologue's sum of squares too: gate/up + SwiGLU of T tokens at once
    equals the same tokens 16 at a time, bit for bit."""
    hidden, inter = 960, 2560
    rng = np.random.default_rng(T)
    wg, wu = q8_weights(inter, hidden, 3), q8_weights(inter, hidden, 4)
    packed = torch.zeros(K.q8_0_packed_bytes(2 * inter, hidden), dtype=torch.uint8, device="cuda:0")
    K.q8_0_pack(ctx, dev(wg), inter, hidden, packed, 2, 0)
    K.q8_0_pack(ctx, dev(wu), inter, hidden, packed, 2, 1)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    h = torch.empty(T * inter, device="cuda:0")
    K.gate_up_swiglu(ctx, packed, dev(x), dev(nw), h, hidden=hidden, intermediate=inter)
    full = host(h).reshape(T, inter)
    for t0 in range(0, T, 16):
        n = min(16, T - t0)
        hc = torch.empty(n * inter, device="cuda:0")
        K.gate_up_swiglu(ctx, packed, dev(x[t0:t0 + n]), dev(nw), hc, hidden=hidden, intermediate=inter)
        assert np.array_equal(full[t0:t0 + n], host(hc).reshape(n, inter)), t0


@pytest.mark.parametrize("T", [37, 300])
def test_gemm_residual(ctx, T):
    rows, cols = 960, 2560
    w = q8_weights(rows, cols, 11)
    packed = K.pack_q8_0_matrix(ctx, dev(w), rows, cols)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    h = rng.standard_normal((T, rows)).astype(np.float32)
    y = dev(h.copy())
    K.gemm_q8_0_residual(ctx, packed, dev(x), y, rows, cols)
    want = h.ravel() + oracle.gemv_q8_0(w, x, rows, cols, nthreads=8)
    assert_close(host(y).ravel(), want, what="residual")


def test_embed_bit_exact(ctx):
    vocab, hidden = 1000, 960
    rng = np.random.default_rng(4)
    table_f = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32)
    table = oracle.quantize_row_q8_0(table_f)
    packed = K.pack_q8_0_matrix(ctx, dev(table), vocab, hidden)
    toks = np.array([0, 999, 5, 5, 512, 17], np.uint32)
    out = torch.empty(toks.size * hidden, dtype=torch.float32, device="cuda:0")
    K.embed_q8_0(ctx, packed, vocab, hidden, dev(toks), out)
    ctx.check_device_status()
    want = oracle.dequant_q8_0_rows(table, hidden)[toks.astype(np.int64)]
    assert np.array_equal(host(out).reshape(toks.size, hidden), want)


def test_embed_token_out_of_range_flags(ctx):
    vocab, hidden = 64, 64
    table = oracle.quantize_row_q8_0(np.ones((vocab, hidden), np.float32))
    packed = K.pack_q8_0_matrix(ctx, dev(table), vocab, hidden)
    out = torch.empty(hidden, dtype=torch.float32, device="cuda:0")
    K.embed_q8_0(ctx, packed, vocab, hidden, dev(np.array([64], np.uint32)), out)
    with pytest.raises(K.EngineError):
        ctx.check_device_status()


def _qkv_case(T, H=15, HKV=5, hidden=960, seed=0, num_blocks=64, bs=16):
    D = 64
    rng = np.random.default_rng(seed)
    wq = q8_weights(H * D, hidden, seed + 1)
    wk = q8_weights(HKV * D, hidden, seed + 2)
    wv = q8_weights(HKV * D, hidden, seed + 3)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    norm_w = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    positions = rng.integers(0, 2000, T).astype(np.int32)
    slots = rng.choice(num_blocks * bs, T, replace=False).astype(np.int64)
    return dict(H=H, HKV=HKV, hidden=hidden, wq=wq, wk=wk, wv=wv, x=x, norm_w=norm_w,
                positions=positions, slots=slots, num_blocks=num_blocks, bs=bs)


@pytest.mark.parametrize("kv", [K.KANSO_KV_INT8, K.KANSO_KV_FP8, K.KANSO_KV_Q8_0])
@pytest.mark.parametrize("T", [1, 20, 70, 300])
def test_qkv_rope_append_quant_matches_two_kernels(ctx, T, kv):
    """The quantizing QKV epilogue writes the bytes of the two-kernel path (F32 rows
    from qkv_rope_append, then kv_append's fused quantize), bit for bit: Q, the
    written pool rows and their scales, and nothing else of the pool."""
    c = _qkv_case(T, seed=100 + T)
    H, HKV, hidden, D = c["H"], c["HKV"], c["hidden"], 64
    rows = (H + 2 * HKV) * D
    packed = torch.zeros(K.q8_0_packed_bytes(rows, hidden), dtype=torch.uint8, device="cuda:0")
    K.q8_0_pack(ctx, dev(c["wq"]), H * D, hidden, packed, 1, 0)
    K.q8_0_pack(ctx, dev(c["wk"]), HKV * D, hidden, packed, 1, 4 * H)
    K.q8_0_pack(ctx, dev(c["wv"]), HKV * D, hidden, packed, 1, 4 * (H + HKV))
    cos_t, sin_t = oracle.rope_table(2048, D)
    nb, bs = c["num_blocks"], c["bs"]
    nslots = nb * bs
    x, nw, pos, sl = dev(c["x"]), dev(c["norm_w"]), dev(c["positions"]), dev(c["slots"])
    # two kernels: F32 staging rows 0..T-1, then the fused append + quantize
    ks_ = torch.zeros(T * HKV * D, device="cuda:0")
    vs_ = torch.zeros_like(ks_)
    q2 = torch.empty(T * H * D, device="cuda:0")
    K.qkv_rope_append(ctx, packed, x, nw, pos, torch.arange(T, dtype=torch.int64, device="cuda:0"),
                      dev(cos_t), dev(sin_t), q2, ks_, vs_, hidden=hidden, num_heads=H,
                      num_kv_heads=HKV, num_blocks=T, block_size=1)

    def pools():
        kp = torch.full((nslots * HKV * D,), 7, dtype=torch.int8, device="cuda:0")
        if kv == K.KANSO_KV_Q8_0:
            sc = torch.full((nslots * HKV * D // 32,), 3.0, dtype=torch.float16, device="cuda:0")
        else:
            sc = torch.full((nslots * HKV,), 3.0, dtype=torch.float32, device="cuda:0")
        return kp, kp.clone(), sc, sc.clone()

    kp2, vp2, kS2, vS2 = pools()
    K.kv_append(ctx, kv, ks_, vs_, sl, nb, bs, HKV, D, kp2, vp2, kS2, vS2)
    kp1, vp1, kS1, vS1 = pools()
    q1 = torch.empty(T * H * D, device="cuda:0")
    K.qkv_rope_append_quant(ctx, packed, x, nw, pos, sl, dev(cos_t), dev(sin_t), q1, kv, kp1, vp1,
                            kS1, vS1, hidden=hidden, num_heads=H, num_kv_heads=HKV,
                            num_blocks=nb, block_size=bs)
    ctx.check_device_status()
    np.testing.assert_array_equal(host(q1), host(q2))
    for a, b in ((kp1, kp2), (vp1, vp2), (kS1, kS2), (vS1, vS2)):
        np.testing.assert_array_equal(host(a), host(b))
    assert (host(kp1).reshape(nslots, -1)[c["slots"]] != 7).any()


@pytest.mark.parametrize("T", [1, 20, 70, 300])
def test_qkv_rope_append(ctx, T):
    c = _qkv_case(T, seed=T)
    H, HKV, hidden, D = c["H"], c["HKV"], c["hidden"], 64
    rows = (H + 2 * HKV) * D
    packed = torch.zeros(K.q8_0_packed_bytes(rows, hidden), dtype=torch.uint8, device="cuda:0")
    K.q8_0_pack(ctx, dev(c["wq"]), H * D, hidden, packed, 1, 0)
    K.q8_0_pack(ctx, dev(c["wk"]), HKV * D, hidden, packed, 1, 4 * H)
    K.q8_0_pack(ctx, dev(c["wv"]), HKV * D, hidden, packed, 1, 4 * (H + HKV))
    cos_t, sin_t = oracle.rope_table(2048, D)
    nslots = c["num_blocks"] * c["bs"]
    kp = torch.zeros(nslots * HKV * D, device="cuda:0")
    vp = torch.zeros_like(kp)
    q = torch.empty(T * H * D, device="cuda:0")
    K.qkv_rope_append(ctx, packed, dev(c["x"]), dev(c["norm_w"]), dev(c["positions"]),
                      dev(c["slots"]), dev(cos_t), dev(sin_t), q, kp, vp, hidden=hidden,
                      num_heads=H, num_kv_heads=HKV, num_blocks=c["num_blocks"],
                      block_size=c["bs"])
    ctx.check_device_status()
    # oracle: rmsnorm -> three projections -> rope on Q and K
    n = oracle.rmsnorm(c["x"], c["norm_w"])
    qw = oracle.gemv_q8_0(c["wq"], n, H * D, hidden, nthreads=8)
    kw = oracle.gemv_q8_0(c["wk"], n, HKV * D, hidden, nthreads=8)
    vw = oracle.gemv_q8_0(c["wv"], n, HKV * D, hidden, nthreads=8)
    qw = oracle.rope_apply(qw, c["positions"], H, D, cos_t, sin_t)
    kw = oracle.rope_apply(kw, c["positions"], HKV, D, cos_t, sin_t)
    assert_close(host(q), qw, what="q")
    kpool = host(kp).reshape(nslots, HKV * D)
    vpool = host(vp).reshape(nslots, HKV * D)
    assert_close(kpool[c["slots"]], kw.reshape(T, -1), what="k")
    assert_close(vpool[c["slots"]], vw.reshape(T, -1), what="v")
    untouched = np.setdiff1d(np.arange(nslots), c["slots"])
    assert not kpool[untouched].any() and not vpool[untouched].any()


@pytest.mark.parametrize("T", [1, 33, 130, 300])
def test_gate_up_swiglu(ctx, T):
    hidden, inter = 960, 2560
    wg = q8_weights(inter, hidden, 21)
    wu = q8_weights(inter, hidden, 22)
    packed = torch.zeros(K.q8_0_packed_bytes(2 * inter, hidden), dtype=torch.uint8,
                         device="cuda:0")
    K.q8_0_pack(ctx, dev(wg), inter, hidden, packed, 2, 0)
    K.q8_0_pack(ctx, dev(wu), inter, hidden, packed, 2, 1)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    h = torch.empty(T * inter, device="cuda:0")
    K.gate_up_swiglu(ctx, packed, dev(x), dev(nw), h, hidden=hidden, intermediate=inter)
    n = oracle.rmsnorm(x, nw)
    want = oracle.silu_mul(oracle.gemv_q8_0(wg, n, inter, hidden, nthreads=8),
                           oracle.gemv_q8_0(wu, n, inter, hidden, nthreads=8))
    assert_close(host(h), want, what="swiglu")


@pytest.mark.parametrize("S,vocab", [(1, 49152), (5, 49152), (64, 49152), (300, 4096)])
def test_lm_head_argmax(ctx, S, vocab):
    hidden = 960
    table = q8_weights(vocab, hidden, 31)
    packed = K.pack_q8_0_matrix(ctx, dev(table), vocab, hidden)
    rng = np.random.default_rng(S)
    T = 3 * S
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    rows = np.sort(rng.choice(T, S, replace=False)).astype(np.int32)
    nw = np.ones(hidden, np.float32)
    logits = torch.empty(S * vocab, device="cuda:0")
    toks = torch.empty(S, dtype=torch.int32, device="cuda:0")
    K.lm_head_argmax(ctx, packed, dev(x), toks, hidden=hidden, vocab=vocab, rows=dev(rows),
                     norm_w=dev(nw), logits=logits)
    got_logits = host(logits).reshape(S, vocab)
    want = oracle.gemv_q8_0(table, oracle.rmsnorm(x[rows], nw), vocab, hidden,
                            nthreads=8).reshape(S, vocab)
    assert_close(got_logits, want, what="logits")
    got_toks = host(toks).view(np.uint32)
    for i in range(S):
        # the fused argmax is exactly greedy_token over the kernel's own logits
        assert got_toks[i] == oracle.greedy(got_logits[i])
        # and the oracle's logit at that token is within tolerance of its maximum
        assert want[i, got_toks[i]] >= want[i].max() - 2e-3


def test_lm_head_first_max_wins(ctx):
    # all-equal logits: the first index must win (greedy_token's strict >)
    vocab, hidden = 256, 64
    table = oracle.quantize_row_q8_0(np.full((vocab, hidden), 0.5, np.float32))
    packed = K.pack_q8_0_matrix(ctx, dev(table), vocab, hidden)
    toks = torch.empty(2, dtype=torch.int32, device="cuda:0")
    K.lm_head_argmax(ctx, packed, dev(np.ones((2, hidden), np.float32)), toks, hidden=hidden,
                     vocab=vocab)
    assert host(toks).tolist() == [0, 0]
