"""GPU Q8_0 / Q4_K GEMV against the oracle at the SmolLM2-360M projection shapes."""
import numpy as np
import pytest
import torch

import kanso_infer_amd as K
import oracle
from gpu_helpers import assert_close, dev, host

pytestmark = pytest.mark.gpu

# (name, out_features, in_features): q, k/v, gate/up, down (SmolLM2-360M)
SHAPES = [("q", 960, 960), ("kv", 320, 960), ("gate_up", 2560, 960), ("down", 960, 2560)]
BATCHES = [1, 4, 8, 16, 32]

_weights = {}


def weights(kind, rows, cols):
    key = (kind, rows, cols)
    if key not in _weights:
        rng = np.random.default_rng(rows * 7 + cols)
        wf = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        w = oracle.quantize_row_q8_0(wf) if kind == "q8_0" else oracle.quantize_row_q4_k(wf)
        _weights[key] = (w, dev(w))
    return _weights[key]


def run(ctx, kind, rows, cols, batch, seed=0):
    w, wd = weights(kind, rows, cols)
    x = np.random.default_rng(seed + batch).standard_normal((batch, cols)).astype(np.float32)
    y = torch.empty(batch * rows, dtype=torch.float32, device="cuda:0")
    fn = K.gemv_q8_0 if kind == "q8_0" else K.gemv_q4_k
    fn(ctx, wd, dev(x), y, rows, cols)
    got = host(y)
    want = (oracle.gemv_q8_0 if kind == "q8_0" else oracle.gemv_q4_k)(w, x, rows, cols, nthreads=8)
    return got, want


@pytest.mark.parametrize("batch", BATCHES)
@pytest.mark.parametrize("name,rows,cols", SHAPES)
def test_q8_0(ctx, name, rows, cols, batch):
    got, want = run(ctx, "q8_0", rows, cols, batch)
    assert_close(got, want, what=f"q8_0 {name} b{batch}")


@pytest.mark.parametrize("batch", BATCHES + [64, 100, 300])
@pytest.mark.parametrize("name,rows,cols", [("down", 960, 2560), ("q_padded", 960, 1024),
                                            ("kv_padded", 320, 1024),
                                            ("gate_up_padded", 2560, 1024)])
def test_q4_k(ctx, name, rows, cols, batch):
    got, want = run(ctx, "q4_k", rows, cols, batch)
    assert_close(got, want, what=f"q4_k {name} b{batch}")


@pytest.mark.parametrize("batch", [1, 40, 300])
@pytest.mark.parametrize("rows,cols", [(16, 64), (80, 96), (1008, 960), (4112, 2560)])
def test_q8_0_ragged_row_counts(ctx, rows, cols, batch):
    """Row counts with an odd number of 16-row groups and of row pairs, so the last
    workgroup holds fewer groups / units than the others (NU > 1 clamps its extra
    units), at 16-token and 32-token tiles; GGUF-layout and packed entry points."""
    got, want = run(ctx, "q8_0", rows, cols, batch, seed=5)
    assert_close(got, want, what=f"q8_0 {rows}x{cols} b{batch}")
    w, wd = weights("q8_0", rows, cols)
    packed = K.pack_q8_0_matrix(ctx, wd, rows, cols)
    x = np.random.default_rng(5 + batch).standard_normal((batch, cols)).astype(np.float32)
    y = torch.empty(batch * rows, dtype=torch.float32, device="cuda:0")
    K.gemm_q8_0(ctx, packed, dev(x), y, rows, cols)
    assert_close(host(y), want, what=f"packed q8_0 {rows}x{cols} b{batch}")


@pytest.mark.parametrize("batch", [1, 40, 300])
@pytest.mark.parametrize("rows,cols", [(80, 256), (1008, 2560)])
def test_q4_k_ragged_row_counts(ctx, rows, cols, batch):
    """Q4_K at odd group / pair counts (partial last workgroup)."""
    got, want = run(ctx, "q4_k", rows, cols, batch, seed=6)
    assert_close(got, want, what=f"q4_k {rows}x{cols} b{batch}")


@pytest.mark.parametrize("kind,rows,cols", [("q4_k", 1008, 2560), ("q8_0", 1008, 960)])
def test_large_batch_equals_small_batches(ctx, kind, rows, cols):
    """300 tokens at once (64-token output tiles) give every token exactly what the
    same tokens give 16 at a time (the decode-sized kernel)."""
    w, wd = weights(kind, rows, cols)
    x = np.random.default_rng(9).standard_normal((300, cols)).astype(np.float32)
    fn = K.gemv_q8_0 if kind == "q8_0" else K.gemv_q4_k
    y = torch.empty(300 * rows, dtype=torch.float32, device="cuda:0")
    fn(ctx, wd, dev(x), y, rows, cols)
    full = host(y).reshape(300, rows)
    for t0 in range(0, 300, 16):
        n = min(16, 300 - t0)
        yc = torch.empty(n * rows, dtype=torch.float32, device="cuda:0")
        fn(ctx, wd, dev(x[t0:t0 + n]), yc, rows, cols)
        assert np.array_equal(full[t0:t0 + n], host(yc).reshape(n, rows)), t0


def test_reference_closed_form(ctx):
    # probes.rs:64-71 with an f16 scale: d = 0.01 (as f16), qs = 1, x = 1
    rows, cols = 64, 1024
    blk = np.concatenate([np.array([0.01], np.float16).view(np.uint8), np.ones(32, np.uint8)])
    w = np.tile(blk, rows * cols // 32)
    y = torch.empty(rows, device="cuda:0")
    K.gemv_q8_0(ctx, dev(w), torch.ones(cols, device="cuda:0"), y, rows, cols)
    d = float(np.float16(0.01))
    np.testing.assert_allclose(host(y), d * cols, rtol=1e-5)


def test_rejects_bad_shapes(ctx):
    y = torch.empty(4, device="cuda:0")
    x = torch.ones(100, device="cuda:0")
    w = torch.zeros(1000, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(K.EngineError):
        K.gemv_q8_0(ctx, w, x, y, 4, 100)  # in % 32 != 0
    with pytest.raises(K.EngineError):
        K.gemv_q4_k(ctx, w, torch.ones(96, device="cuda:0"), y, 4, 96)  # in % 256 != 0
