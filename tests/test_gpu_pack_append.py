"""GPU packing and fused KV append/quantize, bit-exact against the oracle."""
import numpy as np
import pytest
import torch

import kanso_infer_amd as K
import oracle
from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu


def random_plan(rng, S, bs, max_start=3000, chunk_frac=0.2):
    plan, tables, off = [], [], 0
    for s in range(S):
        q_len = int(rng.integers(2, 257)) if rng.random() < chunk_frac else 1
        start = int(rng.integers(0, max_start))
        need = (start + q_len + bs - 1) // bs
        extra = int(rng.integers(0, 4))
        tables.extend(rng.integers(0, 65536, need + extra))
        plan.append([start, q_len, off, need + extra, s * (max_start + 300)])
        off += need + extra
    plan = np.array(plan, np.uint32)
    arena = rng.integers(0, 49152, S * (max_start + 300)).astype(np.uint32)
    return plan, np.array(tables, np.uint32), arena


@pytest.mark.parametrize("seed,S,bs", [(0, 1, 16), (1, 52, 16), (2, 64, 16), (3, 300, 4),
                                       (4, 2000, 16)])
def test_pack_bit_exact(ctx, seed, S, bs):
    rng = np.random.default_rng(seed)
    plan, tables, arena = random_plan(rng, S, bs)
    got = K.pack_step(ctx, plan, dev(arena), dev(tables), bs)
    ctx.check_device_status()
    want = oracle.pack_step(plan, arena, tables, bs)
    assert got.max_blocks == want["max_blocks"]
    for name in ("cu_seqlens", "seq_of_query", "positions", "slot_mapping", "context_lens"):
        np.testing.assert_array_equal(host(getattr(got, name)).astype(np.int64),
                                      want[name].astype(np.int64), err_msg=name)
    np.testing.assert_array_equal(host(got.tokens).view(np.uint32), want["tokens"])
    np.testing.assert_array_equal(host(got.block_tables).view(np.uint32), want["block_tables"])


def test_pack_short_table_flagged(ctx):
    plan = np.array([[15, 2, 0, 1, 0]], np.uint32)
    K.pack_step(ctx, plan, dev(np.zeros(64, np.uint32)), dev(np.array([3], np.uint32)), 16)
    with pytest.raises(K.EngineError):
        ctx.check_device_status()


KV_KINDS = [oracle.KV_F32, oracle.KV_INT8, oracle.KV_Q8_0, oracle.KV_FP8]


def _pools(kv, nb, bs, h, d):
    kp, vp, ks, vs = oracle.kv_pool_arrays(kv, nb, bs, h, d)
    return [kp, vp, ks, vs], [None if a is None else dev(a) for a in (kp, vp, ks, vs)]


@pytest.mark.parametrize("kv", KV_KINDS)
@pytest.mark.parametrize("h,d,T", [(5, 64, 512), (4, 64, 32), (2, 128, 7), (1, 256, 3), (3, 32, 1)])
def test_append_bit_exact(ctx, kv, h, d, T):
    rng = np.random.default_rng(h * 1000 + d + T)
    nb, bs = 200, 16
    slots = rng.choice(nb * bs, size=T, replace=False).astype(np.int64)
    k = (rng.standard_normal((T, h * d)) * rng.uniform(0.01, 20, (T, 1))).astype(np.float32)
    v = rng.standard_normal((T, h * d)).astype(np.float32)
    if T > 2:
        k[1] = 0.0  # all-zero row: INT8 scale 1.0, Q8_0 d = 0
        v[2, :d] = np.float32(1e-30)  # tiny amax: exercises denormal-range scales
    host_arrays, dev_arrays = _pools(kv, nb, bs, h, d)
    K.kv_append(ctx, kv, dev(k), dev(v), dev(slots), nb, bs, h, d, *dev_arrays)
    ctx.check_device_status()
    oracle.kv_append(kv, k, v, slots, nb, bs, h, d, *host_arrays)
    for want, got in zip(host_arrays, dev_arrays):
        if want is None:
            continue
        np.testing.assert_array_equal(host(got).view(want.dtype), want)


@pytest.mark.parametrize("kv", KV_KINDS)
def test_append_config3_round_trip(ctx, kv):
    """Granite shape: 32 new tokens appended; dequantized values within half a step."""
    rng = np.random.default_rng(11)
    nb, bs, h, d, T = 4096, 16, 4, 64, 32
    slots = rng.choice(nb * bs, size=T, replace=False).astype(np.int64)
    k = rng.standard_normal((T, h * d)).astype(np.float32)
    v = rng.standard_normal((T, h * d)).astype(np.float32)
    host_arrays, dev_arrays = _pools(kv, nb, bs, h, d)
    K.kv_append(ctx, kv, dev(k), dev(v), dev(slots), nb, bs, h, d, *dev_arrays)
    ctx.check_device_status()
    kp = host(dev_arrays[0]).view(host_arrays[0].dtype)
    if kv == oracle.KV_F32:
        np.testing.assert_array_equal(kp.reshape(-1, h * d)[slots], k)
        return
    rows = (slots[:, None] * h + np.arange(h)).ravel()
    q = kp.reshape(-1, d)[rows].astype(np.float32)
    if kv == oracle.KV_FP8:
        # E4M3: 3 mantissa bits, so half a step is 1/16 of the value (normal range)
        # or half of the 2^-9 subnormal step
        dec = np.array([oracle.e4m3_to_f32(b) for b in range(256)], np.float32)
        sc = host(dev_arrays[2]).view(np.float32)[rows][:, None]
        recon = dec[kp.reshape(-1, d)[rows].view(np.uint8)] * sc
        err = np.abs(recon - k.reshape(-1, d))
        assert (err <= np.abs(k.reshape(-1, d)) / 16 + sc * 2.0 ** -10 + 1e-6).all()
        return
    if kv == oracle.KV_INT8:
        sc = host(dev_arrays[2]).view(np.float32)[rows][:, None]
        recon = q * sc
        step = sc
    else:
        sc = host(dev_arrays[2]).view(np.float16).astype(np.float32).reshape(-1, d // 32)[rows]
        sc = np.repeat(sc, 32, axis=1)
        recon = q * sc
        step = sc
    err = np.abs(recon - k.reshape(-1, d))
    assert (err <= 0.5 * step + 2e-3 * np.abs(k.reshape(-1, d)) + 1e-6).all()


def test_append_slot_out_of_bounds_flagged(ctx):
    nb, bs, h, d = 4, 16, 2, 64
    _, dev_arrays = _pools(oracle.KV_F32, nb, bs, h, d)
    k = torch.ones(1, h * d, device="cuda:0")
    K.kv_append(ctx, oracle.KV_F32, k, k, dev(np.array([nb * bs], np.int64)), nb, bs, h, d,
                *dev_arrays)
    with pytest.raises(K.EngineError):
        ctx.check_device_status()
    assert not host(dev_arrays[0]).any()


@pytest.mark.parametrize("kv", KV_KINDS)
def test_reset_blocks(ctx, kv):
    nb, bs, h, d = 8, 16, 2, 64
    rng = np.random.default_rng(12)
    host_arrays, dev_arrays = _pools(kv, nb, bs, h, d)
    k = rng.standard_normal((nb * bs, h * d)).astype(np.float32)
    K.kv_append(ctx, kv, dev(k), dev(k), dev(np.arange(nb * bs, dtype=np.int64)), nb, bs, h, d,
                *dev_arrays)
    K.kv_reset_blocks(ctx, kv, dev(np.array([1, 6], np.uint32)), nb, bs, h, d, *dev_arrays)
    ctx.check_device_status()
    kp = host(dev_arrays[0]).reshape(nb, -1)
    assert not kp[[1, 6]].any() and kp[[0, 2, 3, 4, 5, 7]].any()
    if kv in (oracle.KV_INT8, oracle.KV_FP8):
        ks = host(dev_arrays[2]).view(np.float32).reshape(nb, -1)
        assert (ks[[1, 6]] == 1.0).all()
    if kv == oracle.KV_Q8_0:
        ks = host(dev_arrays[2]).reshape(nb, -1)
        assert not ks[[1, 6]].any()
