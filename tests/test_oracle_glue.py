"""Pins the oracle's decoder glue: RMSNorm / SiLU known answers from
tests/test_metal_kernel_parity.rs, RoPE identities, greedy argmax, FNV-1a."""
import numpy as np

import oracle


def test_rmsnorm_known_answer():
    y = oracle.rmsnorm([1.0, 2.0, 3.0, 4.0], [1.0] * 4, 1e-5)
    np.testing.assert_allclose(y, np.array([1, 2, 3, 4]) / 2.7386127, atol=1e-4)


def test_silu_gate_known_answer():
    y = oracle.silu_mul([0.0, 1.0], [2.0, 3.0])
    assert abs(y[0]) < 1e-4 and abs(y[1] - 2.1931758) < 1e-4


def test_rope_identities():
    D, H = 64, 3
    c, s = oracle.rope_table(2048, D)
    np.testing.assert_array_equal(c[0], 1.0)
    np.testing.assert_array_equal(s[0], 0.0)
    theta = 10000.0 ** (-2 * np.arange(D // 2) / D)
    np.testing.assert_allclose(c[1000], np.cos(1000 * theta), atol=2e-4)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, H, D)).astype(np.float32)
    pos = np.array([0, 1, 17, 999, 2047], np.int32)
    y = oracle.rope_apply(x, pos, H, D, c, s).reshape(5, H, D)
    np.testing.assert_array_equal(y[0], x[0])                     # position 0: identity
    np.testing.assert_allclose(np.linalg.norm(y, axis=2), np.linalg.norm(x, axis=2), rtol=1e-5)
    # rotate-half: pair (j, j+D/2) rotated by angle pos*theta_j
    a = pos[3] * theta
    want = np.concatenate([x[3, :, :32] * np.cos(a) - x[3, :, 32:] * np.sin(a),
                           x[3, :, :32] * np.sin(a) + x[3, :, 32:] * np.cos(a)], axis=1)
    np.testing.assert_allclose(y[3], want, atol=2e-3)


def test_greedy_first_max_wins():
    assert oracle.greedy([0.1, 3.0, 3.0, -1.0]) == 1
    assert oracle.greedy([-np.inf, -5.0]) == 1
    assert oracle.greedy([2.0]) == 0


def test_fnv1a_64():
    def ref(tokens):
        h = 0xcbf29ce484222325
        for t in tokens:
            h = ((h ^ t) * 0x100000001b3) % (1 << 64)
        return h
    assert oracle.fnv1a_64([]) == 0xcbf29ce484222325
    for toks in ([0], [1, 2, 3], list(range(1000)), [49151, 7, 0xFFFFFFFF]):
        assert oracle.fnv1a_64(toks) == ref(toks)
    # one XOR per u32 token, not per byte: differs from byte-wise FNV of the LE bytes
    assert oracle.fnv1a_64([0x01020304]) != ref([4, 3, 2, 1])
