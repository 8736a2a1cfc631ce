"""The host restatement of kanso_model_init_random (oracle_init_random_q8_0): its
splitmix64 against the published output sequence, and the statistics the
Irwin-Hall(4) draw fixes. The byte-for-byte comparison with the device's weights is
tests/test_gpu_model.py::test_init_random_matches_oracle."""
import numpy as np

import oracle


def test_splitmix64_published_sequence():
    # splitmix64 from state 0 (Steele, Lea & Flood 2014; the reference sequence of
    # every SplitMix64 implementation)
    want = [0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f, 0xf88bb8a8724c81ec]
    x = 0
    for w in want:
        assert oracle.splitmix64(x) == w
        x = (x + 0x9e3779b97f4a7c15) % 2**64


def test_init_statistics():
    """Mean 0 and standard deviation std (Irwin-Hall(4) of 16-bit fields scaled by
    std * sqrt(3) / 65536), bounded by 131070 steps; checked on the dequantized
    weights of a 512 x 1024 matrix (Q8_0 error is ~0.4% of a block's max)."""
    std = 0.02
    w = oracle.init_random_q8_0(0xABCDEF, 512, 1024, std)
    x = oracle.dequant_q8_0_rows(w, 1024)
    assert abs(x.mean()) < 3 * std / np.sqrt(x.size) * 1.5
    assert abs(x.std() / std - 1) < 0.01
    c = oracle.lib().oracle_randn_scale(std)
    assert np.abs(x).max() <= 131070 * c * (1 + 1 / 127)
    # excess kurtosis of Irwin-Hall(4): -6 / (5 * 4) = -0.3
    k = ((x - x.mean()) ** 4).mean() / x.var() ** 2 - 3
    assert abs(k + 0.3) < 0.05


def test_init_streams_differ_and_repeat():
    a = oracle.init_random_q8_0(1, 32, 64, 0.02)
    assert np.array_equal(a, oracle.init_random_q8_0(1, 32, 64, 0.02))
    assert not np.array_equal(a, oracle.init_random_q8_0(2, 32, 64, 0.02))
    # element i depends on the flat index only: the first rows of a taller matrix agree
    assert np.array_equal(a, oracle.init_random_q8_0(1, 64, 64, 0.02)[:a.size])
