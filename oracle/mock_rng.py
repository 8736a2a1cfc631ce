"""The reference's seeded mock-model weights, restated (TEST INFRASTRUCTURE ONLY:
the checker behind the golden-logits test; nothing in the product imports it).

Model::create_mock_tiny (src/model.rs:509-587) draws every weight matrix from one
`StdRng::seed_from_u64(0x5EED_0057)` stream (:201) through mock_randn_vec
(:213-227): u1 = random_range(f64::MIN_POSITIVE..1.0), u2 = random_range(0.0..1.0),
r = sqrt(-2 ln u1), theta = 2 pi u2, then r cos(theta) and r sin(theta) as f32.

The generator is a dependency absent from the reference tree: rand 0.9.5 / rand_core
0.9 / rand_chacha 0.9.0 (the reference's Cargo.lock). Their published algorithms,
restated here:

* rand_core `SeedableRng::seed_from_u64`: the 32-byte seed is eight PCG32 outputs
  (state = state * 6364136223846793005 + 11634580027462260723, then the XSH-RR
  output of the new state), little-endian.
* rand 0.9 `StdRng` is rand_chacha's ChaCha12Rng: the ChaCha block function (Bernstein)
  with 12 rounds, key = the seed, a 64-bit block counter in words 12-13 starting at
  0, stream 0 in words 14-15; output words in keystream order; `next_u64` takes two
  consecutive words, the first as the low half.
* rand 0.9 `UniformFloat<f64>::sample_single(low, high)`: scale = high - low; a value
  in [1, 2) from the top 52 bits of `next_u64` (bits >> 12 with exponent 0), minus 1,
  times scale, plus low (two roundings, no fused multiply-add); redrawn if not
  below high.

Pinned in tests by the ChaCha20 zero-key keystream (the published test vector of the
block function) and by the reference's own fixture tests/fixtures/golden_logits.json,
which only matches if every weight is reproduced.
"""
from __future__ import annotations

import math

import numpy as np

MOCK_SEED = 0x5EED0057
_M32 = 0xFFFFFFFF
_M64 = 0xFFFFFFFFFFFFFFFF


def seed_from_u64(state: int) -> list[int]:
    """rand_core 0.9 SeedableRng::seed_from_u64 for a 32-byte seed: 8 key words."""
    words = []
    for _ in range(8):
        state = (state * 6364136223846793005 + 11634580027462260723) & _M64
        xorshifted = (((state >> 18) ^ state) >> 27) & _M32
        rot = state >> 59
        words.append(((xorshifted >> rot) | (xorshifted << ((32 - rot) & 31))) & _M32)
    return words


def _rotl(x: int, n: int) -> int:
    return ((x << n) | (x >> (32 - n))) & _M32


def chacha_block(key: list[int], counter: int, stream: int = 0, rounds: int = 12) -> list[int]:
    """One 64-byte ChaCha block as 16 little-endian words."""
    s = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574, *key,
         counter & _M32, (counter >> 32) & _M32, stream & _M32, (stream >> 32) & _M32]
    x = list(s)

    def qr(a, b, c, d):
        x[a] = (x[a] + x[b]) & _M32
        x[d] = _rotl(x[d] ^ x[a], 16)
        x[c] = (x[c] + x[d]) & _M32
        x[b] = _rotl(x[b] ^ x[c], 12)
        x[a] = (x[a] + x[b]) & _M32
        x[d] = _rotl(x[d] ^ x[a], 8)
        x[c] = (x[c] + x[d]) & _M32
        x[b] = _rotl(x[b] ^ x[c], 7)

    for _ in range(rounds // 2):
        qr(0, 4, 8, 12)
        qr(1, 5, 9, 13)
        qr(2, 6, 10, 14)
        qr(3, 7, 11, 15)
        qr(0, 5, 10, 15)
        qr(1, 6, 11, 12)
        qr(2, 7, 8, 13)
        qr(3, 4, 9, 14)
    return [(x[i] + s[i]) & _M32 for i in range(16)]


class StdRng:
    """rand 0.9 StdRng (ChaCha12) seeded by seed_from_u64; only next_u64 is needed."""

    def __init__(self, seed: int, rounds: int = 12):
        self.key = seed_from_u64(seed)
        self.rounds = rounds
        self.counter = 0
        self.words: list[int] = []
        self.pos = 0

    def next_u32(self) -> int:
        if self.pos == len(self.words):
            self.words = chacha_block(self.key, self.counter, 0, self.rounds)
            self.counter += 1
            self.pos = 0
        w = self.words[self.pos]
        self.pos += 1
        return w

    def next_u64(self) -> int:
        lo = self.next_u32()
        return lo | (self.next_u32() << 32)

    def random_range_f64(self, low: float, high: float) -> float:
        scale = np.float64(high) - np.float64(low)
        while True:
            bits = (self.next_u64() >> 12) | (1023 << 52)
            value0_1 = np.float64(np.uint64(bits).view(np.float64)) - np.float64(1.0)
            res = value0_1 * scale + np.float64(low)
            if res < high:
                return float(res)


def mock_randn_vec(n: int, rng: StdRng) -> np.ndarray:
    """mock_randn_vec (src/model.rs:213-227)."""
    out = []
    tiny = np.finfo(np.float64).tiny  # f64::MIN_POSITIVE
    while len(out) < n:
        u1 = rng.random_range_f64(tiny, 1.0)
        u2 = rng.random_range_f64(0.0, 1.0)
        r = math.sqrt(-2.0 * math.log(u1))
        theta = 2.0 * math.pi * u2
        out.append(np.float32(r * math.cos(theta)))
        if len(out) < n:
            out.append(np.float32(r * math.sin(theta)))
    return np.asarray(out, dtype=np.float32)


def mock_tiny_weights(hidden: int, heads: int, kv_heads: int, layers: int, vocab: int):
    """Model::create_mock_tiny (src/model.rs:509-587): (config dict, weights dict) in
    the oracle's layout, F32 matrices [out][in]. Draw order: per layer q, k, v, o,
    gate, up, down; then the embedding; then the lm_head. Norm weights are ones."""
    hd = hidden // heads
    inter = 2 * hidden
    rng = StdRng(MOCK_SEED)

    def randn(rows, cols):
        return mock_randn_vec(rows * cols, rng).reshape(rows, cols)

    ws = []
    for _ in range(layers):
        layer = {"wq": randn(heads * hd, hidden), "wk": randn(kv_heads * hd, hidden),
                 "wv": randn(kv_heads * hd, hidden), "wo": randn(hidden, heads * hd),
                 "attn_norm": np.ones(hidden, np.float32)}
        layer.update({"w_gate": randn(inter, hidden), "w_up": randn(inter, hidden),
                      "w_down": randn(hidden, inter), "ffn_norm": np.ones(hidden, np.float32)})
        ws.append(layer)
    embed = randn(vocab, hidden)
    lm_head = randn(vocab, hidden)
    cfg = dict(hidden=hidden, num_heads=heads, num_kv_heads=kv_heads, head_dim=hd,
               num_layers=layers, intermediate=inter, vocab=vocab, eps=1e-5,
               rope_theta=10000.0, weight_format=1)
    weights = {"embed": embed, "lm_head": lm_head, "final_norm": np.ones(hidden, np.float32),
               "layers": ws}
    return cfg, weights
