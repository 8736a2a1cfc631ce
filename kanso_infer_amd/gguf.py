"""GGUF model files for the device model: the reader, the hyperparameters and the
weight mapping of ModelWeights::load_from_gguf (src/weights.rs:328-486).

The file layout is the public GGUF format (versions 2 and 3): a little-endian
header ("GGUF", version, tensor count, metadata count), typed metadata key/value
pairs, one info record per tensor (name, dims with ne[0] innermost, ggml type,
offset), then the tensor data at `general.alignment` (default 32). Tensor bytes
are memory-mapped, never read whole.

Weights go to the device model as GGUF Q8_0 rows, or as GGUF Q4_K rows, which the
model keeps in that format (the reference keeps every GGUF type as a QMatMul,
src/weights.rs:33-39). Three steps differ from a plain copy, all on the host at
load time:

* Q / K rows are reordered per head from llama.cpp's interleaved layout
  (x0, y0, x1, y1, ...) to the rotate-half layout the RoPE epilogue uses (evens,
  then odds: interleaved_permutation, src/weights.rs:231-252). The reference
  applies this index to the projected activations (QkPerm); a row of a Q8_0
  matrix is one output feature, so reordering whole rows is the same map, exactly.
* F32 / F16 / BF16 matrices are quantized to Q8_0 with this library's rounding
  (BlockQ8_0::from_f32_slice, src/quant/q8_0.rs:13-32); the reference would run
  them in their own format.
* Q6_K matrices, Q4_K embedding tables, and Q4_K matrices that share a fused
  product with a matrix of another type (a layer's Q / K / V, its gate / up) or
  whose rows are not whole 256-element super-blocks, are dequantized and
  quantized again to Q8_0: an approximation of the file's weights (Q8_0 keeps
  1/254 of each block's range), where the reference would use them exactly.
Other block formats are rejected with an error.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

GGUF_MAGIC = b"GGUF"

# ggml tensor types (the public ggml enum)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
GGML_Q4_K, GGML_Q6_K = 12, 14
# (block elements, block bytes) of the types this loader sizes
_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_BF16: (1, 2), GGML_Q8_0: (32, 34),
          2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 9: (32, 36), 10: (256, 84),
          11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292)}

# metadata value types
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
            10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file (EngineError::Config in the reference)."""


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple  # ne[0] first (innermost), as stored
    ggml_type: int
    offset: int   # absolute file offset of the data
    nbytes: int


class _Reader:
    def __init__(self, buf: memoryview):
        self.buf, self.pos = buf, 0

    def take(self, fmt: str):
        size = struct.calcsize(fmt)
        if self.pos + size > len(self.buf):
            raise GGUFError("truncated GGUF header")
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += size
        return v

    def string(self) -> str:
        n = self.take("<Q")
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated GGUF string")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vtype: int):
        if vtype in _SCALARS:
            return self.take(_SCALARS[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, count = self.take("<I"), self.take("<Q")
            return [self.value(etype) for _ in range(count)]
        raise GGUFError(f"unknown GGUF metadata type {vtype}")


class GGUFFile:
    """Parsed header of a GGUF file; tensor data stays memory-mapped."""

    def __init__(self, path):
        self.path = Path(path)
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        r = _Reader(memoryview(self._map))
        if bytes(self._map[:4]) != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: not a GGUF file")
        r.pos = 4
        self.version = r.take("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version} not supported (2, 3)")
        n_tensors, n_kv = r.take("<Q"), r.take("<Q")
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.take("<I"))
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.take("<I")
            shape = tuple(r.take("<Q") for _ in range(nd))
            infos.append((name, shape, r.take("<I"), r.take("<Q")))
        align = int(self.metadata.get("general.alignment", 32))
        data_start = (r.pos + align - 1) // align * align
        self.tensors: dict[str, TensorInfo] = {}
        for name, shape, gtype, off in infos:
            if gtype not in _BLOCK:
                raise GGUFError(f"tensor {name}: ggml type {gtype} not supported")
            be, bb = _BLOCK[gtype]
            n = int(np.prod(shape)) if shape else 1
            if shape[0] % be:
                raise GGUFError(f"tensor {name}: row of {shape[0]} not a multiple of {be}")
            nbytes = n // be * bb
            start = data_start + off
            if start + nbytes > self._map.size:
                raise GGUFError(f"tensor {name}: data past the end of the file")
            self.tensors[name] = TensorInfo(name, shape, gtype, start, nbytes)

    def raw(self, name: str) -> np.ndarray:
        """The stored bytes of a tensor (a read-only view of the mapping)."""
        t = self._info(name)
        return self._map[t.offset:t.offset + t.nbytes]

    def _info(self, name: str) -> TensorInfo:
        if name not in self.tensors:
            raise GGUFError(f"missing GGUF tensor '{name}'")
        return self.tensors[name]

    def f32(self, name: str) -> np.ndarray:
        """A dense tensor (F32 / F16 / BF16) as f32, flattened."""
        t = self._info(name)
        raw = self.raw(name)
        if t.ggml_type == GGML_F32:
            return raw.view(np.float32).copy()
        if t.ggml_type == GGML_F16:
            return raw.view(np.float16).astype(np.float32)
        if t.ggml_type == GGML_BF16:
            return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        raise GGUFError(f"tensor {name}: ggml type {t.ggml_type} is not a dense type")

    def q8_0_rows(self, name: str, quantize) -> np.ndarray:
        """A matrix as GGUF Q8_0 rows ([rows][in/32] x 34 B): stored Q8_0 bytes as they
        are; dense, Q4_K and Q6_K matrices (dequantized) quantized by `quantize`
        (f32 [rows, in] -> Q8_0 bytes)."""
        t = self._info(name)
        if len(t.shape) != 2:
            raise GGUFError(f"tensor {name}: expected a matrix, got shape {t.shape}")
        rows, cols = t.shape[1], t.shape[0]
        if t.ggml_type == GGML_Q8_0:
            return np.asarray(self.raw(name))
        if t.ggml_type in (GGML_F32, GGML_F16, GGML_BF16):
            return quantize(self.f32(name).reshape(rows, cols))
        if t.ggml_type == GGML_Q4_K:
            return quantize(dequant_q4_k(self.raw(name)).reshape(rows, cols))
        if t.ggml_type == GGML_Q6_K:
            return quantize(dequant_q6_k(self.raw(name)).reshape(rows, cols))
        raise GGUFError(f"tensor {name}: ggml type {t.ggml_type} cannot feed the model "
                        "(Q8_0, Q4_K, Q6_K, F32, F16 and BF16 load)")

    def ggml_type(self, name: str) -> int:
        return self._info(name).ggml_type


def _f16(raw: np.ndarray, at: int) -> np.ndarray:
    return raw[:, at:at + 2].copy().view(np.float16).astype(np.float32)[:, 0]


def dequant_q4_k(raw) -> np.ndarray:
    """GGUF block_q4_K bytes (256 elements: f16 d, f16 dmin, 12 bytes of packed 6-bit
    scales / mins, 128 nibble bytes) to f32: element 64 j + l is
    d * sc(2j) * (qs[32 j + l] & 15) - dmin * m(2j), element 64 j + 32 + l the same
    with the high nibble and sub-block 2j + 1 (BlockQ4_K::dequantize,
    src/quant/q4_k.rs:16-55)."""
    b = np.asarray(raw, np.uint8).reshape(-1, 144)
    d, dmin = _f16(b, 0), _f16(b, 2)
    sc = b[:, 4:16].astype(np.uint32)
    scale = np.empty((b.shape[0], 8), np.float32)
    mins = np.empty((b.shape[0], 8), np.float32)
    for j in range(8):  # get_scale_min_k4
        if j < 4:
            s_, m_ = sc[:, j] & 63, sc[:, j + 4] & 63
        else:
            s_ = (sc[:, j + 4] & 0xF) | ((sc[:, j - 4] >> 6) << 4)
            m_ = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
        scale[:, j] = d * s_.astype(np.float32)
        mins[:, j] = dmin * m_.astype(np.float32)
    qs = b[:, 16:144].reshape(-1, 4, 32)
    out = np.empty((b.shape[0], 4, 2, 32), np.float32)
    out[:, :, 0, :] = scale[:, 0::2, None] * (qs & 15).astype(np.float32) - mins[:, 0::2, None]
    out[:, :, 1, :] = scale[:, 1::2, None] * (qs >> 4).astype(np.float32) - mins[:, 1::2, None]
    return out.reshape(-1)


def dequant_q6_k(raw) -> np.ndarray:
    """GGUF block_q6_K bytes (256 elements: 128 bytes of low nibbles, 64 bytes of high
    bit pairs, 16 int8 sub-block scales, f16 d) to f32, from the public GGUF layout:
    in each 128-element half h, element 32 k + l (k = 0..3, l = 0..31) takes the low
    or high nibble of ql[64 h + 32 (k % 2) + l] (high for k >= 2) and bits 2k, 2k+1
    of qh[32 h + l] as its top two bits; w = d * scale[8 h + 2 k + l / 16] * (q - 32)."""
    b = np.asarray(raw, np.uint8).reshape(-1, 210)
    ql = b[:, 0:128].reshape(-1, 2, 2, 32).astype(np.int32)   # [half][k % 2][l]
    qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int32)     # [half][l]
    sc = b[:, 192:208].view(np.int8).astype(np.float32).reshape(-1, 2, 8)
    d = _f16(b, 208)
    q = np.empty((b.shape[0], 2, 4, 32), np.int32)
    for k in range(4):
        low = ql[:, :, k % 2, :]
        nib = (low >> 4) if k >= 2 else (low & 15)
        q[:, :, k, :] = (nib | (((qh >> (2 * k)) & 3) << 4)) - 32
    s_idx = (2 * np.arange(4)[:, None] + np.arange(32)[None, :] // 16)  # [k][l] -> scale slot
    scale = sc[:, :, s_idx]                                              # [blk][half][k][l]
    return (d[:, None, None, None] * scale * q.astype(np.float32)).reshape(-1)


def interleaved_permutation(num_heads: int, head_dim: int) -> np.ndarray:
    """Per head: even dimensions, then odd ones (src/weights.rs:231-252). Row j of the
    rotate-half matrix is row perm[j] of the interleaved one."""
    half = head_dim // 2
    base = np.arange(num_heads)[:, None] * head_dim
    idx = np.concatenate([2 * np.arange(half), 2 * np.arange(half) + 1])
    return (base + idx[None, :]).ravel()


def permute_q8_0_rows(rows: np.ndarray, num_heads: int, head_dim: int) -> np.ndarray:
    """Reorders the rows of a Q8_0 matrix (whole rows: exact) by interleaved_permutation."""
    r = np.asarray(rows).reshape(num_heads * head_dim, -1)
    return np.ascontiguousarray(r[interleaved_permutation(num_heads, head_dim)])


def _meta(g: GGUFFile, key: str):
    if key not in g.metadata:
        raise GGUFError(f"Missing GGUF metadata key '{key}'")
    return g.metadata[key]


def model_config(g: GGUFFile, max_position: int = 8192):
    """ModelConfig from the GGUF metadata (src/weights.rs:362-407)."""
    from .engine import ModelConfig
    arch = g.metadata.get("general.architecture")
    if arch is None:
        raise GGUFError("Missing GGUF metadata key 'general.architecture'")
    if arch not in ("llama", "granite"):
        raise GGUFError(f"unsupported GGUF architecture '{arch}': only 'llama' and 'granite' load")
    heads = int(_meta(g, f"{arch}.attention.head_count"))
    kv_heads = int(_meta(g, f"{arch}.attention.head_count_kv"))
    hidden = int(_meta(g, f"{arch}.embedding_length"))
    if heads == 0 or kv_heads == 0 or hidden < heads:
        raise GGUFError(f"cannot build KV storage: {heads} attention heads, {kv_heads} KV heads, "
                        f"hidden size {hidden}")
    head_dim = hidden // heads
    if head_dim != 64:
        raise GGUFError(f"head_dim {head_dim}: the device model's fused QKV/RoPE needs 64")
    vocab = int(g.tensors["token_embd.weight"].shape[1]) if "token_embd.weight" in g.tensors \
        else None
    if vocab is None:
        raise GGUFError("missing GGUF tensor 'token_embd.weight'")
    return ModelConfig(
        hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=kv_heads,
        num_hidden_layers=int(_meta(g, f"{arch}.block_count")),
        intermediate_size=int(_meta(g, f"{arch}.feed_forward_length")), vocab_size=vocab,
        rms_norm_eps=float(g.metadata.get(f"{arch}.attention.layer_norm_rms_epsilon", 1e-5)),
        rope_theta=float(g.metadata.get(f"{arch}.rope.freq_base", 10000.0)),
        max_position=max_position, tied_embeddings="output.weight" not in g.tensors,
        # Granite multipliers (src/weights.rs:395-406); absent = 0 = identity
        **({k: float(g.metadata.get(key, 0.0)) for k, key in (
            ("embedding_scale", "granite.embedding_scale"),
            ("attention_scale", "granite.attention.scale"),
            ("residual_scale", "granite.residual_scale"),
            ("logit_scale", "granite.logit_scale"))} if arch == "granite" else {}))


def load_weights(g: GGUFFile, cfg, quantize) -> dict:
    """The weights dict Model.load_weights takes, from the GGUF tensors
    (src/weights.rs:408-461 names), Q/K rows in rotate-half order. `quantize` turns
    a dense f32 [rows, in] matrix into Q8_0 rows (Model.from_gguf passes the
    device quantizer)."""
    hd = cfg.head_dim
    H, KV = cfg.num_attention_heads, cfg.num_key_value_heads
    w = {"embed": g.q8_0_rows("token_embd.weight", quantize),
         "final_norm": g.f32("output_norm.weight"), "layers": []}
    if not cfg.tied_embeddings:
        w["lm_head"] = g.q8_0_rows("output.weight", quantize)
    # names of each fused product (one format for all its matrices)
    groups = (("wq", "wk", "wv"), ("wo",), ("w_gate", "w_up"), ("w_down",))
    files = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
             "w_gate": "ffn_gate", "w_up": "ffn_up", "w_down": "ffn_down"}
    heads = {"wq": H, "wk": KV}
    for i in range(cfg.num_hidden_layers):
        p = f"blk.{i}."
        layer = {"attn_norm": g.f32(p + "attn_norm.weight"),
                 "ffn_norm": g.f32(p + "ffn_norm.weight"), "fmt": {}}
        for names in groups:
            tnames = [f"{p}{files[n]}.weight" for n in names]
            q4k = all(g.ggml_type(t) == GGML_Q4_K and g.tensors[t].shape[0] % 256 == 0
                      for t in tnames)
            for n, t in zip(names, tnames):
                rows = np.asarray(g.raw(t)) if q4k else g.q8_0_rows(t, quantize)
                if n in heads:  # whole rows: the same reorder in either format
                    rows = permute_q8_0_rows(rows, heads[n], hd)
                layer[n] = rows
                layer["fmt"][n] = GGML_Q4_K if q4k else GGML_Q8_0
        w["layers"].append(layer)
    return w
