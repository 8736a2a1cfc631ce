"""GGUF model files for the device model: the reader, the hyperparameters and the
weight mapping of ModelWeights::load_from_gguf (src/weights.rs:328-486).

The file layout is the public GGUF format (versions 2 and 3): a little-endian
header ("GGUF", version, tensor count, metadata count), typed metadata key/value
pairs, one info record per tensor (name, dims with ne[0] innermost, ggml type,
offset), then the tensor data at `general.alignment` (default 32). Tensor bytes
are memory-mapped, never read whole.

Weights go to the device model as GGUF Q8_0 rows. Two steps differ from a plain
copy, both on the host at load time:

* Q / K rows are reordered per head from llama.cpp's interleaved layout
  (x0, y0, x1, y1, ...) to the rotate-half layout the RoPE epilogue uses (evens,
  then odds: interleaved_permutation, src/weights.rs:231-252). The reference
  applies this index to the projected activations (QkPerm); a row of a Q8_0
  matrix is one output feature, so reordering whole rows is the same map, exactly.
* F32 / F16 / BF16 matrices are quantized to Q8_0 with this library's rounding
  (BlockQ8_0::from_f32_slice, src/quant/q8_0.rs:13-32); the reference would run
  them in their own format. Other block formats are rejected with an error.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

GGUF_MAGIC = b"GGUF"

# ggml tensor types (the public ggml enum)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
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
        are; dense matrices quantized by `quantize` (f32 [rows, in] -> Q8_0 bytes)."""
        t = self._info(name)
        if len(t.shape) != 2:
            raise GGUFError(f"tensor {name}: expected a matrix, got shape {t.shape}")
        if t.ggml_type == GGML_Q8_0:
            return np.asarray(self.raw(name))
        if t.ggml_type in (GGML_F32, GGML_F16, GGML_BF16):
            return quantize(self.f32(name).reshape(t.shape[1], t.shape[0]))
        raise GGUFError(f"tensor {name}: ggml type {t.ggml_type} cannot feed the Q8_0 model "
                        "(Q8_0, F32, F16 and BF16 load)")


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
    if arch == "granite":
        scales = [k for k in ("granite.embedding_scale", "granite.attention.scale",
                              "granite.residual_scale", "granite.logit_scale") if k in g.metadata]
        if scales:
            raise GGUFError(f"granite multipliers {scales} are not implemented by the device model")
    elif arch != "llama":
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
        max_position=max_position, tied_embeddings="output.weight" not in g.tensors)


def load_weights(g: GGUFFile, cfg, quantize) -> dict:
    """The weights dict Model.load_weights takes, from the GGUF tensors
    (src/weights.rs:408-461 names), Q/K rows in rotate-half order. `quantize` turns
    a dense f32 [rows, in] matrix into Q8_0 rows (Model.from_gguf passes the
    device quantizer)."""
    hd = cfg.head_dim
    w = {"embed": g.q8_0_rows("token_embd.weight", quantize),
         "final_norm": g.f32("output_norm.weight"), "layers": []}
    if not cfg.tied_embeddings:
        w["lm_head"] = g.q8_0_rows("output.weight", quantize)
    for i in range(cfg.num_hidden_layers):
        p = f"blk.{i}."
        w["layers"].append({
            "attn_norm": g.f32(p + "attn_norm.weight"),
            "ffn_norm": g.f32(p + "ffn_norm.weight"),
            "wq": permute_q8_0_rows(g.q8_0_rows(p + "attn_q.weight", quantize),
                                    cfg.num_attention_heads, hd),
            "wk": permute_q8_0_rows(g.q8_0_rows(p + "attn_k.weight", quantize),
                                    cfg.num_key_value_heads, hd),
            "wv": g.q8_0_rows(p + "attn_v.weight", quantize),
            "wo": g.q8_0_rows(p + "attn_output.weight", quantize),
            "w_gate": g.q8_0_rows(p + "ffn_gate.weight", quantize),
            "w_up": g.q8_0_rows(p + "ffn_up.weight", quantize),
            "w_down": g.q8_0_rows(p + "ffn_down.weight", quantize),
        })
    return w
