"""A minimal GGUF v3 writer for tests: builds model files the loader reads (no
real checkpoints are available offline). Test infrastructure only."""
from __future__ import annotations

import struct

import numpy as np

T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64 = 4, 5, 6, 7, 8, 9, 10
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
        11: "<q", 12: "<d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == T_STRING:
        return _string(v)
    if vtype == T_ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, metadata, tensors, alignment: int = 32, version: int = 3) -> None:
    """metadata: [(key, vtype, value)]; tensors: [(name, ggml_type, ne tuple, bytes)]."""
    meta = list(metadata)
    if alignment != 32:
        meta.append(("general.alignment", T_U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, vtype, value in meta:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, gtype, ne, _), o in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", gtype, o)
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for (_, _, _, data), o in zip(tensors, offsets):
            f.write(bytes(data))
            f.write(b"\0" * ((-len(data)) % alignment))


def interleave_rows(rot_half_rows: np.ndarray, num_heads: int, head_dim: int) -> np.ndarray:
    """Inverse of the loader's permutation: rotate-half rows -> llama.cpp's interleaved
    order (row perm[j] of the file is row j of the rotate-half matrix)."""
    from kanso_infer_amd.gguf import interleaved_permutation
    r = np.asarray(rot_half_rows).reshape(num_heads * head_dim, -1)
    out = np.empty_like(r)
    out[interleaved_permutation(num_heads, head_dim)] = r
    return out


def llama_file(path, cfg: dict, weights: dict, dense=(), arch="llama", extra_meta=(), q4k=()) -> None:
    """A llama GGUF holding `weights` (the Model.load_weights dict, rotate-half Q/K) with
    Q/K rows interleaved as llama.cpp stores them. Names in `dense` are written as F16
    (quantized again by the loader), names in `q4k` as Q4_K (this build's quantizer
    over the dequantized Q8_0 rows)."""
    h, H, KV, D = cfg["hidden"], cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    meta = [("general.architecture", T_STRING, arch),
            (f"{arch}.block_count", T_U32, cfg["num_layers"]),
            (f"{arch}.attention.head_count", T_U32, H),
            (f"{arch}.attention.head_count_kv", T_U32, KV),
            (f"{arch}.embedding_length", T_U32, h),
            (f"{arch}.feed_forward_length", T_U32, cfg["intermediate"]),
            (f"{arch}.attention.layer_norm_rms_epsilon", T_F32, 1e-5),
            (f"{arch}.rope.freq_base", T_F32, 10000.0),
            ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, ["<a>", "<b>"]))] + list(extra_meta)
    tensors = []

    def mat(name, rows_q8, rows, cols):
        if name in dense:
            import oracle
            f = oracle.dequant_q8_0_rows(rows_q8, cols).astype(np.float16)
            tensors.append((name, 1, (cols, rows), f.tobytes()))
        elif name in q4k:
            import oracle
            f = oracle.dequant_q8_0_rows(rows_q8, cols)
            tensors.append((name, 12, (cols, rows), oracle.quantize_row_q4_k(f).tobytes()))
        else:
            tensors.append((name, 8, (cols, rows), np.asarray(rows_q8).tobytes()))

    V = cfg["vocab"]
    mat("token_embd.weight", weights["embed"], V, h)
    tensors.append(("output_norm.weight", 0, (h,), weights["final_norm"].astype(np.float32).tobytes()))
    if "lm_head" in weights:
        mat("output.weight", weights["lm_head"], V, h)
    for i, L in enumerate(weights["layers"]):
        p = f"blk.{i}."
        tensors.append((p + "attn_norm.weight", 0, (h,), L["attn_norm"].astype(np.float32).tobytes()))
        tensors.append((p + "ffn_norm.weight", 0, (h,), L["ffn_norm"].astype(np.float32).tobytes()))
        mat(p + "attn_q.weight", interleave_rows(L["wq"], H, D), H * D, h)
        mat(p + "attn_k.weight", interleave_rows(L["wk"], KV, D), KV * D, h)
        mat(p + "attn_v.weight", L["wv"], KV * D, h)
        mat(p + "attn_output.weight", L["wo"], h, H * D)
        mat(p + "ffn_gate.weight", L["w_gate"], cfg["intermediate"], h)
        mat(p + "ffn_up.weight", L["w_up"], cfg["intermediate"], h)
        mat(p + "ffn_down.weight", L["w_down"], h, cfg["intermediate"])
    write_gguf(path, meta, tensors)
