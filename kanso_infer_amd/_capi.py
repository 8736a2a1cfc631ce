"""ctypes declaration of libkanso_hip.so (include/kanso_hip.h).

torch is imported before the library is loaded: torch ships its own HIP runtime
(libamdhip64.so.7), and loading it first makes the library bind to that same
runtime, so torch's device buffers and streams are valid handles for it.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libkanso_hip.so"

KANSO_OK = 0
KANSO_E_INVALID_ARG = -1
KANSO_E_INVALID_SHAPE = -2
KANSO_E_OUT_OF_BOUNDS = -3
KANSO_E_HIP = -4
KANSO_E_DEVICE_CHECK = -5

KANSO_DEV_EMPTY_CONTEXT = 1 << 0
KANSO_DEV_CONTEXT_OVERFLOW = 1 << 1
KANSO_DEV_QUERY_OVERFLOW = 1 << 2
KANSO_DEV_TABLE_SHORT = 1 << 3
KANSO_DEV_SLOT_OOB = 1 << 4
KANSO_DEV_BLOCK_OOB = 1 << 5
KANSO_DEV_POSITION_OOB = 1 << 6
KANSO_DEV_TOKEN_OOB = 1 << 7
KANSO_DEV_PARTS_OOB = 1 << 8

KANSO_KV_F32 = 0
KANSO_KV_INT8 = 1
KANSO_KV_Q8_0 = 2
KANSO_KV_FP8 = 3
KANSO_RAGGED_WORK_ITEM_WORDS = 64  # kanso_hip.h

KANSO_POOL_TOKEN_MAJOR = 0
KANSO_POOL_HEAD_MAJOR = 1


class PagedAttentionParamsC(C.Structure):
    _fields_ = [
        ("num_seqs", C.c_uint32),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("block_size", C.c_uint32),
        ("max_num_blocks_per_seq", C.c_uint32),
        ("scale", C.c_float),
    ]


class RaggedAttentionParamsC(C.Structure):
    _fields_ = [
        ("num_seqs", C.c_uint32),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("block_size", C.c_uint32),
        ("max_num_blocks_per_seq", C.c_uint32),
        ("scale", C.c_float),
        ("total_q", C.c_uint32),
        ("kv_dtype", C.c_uint32),
        ("num_blocks", C.c_uint32),
        ("max_q_len", C.c_uint32),
        ("pool_layout", C.c_uint32),
        ("partition_size", C.c_uint32),
        ("chunk_partition_size", C.c_uint32),
    ]


class SeqPlanC(C.Structure):
    _fields_ = [
        ("start_pos", C.c_uint32),
        ("q_len", C.c_uint32),
        ("table_offset", C.c_uint32),
        ("table_len", C.c_uint32),
        ("token_offset", C.c_uint32),
    ]


class PackedStepC(C.Structure):
    _fields_ = [
        ("cu_seqlens", C.c_void_p),
        ("seq_of_query", C.c_void_p),
        ("positions", C.c_void_p),
        ("slot_mapping", C.c_void_p),
        ("tokens", C.c_void_p),
        ("block_tables", C.c_void_p),
        ("context_lens", C.c_void_p),
    ]


class QkvParamsC(C.Structure):
    _fields_ = [
        ("num_tokens", C.c_uint32),
        ("hidden", C.c_uint32),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("max_pos", C.c_uint32),
        ("eps", C.c_float),
        ("num_blocks", C.c_uint32),
        ("block_size", C.c_uint32),
    ]


class ModelConfigC(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("num_layers", C.c_uint32),
        ("intermediate", C.c_uint32),
        ("vocab", C.c_uint32),
        ("eps", C.c_float),
        ("rope_theta", C.c_float),
        ("max_position", C.c_uint32),
        ("tied_embeddings", C.c_uint32),
        ("embedding_scale", C.c_float),
        ("attention_scale", C.c_float),
        ("residual_scale", C.c_float),
        ("logit_scale", C.c_float),
    ]


class StepOutputC(C.Structure):
    _fields_ = [
        ("request_id", C.c_uint64),
        ("token_id", C.c_uint32),
        ("is_finished", C.c_uint32),
    ]


KANSO_W_EMBED, KANSO_W_LM_HEAD, KANSO_W_FINAL_NORM, KANSO_W_ATTN_NORM, KANSO_W_FFN_NORM = range(5)
KANSO_W_Q, KANSO_W_K, KANSO_W_V, KANSO_W_O, KANSO_W_GATE, KANSO_W_UP, KANSO_W_DOWN = range(5, 12)


# Every symbol the header declares, with its signature.
_P = C.c_void_p
_U = C.c_uint32
_I = C.c_int
SIGNATURES: dict[str, tuple] = {
    "kanso_last_error": (C.c_char_p, []),
    "kanso_create": (_I, [_I, C.POINTER(_P)]),
    "kanso_destroy": (_I, [_P]),
    "kanso_check_device_status": (_I, [_P, _P, C.POINTER(_U)]),
    "kanso_paged_attention_num_partitions": (_U, [C.POINTER(PagedAttentionParamsC)]),
    "kanso_validate_paged_attention_params": (_I, [C.POINTER(PagedAttentionParamsC)]),
    "kanso_paged_attention_v2": (_I, [_P, C.POINTER(PagedAttentionParamsC), _P, _P, _P, _P, _P, _P, _P]),
    "kanso_ragged_partition_size": (C.c_uint32, [_P, C.POINTER(RaggedAttentionParamsC), _P, _P]),
    "kanso_ragged_chunk_partition_size": (C.c_uint32, [_P, C.POINTER(RaggedAttentionParamsC), _P, _P]),
    "kanso_ragged_paged_attention": (
        _I, [_P, C.POINTER(RaggedAttentionParamsC), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "kanso_ragged_work_items": (C.c_uint32, [C.POINTER(RaggedAttentionParamsC), _P, _P, _P]),
    "kanso_ragged_build_work": (_I, [C.POINTER(RaggedAttentionParamsC), _P, _P, _P, _P, _U]),
    "kanso_ragged_paged_attention_work": (
        _I, [_P, C.POINTER(RaggedAttentionParamsC), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _U, _U, _P]),
    "kanso_ragged_paged_attention_noalloc": (
        _I, [_P, C.POINTER(RaggedAttentionParamsC), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "kanso_pack_step": (_I, [_P, _P, _U, _P, _P, _U, _U, _U, C.POINTER(PackedStepC), _P]),
    "kanso_kv_append": (_I, [_P, _U, _P, _P, _P, _U, _U, _U, _U, _U, _P, _P, _P, _P, _P]),
    "kanso_kv_reset_blocks": (_I, [_P, _U, _P, _U, _U, _U, _U, _U, _P, _P, _P, _P, _P]),
    "kanso_gemv_q8_0": (_I, [_P, _P, _P, _P, _U, _U, _U, _P]),
    "kanso_gemv_q4_k": (_I, [_P, _P, _P, _P, _U, _U, _U, _P]),
    "kanso_q8_0_packed_bytes": (C.c_size_t, [_U, _U]),
    "kanso_q8_0_pack": (_I, [_P, _P, _U, _U, _P, _U, _U, _P]),
    "kanso_gemm_q8_0": (_I, [_P, _P, _P, _P, _U, _U, _U, _P]),
    "kanso_gemm_q8_0_residual": (_I, [_P, _P, _P, _P, _U, _U, _U, _P]),
    "kanso_embed_q8_0": (_I, [_P, _P, _U, _U, _P, _U, _P, _P]),
    "kanso_qkv_rope_append": (_I, [_P, C.POINTER(QkvParamsC), _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _P, _P]),
    "kanso_qkv_rope_append_quant": (_I, [_P, C.POINTER(QkvParamsC), _P, _P, _P, _P, _P, _P, _P, _P, _U,
                                         _P, _P, _P, _P, _P]),
    "kanso_gate_up_swiglu": (_I, [_P, _P, _P, _P, C.c_float, _U, _U, _U, _P, _P]),
    "kanso_lm_head_argmax": (_I, [_P, _P, _P, _P, _P, C.c_float, _U, _U, _U, _P, _P, _P]),
    "kanso_quantize_q8_0": (_I, [_P, _P, C.c_uint64, _P, _P]),
    "kanso_model_create": (_I, [_P, C.POINTER(ModelConfigC), C.POINTER(_P)]),
    "kanso_model_destroy": (_I, [_P]),
    "kanso_model_set_weight": (_I, [_P, _U, _U, _P, C.c_size_t]),
    "kanso_model_init_random": (_I, [_P, C.c_uint64, C.c_float]),
    "kanso_model_get_weight": (_I, [_P, _U, _U, _P, C.c_size_t]),
    "kanso_model_set_weight_q4_k": (_I, [_P, _U, _U, _P, C.c_size_t]),
    "kanso_model_alloc_kv": (_I, [_P, _U, _U, _U, _U]),
    "kanso_model_alloc_kv_quant": (_I, [_P, _U, _U, _U, _U, _U]),
    "kanso_model_kv_pool": (_I, [_P, _U, C.POINTER(_P), C.POINTER(_P)]),
    "kanso_model_reset_blocks": (_I, [_P, _P, _U, _P]),
    "kanso_model_read_kv_rows": (_I, [_P, _U, _P, _U, _P, _P]),
    "kanso_model_forward": (_I, [_P, _P, _U, _P, _U, _P, _U, _P, _P, _P]),
    "kanso_model_forward_all_rows": (_I, [_P, _P, _U, _P, _U, _P, _U, _P, _P, _P]),
    "kanso_engine_create": (_I, [_P, _U, _U, _U, _U, _U, C.POINTER(_P)]),
    "kanso_engine_destroy": (_I, [_P]),
    "kanso_engine_add_request": (_I, [_P, _P, _U, _U, _P, _U, C.POINTER(C.c_uint64)]),
    "kanso_engine_step": (_I, [_P, _P, _U, C.POINTER(_U)]),
    "kanso_engine_last_plan": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "kanso_engine_stats": (_I, [_P, _P]),
    "kanso_engine_cancel": (_I, [_P, C.c_uint64, C.POINTER(_U)]),
    "kanso_engine_drain_finished": (_I, [_P, C.POINTER(_U)]),
    "kanso_engine_dry_token": (_U, [C.c_uint64, _U, _U]),
    "kanso_set_profiling": (_I, [_P, _I]),
    "kanso_get_kernel_time": (_I, [_P, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
}

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Loads libkanso_hip.so; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("KANSO_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: build it with `python -m kanso_infer_amd.build` "
            "(there is no CPU fallback for the HIP path)")
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
