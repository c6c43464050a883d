"""ctypes binding of libanima_hip (include/anima_hip.h).

The library is loaded from this package directory (built in-tree by
``animaxs_amd.build``).  There is no fallback: if the library is missing or
fails to load, ``load()`` raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libanima_hip.so"

# anima_status
(OK, E_INVALID_SHAPE, E_OUT_OF_BOUNDS, E_OVERFLOW, E_MISALIGNED, E_UNSUPPORTED, E_DEVICE, E_INVALID_ARGUMENT,
 E_FORMAT, E_IO) = range(10)
STATUS_NAMES = {
    0: "OK", 1: "INVALID_SHAPE", 2: "OUT_OF_BOUNDS", 3: "OVERFLOW", 4: "MISALIGNED",
    5: "UNSUPPORTED", 6: "DEVICE", 7: "INVALID_ARGUMENT", 8: "FORMAT", 9: "IO",
}

# enums
LAYOUT_HEAD_MAJOR, LAYOUT_TOKEN_MAJOR = 0, 1
NUMERICS_LEGACY, NUMERICS_FP32_SCORES, NUMERICS_BF16_COMPUTE = 0, 1, 2
ATTN_AUTO, ATTN_FLASH, ATTN_GENERIC, ATTN_LEGACY_MPS = 0, 1, 2, 3
STORAGE_W4, STORAGE_W8, STORAGE_FP16, STORAGE_FP32 = 0, 1, 2, 3
LINEAR_AUTO, LINEAR_FUSED, LINEAR_DEQUANT_THEN_GEMM = 0, 1, 2
FAMILY_OTHER, FAMILY_ATTENTION_PROJECTION, FAMILY_MLP_UP, FAMILY_MLP_DOWN = 0, 1, 2, 3


class AnimaError(RuntimeError):
    """A non-zero anima_status (AnimapkError.validation analog)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{STATUS_NAMES.get(status, status)}] {message}")
        self.status = status
        self.message = message


class Buffer(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("length", C.c_int64)]


class AttentionConfig(C.Structure):
    _fields_ = [("tile_rows", C.c_int32), ("numerics", C.c_int32), ("backend", C.c_int32),
                ("layout", C.c_int32), ("token_stride", C.c_int64), ("flash_rows", C.c_int32)]


class QKPrologue(C.Structure):
    _fields_ = [("q_norm_weight", Buffer), ("k_norm_weight", Buffer), ("eps", C.c_float),
                ("rope", Buffer), ("rope_tokens", C.c_int64), ("rope_q", C.c_int32), ("rope_k", C.c_int32),
                ("k_rope", Buffer), ("k_rope_tokens", C.c_int64)]


class AttentionArgs(C.Structure):
    _fields_ = [
        ("query", Buffer), ("query_offset", C.c_int64),
        ("key", Buffer), ("key_offset", C.c_int64),
        ("value", Buffer), ("value_offset", C.c_int64),
        ("output", Buffer), ("output_offset", C.c_int64),
        ("heads", C.c_int64), ("query_count", C.c_int64), ("key_count", C.c_int64),
        ("head_dim", C.c_int64), ("key_value_heads", C.c_int64),
        ("causal", C.c_int32), ("layout", C.c_int32), ("token_stride", C.c_int64),
        ("batch", C.c_int64), ("key_lengths", C.c_void_p), ("key_lengths_on_device", C.c_int32),
        ("scale", C.c_float), ("prologue", C.POINTER(QKPrologue)),
        ("kv_token_stride", C.c_int64),
    ]


class QWeight(C.Structure):
    _fields_ = [
        ("storage", C.c_int32),
        ("packed", Buffer), ("packed_offset", C.c_int64),
        ("scale", Buffer), ("scale_offset", C.c_int64),
        ("zero", Buffer), ("zero_offset", C.c_int64),
        ("rows", C.c_int64), ("columns", C.c_int64), ("packed_row_stride", C.c_int64),
    ]


class LinearConfig(C.Structure):
    _fields_ = [("tile_rows", C.c_int32), ("backend", C.c_int32)]


class DitBlockWeights(C.Structure):
    _fields_ = [(n, QWeight) for n in (
        "self_q", "self_k", "self_v", "self_o", "cross_q", "cross_k", "cross_v", "cross_o", "mlp1", "mlp2",
        "mod_self_w1", "mod_self_w2", "mod_cross_w1", "mod_cross_w2", "mod_mlp_w1", "mod_mlp_w2")] + [
        ("self_q_norm", Buffer), ("self_k_norm", Buffer),
        ("cross_q_norm", Buffer), ("cross_k_norm", Buffer)]


class DitBlockArgs(C.Structure):
    _fields_ = [("residual", Buffer), ("emb", Buffer), ("adaln_lora", Buffer), ("context", Buffer),
                ("rope", Buffer), ("tokens", C.c_int64), ("dim", C.c_int64), ("heads", C.c_int64),
                ("head_dim", C.c_int64), ("context_tokens", C.c_int64), ("context_dim", C.c_int64),
                ("mlp_hidden", C.c_int64), ("eps", C.c_float)]


class QwenLayerWeights(C.Structure):
    _fields_ = [(n, QWeight) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        ("input_norm", Buffer), ("post_attention_norm", Buffer),
        ("q_norm", Buffer), ("k_norm", Buffer)]


class QwenLayerArgs(C.Structure):
    _fields_ = [("residual", Buffer), ("rope", Buffer), ("key_lengths", C.c_void_p),
                ("batch", C.c_int64), ("tokens", C.c_int64), ("hidden", C.c_int64), ("heads", C.c_int64),
                ("kv_heads", C.c_int64), ("head_dim", C.c_int64), ("intermediate", C.c_int64),
                ("eps", C.c_float)]


class DitPrepareWeights(C.Structure):
    _fields_ = [("x_embed", QWeight), ("t_embed1", QWeight), ("t_embed2", QWeight), ("t_norm", Buffer)]


class DitPrepareArgs(C.Structure):
    _fields_ = [("latent", Buffer), ("height", C.c_int64), ("width", C.c_int64), ("sigma", C.c_float),
                ("residual", Buffer), ("emb", Buffer), ("adaln_lora", Buffer), ("dim", C.c_int64),
                ("eps", C.c_float)]


class DitFinalWeights(C.Structure):
    _fields_ = [("mod_w1", QWeight), ("mod_w2", QWeight), ("proj", QWeight)]


class DitFinalArgs(C.Structure):
    _fields_ = [("residual", Buffer), ("emb", Buffer), ("adaln_lora", Buffer), ("velocity", Buffer),
                ("height", C.c_int64), ("width", C.c_int64), ("dim", C.c_int64), ("eps", C.c_float)]


class PackInfo(C.Structure):
    _fields_ = [("version", C.c_int32), ("component", C.c_int32), ("alignment", C.c_int64),
                ("tensor_count", C.c_int64), ("json_offset", C.c_int64), ("json_size", C.c_int64),
                ("table_offset", C.c_int64), ("table_bytes", C.c_int64), ("payload_offset", C.c_int64),
                ("file_size", C.c_int64), ("record_size", C.c_int32), ("quant_group", C.c_int32),
                ("quant_scheme", C.c_char_p), ("component_name", C.c_char_p)]


class PackTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("storage", C.c_int32), ("rank", C.c_int32), ("shape", C.c_int64 * 8),
                ("blob_offset", C.c_int64), ("blob_size", C.c_int64), ("data_offset", C.c_int64),
                ("data_size", C.c_int64), ("scale_offset", C.c_int64), ("scale_size", C.c_int64),
                ("zero_offset", C.c_int64), ("zero_size", C.c_int64), ("block_index", C.c_int64),
                ("crc32", C.c_uint32), ("has_crc32", C.c_int32), ("logical_dtype", C.c_char_p),
                ("quantization_format", C.c_char_p)]


class PackRange(C.Structure):
    _fields_ = [("logical_index", C.c_int64), ("file_offset", C.c_int64), ("length", C.c_int64),
                ("tensor_count", C.c_int64), ("host", C.c_void_p)]


# name -> (restype, argtypes)
_P = C.c_void_p
_PP = C.POINTER(C.c_void_p)
_I64 = C.c_int64
_I32 = C.c_int32
_S = C.c_int
SIGNATURES = {
    "anima_last_error": (C.c_char_p, []),
    "anima_abi_version": (C.c_int32, []),
    "anima_ctx_create": (_S, [_I32, _PP]),
    "anima_ctx_destroy": (_S, [_P]),
    "anima_ctx_set_stream": (_S, [_P, _P]),
    "anima_ctx_synchronize": (_S, [_P]),
    "anima_attention_create": (_S, [_P, C.POINTER(AttentionConfig), _PP]),
    "anima_attention_destroy": (_S, [_P]),
    "anima_attention_encode": (_S, [_P, C.POINTER(AttentionArgs)]),
    "anima_attention_execute": (_S, [_P, C.POINTER(AttentionArgs)]),
    "anima_attention_encode_noalloc": (_S, [_P, C.POINTER(AttentionArgs)]),
    "anima_attention_max_score_scratch_bytes": (_S, [_P, _I64, _I64, C.POINTER(_I64)]),
    "anima_attention_workspace_bytes": (_S, [_P, C.POINTER(_I64)]),
    "anima_linear_create": (_S, [_P, C.POINTER(LinearConfig), _PP]),
    "anima_linear_destroy": (_S, [_P]),
    "anima_linear_encode": (_S, [_P, Buffer, _I64, C.POINTER(QWeight), Buffer, _I64, _I64, _I32]),
    "anima_linear_execute": (_S, [_P, Buffer, _I64, C.POINTER(QWeight), Buffer, _I64, _I64, _I32]),
    "anima_linear_encode_group": (_S, [_P, Buffer, _P, _P, _I32, _I64, _I32]),
    "anima_linear_encode_epilogue": (_S, [_P, Buffer, _I64, C.POINTER(QWeight), Buffer, _I64, _I64, _I32, _I32,
                                          Buffer, Buffer]),
    "anima_matvec_encode": (_S, [_P, C.POINTER(QWeight), Buffer, _I64, Buffer, _I64]),
    "anima_dequant_to_half_encode": (_S, [_P, C.POINTER(QWeight), Buffer, _I64, _I64]),
    "anima_read_probe_encode": (_S, [_P, Buffer, _I64, _I64, Buffer]),
    "anima_read_probe_sink_bytes": (_I64, [_I64]),
    "anima_numerics_probe_reset_encode": (_S, [_P, Buffer, _I32]),
    "anima_numerics_probe_encode": (_S, [_P, Buffer, _I64, _I64, _I32, Buffer, _I32]),
    "anima_dequant_w4": (_S, [_P, _P, _P, _I64, _I64, _P]),
    "anima_dequant_w4_matrix": (_S, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "anima_dequant_w8": (_S, [_P, _P, _P, _I64, _I64, _P]),
    "anima_dequant_w8_matrix": (_S, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "anima_fp16_to_float32": (_S, [_P, _I64, _P]),
    "anima_rope_dit3d": (_S, [_I64, _I64, _I64, _P]),
    "anima_rope_neox": (_S, [_I64, _I64, C.c_float, _P]),
    "anima_layernorm_modulate_to_half_encode": (_S, [_P, Buffer, Buffer, Buffer, _I64, _I64, C.c_float, _I64]),
    "anima_gate_add_half_f32_encode": (_S, [_P, Buffer, Buffer, Buffer, _I64, _I64]),
    "anima_gelu_half_inplace_encode": (_S, [_P, Buffer, _I64]),
    "anima_silu_f32_encode": (_S, [_P, Buffer, Buffer, _I64]),
    "anima_add_f32_encode": (_S, [_P, Buffer, Buffer, _I64]),
    "anima_rmsnorm_f32_to_half_encode": (_S, [_P, Buffer, Buffer, Buffer, _I64, _I64, C.c_float]),
    "anima_gated_silu_half_encode": (_S, [_P, Buffer, Buffer, Buffer, _I64]),
    "anima_add_half_into_float_encode": (_S, [_P, Buffer, Buffer, _I64]),
    "anima_qwen_layer_create": (_S, [_P, _PP]),
    "anima_qwen_layer_destroy": (_S, [_P]),
    "anima_qwen_layer_encode": (_S, [_P, C.POINTER(QwenLayerWeights), C.POINTER(QwenLayerArgs)]),
    "anima_dit_block_create": (_S, [_P, _PP]),
    "anima_dit_block_destroy": (_S, [_P]),
    "anima_dit_block_encode": (_S, [_P, C.POINTER(DitBlockWeights), C.POINTER(DitBlockArgs)]),
    "anima_dit_block_encode_cached": (_S, [_P, C.POINTER(DitBlockWeights), C.POINTER(DitBlockArgs), _P, _I64]),
    "anima_dit_forward_encode": (_S, [_P, C.POINTER(DitBlockWeights), _I64, C.POINTER(DitBlockArgs), _P]),
    "anima_dit_forward_encode_streamed": (_S, [_P, _P, C.POINTER(DitBlockWeights), _P, _P, _I64,
                                               C.POINTER(DitBlockArgs), _P]),
    "anima_cross_kv_cache_create": (_S, [_P, _I64, _I64, _I64, _PP]),
    "anima_cross_kv_cache_destroy": (_S, [_P]),
    "anima_cross_kv_cache_reset": (_S, [_P]),
    "anima_cross_kv_cache_is_ready": (_S, [_P, _I64, C.POINTER(_I32)]),
    "anima_cross_kv_cache_bytes": (_S, [_P, C.POINTER(_I64)]),
    "anima_weight_streamer_create": (_S, [_P, _I64, _I32, _PP]),
    "anima_weight_streamer_destroy": (_S, [_P]),
    "anima_linear_encode_head_rmsnorm": (_S, [_P, Buffer, _I64, C.POINTER(QWeight), Buffer, _I64, _I64, _I32,
                                              Buffer, _I64, C.c_float]),
    "anima_patchify17_encode": (_S, [_P, Buffer, _I64, _I64, _I64, Buffer]),
    "anima_unpatchify16_encode": (_S, [_P, Buffer, _I64, _I64, Buffer]),
    "anima_unpatchify_velocity16_encode": (_S, [_P, Buffer, _I64, _I64, Buffer]),
    "anima_flow_velocity_to_denoised_encode": (_S, [_P, Buffer, Buffer, Buffer, C.c_float, _I64]),
    "anima_euler_step_encode": (_S, [_P, Buffer, Buffer, Buffer, C.c_float, C.c_float, _I64]),
    "anima_dit_prepare_create": (_S, [_P, _PP]),
    "anima_dit_prepare_destroy": (_S, [_P]),
    "anima_dit_prepare_encode": (_S, [_P, C.POINTER(DitPrepareWeights), C.POINTER(DitPrepareArgs)]),
    "anima_dit_final_create": (_S, [_P, _PP]),
    "anima_dit_final_destroy": (_S, [_P]),
    "anima_dit_final_encode": (_S, [_P, C.POINTER(DitFinalWeights), C.POINTER(DitFinalArgs)]),
    "anima_pack_open": (_S, [C.c_char_p, _PP]),
    "anima_pack_close": (_S, [_P]),
    "anima_pack_get_info": (_S, [_P, C.POINTER(PackInfo)]),
    "anima_pack_tensor_at": (_S, [_P, _I64, C.POINTER(PackTensor)]),
    "anima_pack_find": (_S, [_P, C.c_char_p, C.POINTER(PackTensor)]),
    "anima_pack_crc32_mismatch_count": (_S, [_P, C.POINTER(C.c_int64)]),
    "anima_pack_bytes": (_S, [_P, _I64, _I64, C.POINTER(C.c_void_p)]),
    "anima_pack_execution_ranges": (_S, [_P, C.c_char_p, _I64, C.POINTER(PackRange)]),
    "anima_pack_dit_block": (_S, [_P, _I64, C.POINTER(DitBlockWeights), C.POINTER(PackRange)]),
    "anima_pack_dit_prepare": (_S, [_P, _I64, C.POINTER(DitPrepareWeights), C.POINTER(PackRange)]),
    "anima_pack_dit_final": (_S, [_P, _I64, C.POINTER(DitFinalWeights), C.POINTER(PackRange)]),
    "anima_dit_block_weights_rebase": (_S, [C.POINTER(DitBlockWeights), _P, _I64, C.POINTER(DitBlockWeights)]),
    "anima_dit_prepare_weights_rebase": (_S, [C.POINTER(DitPrepareWeights), _P, _I64,
                                              C.POINTER(DitPrepareWeights)]),
    "anima_dit_final_weights_rebase": (_S, [C.POINTER(DitFinalWeights), _P, _I64, C.POINTER(DitFinalWeights)]),
}

_lib = None


def load() -> C.CDLL:
    """Load the in-tree libanima_hip.so (raises if it is absent)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m animaxs_amd.build` "
                               "(there is no CPU fallback)")
        lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = load().anima_last_error()
        raise AnimaError(status, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
