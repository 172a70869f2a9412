"""Loads libmyl_hip.so (built in-tree by myelith_amd.build) and declares its C ABI.

The library is required: there is no fallback path.  Import fails loudly if
the shared object is missing, so a silently substituted implementation can
never stand in for the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmyl_hip.so"

P = C.c_void_p
u8, i8, i16, i32, i64, u32, u64, sz = (C.c_uint8, C.c_int8, C.c_int16, C.c_int32, C.c_int64, C.c_uint32,
                                        C.c_uint64, C.c_size_t)
INT = C.c_int

MYL_OK, MYL_E_INVALID, MYL_E_HIP, MYL_E_NOMEM, MYL_E_UNSUPPORTED = 0, -1, -2, -3, -4


class SynthSpec(C.Structure):
    """myl_synth_spec (include/myl_theta_v.h)."""
    _fields_ = [("seed", u64), ("vocab", u32), ("hidden", u32), ("layers", u32), ("heads", u32),
                ("kv_heads", u32), ("head_dim", u32), ("inter", u32), ("max_pos", u32),
                ("lm_head_int16", i32), ("attention_bias", i32)]


class MoeSpec(C.Structure):
    """myl_moe_spec (include/myl_theta_v.h)."""
    _fields_ = [("seed", u64), ("hidden", u32), ("n_experts", u32), ("inter", u32), ("top_k", u32),
                ("shared_inter", u32)]


class LayerFracs(C.Structure):
    """myl_layer_fracs (include/myl_theta_v.h): LayerScales of model.rs."""
    _fields_ = [("norm_attn_frac", u8), ("q_frac", u8), ("k_frac", u8), ("v_frac", u8), ("attn_out_frac", u8),
                ("norm_mlp_frac", u8), ("gate_frac", u8), ("up_frac", u8), ("down_in_frac", u8)]


class ModelDims(C.Structure):
    """myl_model_dims (include/myl_theta_v.h): ModelDims of loader.rs."""
    _fields_ = [("vocab", u32), ("hidden", u32), ("layers", u32), ("heads", u32), ("kv_heads", u32),
                ("head_dim", u32), ("inter", u32), ("max_context", u32), ("tie_word_embeddings", i32),
                ("attention_bias", i32), ("lm_head_int16", i32)]


class Luts(C.Structure):
    """myl_luts (include/myl_theta_v.h)."""
    _fields_ = [("rsqrt", P), ("rsqrt_len", sz), ("silu", P), ("silu_len", sz), ("exp", P),
                ("exp_len", sz), ("cos", P), ("sin", P), ("rope_len", sz)]


# name -> (restype, argtypes); the exported symbol set of include/myl_hip.h.
SIGNATURES: dict[str, tuple] = {
    "myl_backend_name": (C.c_char_p, []),
    "myl_hardware_family": (C.c_char_p, []),
    "myl_feature_tag": (C.c_char_p, []),
    "myl_init": (INT, [INT, C.POINTER(P)]),
    "myl_destroy": (None, [P]),
    "myl_last_error": (C.c_char_p, [P]),
    "myl_device_info": (INT, [P, C.c_char_p, sz, C.POINTER(INT), C.POINTER(u64)]),
    "myl_synchronize": (INT, [P]),
    "myl_stream": (P, [P]),
    "myl_set_stream": (INT, [P, P]),
    "myl_read_probe": (INT, [P, P, sz, P]),
    "myl_malloc": (INT, [P, sz, C.POINTER(P)]),
    "myl_free": (INT, [P, P]),
    "myl_memcpy_htod": (INT, [P, P, P, sz]),
    "myl_memcpy_dtoh": (INT, [P, P, P, sz]),
    "myl_linear_w8a16": (INT, [P, P, P, P, sz, sz, P, u8, u8]),
    "myl_linear_w8a16_pc": (INT, [P, P, P, P, sz, sz, P, u8, P]),
    "myl_add_bias_i16": (INT, [P, P, P, P, sz, u8]),
    "myl_rmsnorm": (INT, [P, P, P, P, P, sz, P, sz, u8, u8, i64, P, u8]),
    "myl_softmax": (INT, [P, P, P, sz, P, sz, u8, u8]),
    "myl_attention": (INT, [P, P, P, P, P, sz, sz, sz, P, i64, u8, P, sz, u8, u8]),
    "myl_rope": (INT, [P, P, P, sz, sz, P, P, sz, P, u8]),
    "myl_mlp": (INT, [P, P, P, P, P, P, sz, sz, P, P, P, P, sz, u8, u8, u8, u8, u8, i16, u8, P]),
    "myl_argmax_int": (INT, [P, P, sz, C.POINTER(i64)]),
    "myl_sample_integer_cdf": (INT, [P, P, sz, u64, C.POINTER(i64), C.POINTER(u64)]),
    "myl_linear_w8a16_dev": (INT, [P, P, sz, sz, P, sz, sz, P, u8, u8, P, P, sz]),
    "myl_linear_w8a16_dev_noalloc": (INT, [P, P, sz, sz, P, sz, sz, P, u8, u8, P, P, sz]),
    "myl_noalloc_scratch_bytes": (sz, []),
    "myl_linear_w8a16_mult_dev": (INT, [P, P, sz, sz, P, sz, sz, P, P, P, sz]),
    "myl_logits_dev": (INT, [P, P, sz, sz, P, INT, sz, sz, P, u8, u8, P, sz]),
    "myl_dot_i8_i16_dev": (INT, [P, P, sz, sz, P, sz, sz, P, sz]),
    "myl_rmsnorm_dev": (INT, [P, P, sz, sz, P, P, P, sz, P, sz, u8, u8, i64, u8, P, sz]),
    "myl_softmax_dev": (INT, [P, P, sz, sz, sz, P, sz, u8, u8, P, sz]),
    "myl_argmax_dev": (INT, [P, P, sz, sz, sz, P]),
    "myl_sample_dev": (INT, [P, P, sz, sz, sz, P, P, P]),
    "myl_logsoftmax_dev": (INT, [P, P, sz, sz, sz, P, sz, P, P]),
    "myl_model_create_synthetic": (INT, [P, C.POINTER(SynthSpec), C.POINTER(Luts), C.POINTER(P)]),
    "myl_model_destroy": (None, [P]),
    "myl_model_reset": (INT, [P]),
    "myl_model_forward_token": (INT, [P, u32, u32, P, C.POINTER(i64)]),
    "myl_model_decode_greedy": (INT, [P, u32, u32, u32, P, P]),
    "myl_model_prefill": (INT, [P, P, u32, u32, P]),
    "myl_model_set_graphs": (INT, [P, INT]),
    "myl_model_set_kernel_repeat": (INT, [P, INT, INT]),
    "myl_model_timing": (INT, [P, INT, P, P]),
    "myl_model_embed_token": (INT, [P, u32, P]),
    "myl_model_run_layers": (INT, [P, P, u32, u32, u32]),
    "myl_model_head_logits": (INT, [P, P, P]),
    "myl_model_read_kv": (INT, [P, u32, u32, u32, P, P]),
    "myl_model_read_tensor": (INT, [P, C.c_char_p, u32, P, sz]),
    "myl_model_batch_begin": (INT, [P, u32]),
    "myl_model_forward_batch": (INT, [P, u32, P, P, P, P, P]),
    "myl_model_batch_logits_dev": (INT, [P, C.POINTER(P)]),
    "myl_model_batch_decode_greedy": (INT, [P, u32, P, P, P, u32, P]),
    "myl_model_batch_read_kv": (INT, [P, u32, u32, u32, u32, P, P]),
    "myl_moe_create_synthetic": (INT, [P, C.POINTER(MoeSpec), P, C.POINTER(Luts), C.POINTER(P)]),
    "myl_moe_destroy": (None, [P]),
    "myl_moe_synth_input": (INT, [P, u32, P]),
    "myl_moe_forward": (INT, [P, P, u32, P]),
    "myl_moe_read_route": (INT, [P, u32, P, P, P, P, P]),
    "myl_artifact_open": (INT, [C.c_char_p, C.POINTER(P), C.c_char_p, sz]),
    "myl_artifact_close": (None, [P]),
    "myl_artifact_last_error": (C.c_char_p, [P]),
    "myl_artifact_dims": (INT, [P, C.POINTER(ModelDims)]),
    "myl_artifact_verify": (INT, [P]),
    "myl_artifact_lut": (INT, [P, C.c_char_p, P, sz, C.POINTER(sz)]),
    "myl_artifact_layer_scales": (INT, [P, u32, C.POINTER(LayerFracs), P, P]),
    "myl_artifact_final_scales": (INT, [P, C.POINTER(u8), P]),
    "myl_sha256_hex": (INT, [P, sz, C.c_char_p]),
    "myl_model_load_artifact": (INT, [P, P, u32, C.POINTER(P)]),
    "myl_model_create": (INT, [P, C.POINTER(ModelDims), u32, C.POINTER(Luts), C.POINTER(P)]),
    "myl_model_upload_tensor": (INT, [P, C.c_char_p, P, INT, C.POINTER(u64), u32, P, sz]),
    "myl_model_download_tensor": (INT, [P, C.c_char_p, INT, P, sz, P, sz]),
    "myl_model_set_layer_scales": (INT, [P, u32, C.POINTER(LayerFracs), P, P]),
    "myl_model_set_final_scales": (INT, [P, u8, P]),
    "myl_model_get_layer_scales": (INT, [P, u32, C.POINTER(LayerFracs), P, P]),
    "myl_model_get_final_scales": (INT, [P, C.POINTER(u8), P]),
    "myl_model_finalize": (INT, [P]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m myelith_amd.build` "
                               "(there is no non-HIP fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
