"""ctypes bindings for the hip backend's C ABI (include/lykuro_hip.h and
include/lykuro_hip_model.h).

The libraries are built in-tree by engine_amd/build.py. Loading fails loudly
when they are missing: there is no CPU or PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import torch  # noqa: F401  -- load PyTorch's HIP runtime first, so one runtime serves both

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
KERNEL_LIB = os.path.join(PKG, "liblykuro_hip.so")
MODEL_LIB = os.path.join(PKG, "liblykuro_hip_model.so")
HEADERS = [os.path.join(ROOT, "include", "lykuro_hip.h"),
           os.path.join(ROOT, "include", "lykuro_hip_model.h")]

P, I, I64, U16, U32, U64, F = (C.c_void_p, C.c_int, C.c_int64, C.c_uint16, C.c_uint32,
                               C.c_uint64, C.c_float)

STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported shape", 3: "workspace too small",
          4: "kernel launch failed", 5: "HIP runtime error"}

EPI_STORE, EPI_ADD, EPI_STORE_F16, EPI_SILU_F16 = 0, 1, 2, 3


class LykError(RuntimeError):
    def __init__(self, fn, code):
        super().__init__(f"{fn} failed: {STATUS.get(code, code)} ({code})")
        self.code = code


_KERNEL_SIGS = {
    "lyk_abi_version": (I, []),
    "lyk_q4_layout": (I, [I64, I64, I, C.POINTER(U64), C.POINTER(U64)]),
    "lyk_q8_layout": (I, [I64, I64, I, C.POINTER(U64), C.POINTER(U64)]),
    "lyk_q4_quantize": (I, [P, I64, I64, P, P]),
    "lyk_q8_quantize": (I, [P, I64, I64, P, P]),
    "lyk_q4_pack": (I, [P, P, P, P, I64, I64, P, P]),
    "lyk_q8_pack": (I, [P, P, P, P, I64, I64, P, P]),
    "lyk_q4_layout_tiled": (I, [I64, I64, I, I, C.POINTER(U64), C.POINTER(U64)]),
    "lyk_q8_layout_tiled": (I, [I64, I64, I, I, C.POINTER(U64), C.POINTER(U64)]),
    "lyk_q4_pack_tiled": (I, [P, P, P, P, I64, I64, I, P, P]),
    "lyk_q8_pack_tiled": (I, [P, P, P, P, I64, I64, I, P, P]),
    "lyk_q4_unpack_tiled": (I, [P, P, I64, I64, I, I, P, P]),
    "lyk_q8_unpack_tiled": (I, [P, P, I64, I64, I, I, P, P]),
    "lyk_hip_q4_unpack": (I, [P, P, I64, I64, I, P, P, P]),
    "lyk_hip_q8_unpack": (I, [P, P, I64, I64, I, P, P, P]),
    "lyk_hip_q4_dequant": (I, [P, P, I64, I64, I, P, P]),
    "lyk_hip_q8_dequant": (I, [P, P, I64, I64, I, P, P]),
    "lyk_hip_gemv_workspace_bytes": (U64, [I64, I64, I, I, I, I]),
    "lyk_hip_rmsnorm_f16": (I, [P, I64, P, F, I, I64, P, I64, P]),
    "lyk_hip_embed_rmsnorm": (I, [P, I64, P, I, I64, P, I64, P, F, P, I64, P]),
    "lyk_hip_rope_kv_append": (I, [P, I64, I, I, I, I, P, P, P, I, P, P, P, P, I, I, I, P]),
    "lyk_hip_attn_workspace_bytes": (U64, [I, I, I, I, I]),
    "lyk_hip_attn_decode": (I, [P, P, P, P, I, P, I, I, I, I, I, I, I, P, I64, P, U64, P]),
    "lyk_hip_argmax_workspace_bytes": (U64, [I, I64]),
    "lyk_hip_argmax": (I, [P, I64, I, I64, P, P, P, P, P, P, U64, P]),
    "lyk_hip_gemm_q": (I, [P, I64, I64, I64, P, P, I64, I, I, I, P, P, I64, P]),
    "lyk_hip_chunk_rope_kv": (I, [P, I64, I, I, I, I, I, P, P, I, P, P, P, P, I, I, I, P]),
    "lyk_hip_chunk_attention": (I, [P, P, P, P, I, I, I, I, I, I, I, I, P, I64, P]),
    "lyk_hip_sample_workspace_bytes": (U64, [I, I64]),
    "lyk_hip_sample": (I, [P, I64, I, I64, C.c_float, C.c_int32, C.c_float, P, P, P, U64, P]),
    "lyk_hip_sample_static": (I, [P, I64, I, I64, C.c_float, C.c_int32, C.c_float, P, P, P]),
    "lyk_rng_new": (P, [U64]),
    "lyk_rng_free": (None, [P]),
    "lyk_rng_canonical": (C.c_double, [P]),
    "lyk_hip_gemv_splits": (I, [I64, I64, I, I, I]),
    "lyk_hip_gemv_q4": (I, [P, P, I64, I64, P, I64, I, I, P, I64, P, I, P, U64, P]),
    "lyk_hip_gemv_q8": (I, [P, P, I64, I64, P, I64, I, I, P, I64, P, I, P, U64, P]),
    "lyk_hip_step_workspace_bytes": (U64, [P, I]),
    "lyk_hip_step_phases": (U32, [P, I]),
    "lyk_hip_step_grid": (I, []),
    "lyk_hip_step_tile_rows": (I, [I64, I64, I, I, I]),
    "lyk_hip_decode_step": (I, [P, P, P, U64, I, P]),
    "lyk_hip_step_reset": (I, [P, U64, P]),
    "lyk_hip_step_error": (I, [P, C.POINTER(C.c_int32), P]),
    "lyk_hip_step_launches": (U64, [P]),
    "lyk_hip_step_set_launches": (I, [P, I, P, U64, U64, P]),
}

class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "vocab_size", "hidden_size", "num_layers", "num_heads", "num_kv_heads", "head_dim",
        "intermediate_size", "max_context_tokens")] + [
        ("rms_norm_eps", C.c_double), ("rope_theta", C.c_double),
        ("tie_word_embeddings", C.c_int32), ("eos_token_id", C.c_uint32)]


class ModelOptions(C.Structure):
    _fields_ = [("device_id", C.c_int32), ("kv_pool_tokens", C.c_uint32),
                ("kv_block_tokens", C.c_uint32), ("quant", C.c_int32),
                ("attn_split_tokens", C.c_int32), ("attn_max_splits", C.c_int32),
                ("tile_rows", C.c_int32 * 5), ("lds_prefetch", C.c_int32),
                ("prefill_chunk", C.c_int32)]


I32P = C.POINTER(C.c_int32)
_MODEL_SIGS = {
    "lyk_model_load_safetensors": (P, [C.c_char_p, C.POINTER(ModelConfig), C.POINTER(ModelOptions), I32P]),
    "lyk_model_load_synthetic": (P, [C.POINTER(ModelConfig), U64, F, C.POINTER(ModelOptions), I32P]),
    "lyk_model_free": (None, [P]),
    "lyk_model_read_tensor_f32": (C.c_int32, [C.c_char_p, C.c_char_p, P, U64, C.POINTER(U64)]),
    "lyk_model_seq_new": (P, [P, U32, C.c_int32, C.c_char_p, I32P]),
    "lyk_model_seq_free": (None, [P]),
    "lyk_model_seq_length": (U32, [P]),
    "lyk_model_seq_capacity": (U32, [P]),
    "lyk_model_prefill": (C.c_int32, [P, P, P, C.c_size_t, P]),
    "lyk_model_decode": (C.c_int32, [P, P, U32, P]),
    "lyk_model_decode_batch": (C.c_int32, [P, P, P, C.c_size_t, P, P]),
    "lyk_model_greedy_run": (C.c_int32, [P, P, U32, U32, P, C.POINTER(U32)]),
    "lyk_model_kv_blocks_total": (U32, [P]),
    "lyk_model_kv_blocks_free": (U32, [P]),
    "lyk_model_prefix_cache_hit_tokens": (U64, [P]),
    "lyk_model_gemv_weight_bytes": (U64, [P]),
    "lyk_model_set_step_tracing": (C.c_int32, [P, C.c_int32]),
    "lyk_model_stream": (P, [P]),
    "lyk_model_step_trace": (C.c_size_t, [P, P, C.c_size_t]),
    "lyk_model_step_launches": (U64, [P]),
    "lyk_model_set_wait_limit": (None, [P, U32]),
    "lyk_model_set_step_launches": (C.c_int32, [P, U64]),
    "lyk_synth_normal": (None, [U64, U64, U64, U64, F, P]),
}

_kernels = None
_model = None


def _bind(lib, sigs):
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args


def kernels():
    """The kernel library (include/lykuro_hip.h)."""
    global _kernels
    if _kernels is None:
        if not os.path.exists(KERNEL_LIB):
            raise RuntimeError(
                f"{KERNEL_LIB} is missing: build it with `python -m engine_amd.build` "
                "(the hip backend has no fallback path)")
        lib = C.CDLL(KERNEL_LIB)
        _bind(lib, _KERNEL_SIGS)
        _kernels = lib
    return _kernels


def model_lib():
    """The host-model library (include/lykuro_hip_model.h)."""
    global _model
    if _model is None:
        kernels()  # its dependency, from the same directory
        if not os.path.exists(MODEL_LIB):
            raise RuntimeError(f"{MODEL_LIB} is missing: build it with `python -m engine_amd.build`")
        lib = C.CDLL(MODEL_LIB)
        _bind(lib, _MODEL_SIGS)
        _model = lib
    return _model


def declared_symbols(header):
    """Function names declared in one of the public headers."""
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lyk_[a-z0-9_]+)\s*\(", text)))


def check(fn, code):
    if code != 0:
        raise LykError(fn, code)
