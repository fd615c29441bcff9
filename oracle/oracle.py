"""ctypes view of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
leg, always as the checker; the product package (engine_amd) never imports
it. Wraps oracle/liboracle.so (the C restatement in qwen_oracle.c) and, where
it was built, oracle/_ref/libqwen_ref.so (the reference engine's own CPU path
compiled from its sources by oracle/Makefile).
"""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libqwen_ref.so")

# numeric values of the reference ErrorCode enum (core/engine/error.h:12-43)
OK, INVALID_REQUEST, CONTEXT_LENGTH_EXCEEDED = 0, 1, 6
CAPACITY_EXHAUSTED, INFERENCE_FAILED, INTERNAL_ERROR = 8, 15, 17

(T_EMBED, T_INPUT_NORM, T_Q_W, T_Q_B, T_K_W, T_K_B, T_V_W, T_V_B, T_O_W,
 T_POST_NORM, T_GATE_W, T_UP_W, T_DOWN_W, T_FINAL_NORM, T_LM_HEAD) = range(15)
LAYER_KINDS = range(T_INPUT_NORM, T_DOWN_W + 1)

# reference tensor names (model/architectures/qwen/qwen_model.cpp:170-198)
LAYER_NAMES = {
    T_INPUT_NORM: "input_layernorm.weight",
    T_Q_W: "self_attn.q_proj.weight", T_Q_B: "self_attn.q_proj.bias",
    T_K_W: "self_attn.k_proj.weight", T_K_B: "self_attn.k_proj.bias",
    T_V_W: "self_attn.v_proj.weight", T_V_B: "self_attn.v_proj.bias",
    T_O_W: "self_attn.o_proj.weight",
    T_POST_NORM: "post_attention_layernorm.weight",
    T_GATE_W: "mlp.gate_proj.weight", T_UP_W: "mlp.up_proj.weight",
    T_DOWN_W: "mlp.down_proj.weight",
}


@dataclass(frozen=True)
class QwenConfig:
    vocab_size: int
    hidden_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate_size: int
    max_context_tokens: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    tie_word_embeddings: bool = True
    eos_token_id: int = 0

    def shape(self, kind):
        h, q = self.hidden_size, self.num_heads * self.head_dim
        kv, i, v = self.num_kv_heads * self.head_dim, self.intermediate_size, self.vocab_size
        return {
            T_EMBED: (v, h), T_INPUT_NORM: (h,), T_POST_NORM: (h,), T_FINAL_NORM: (h,),
            T_Q_W: (q, h), T_Q_B: (q,), T_K_W: (kv, h), T_K_B: (kv,),
            T_V_W: (kv, h), T_V_B: (kv,), T_O_W: (h, q),
            T_GATE_W: (i, h), T_UP_W: (i, h), T_DOWN_W: (h, i),
            T_LM_HEAD: None if self.tie_word_embeddings else (v, h),
        }[kind]


# tests/testutil/tiny_model.h:9-20 and the parity fixture of
# tests/cuda/cuda_parity_test.cpp:48-51 (vocab 303, eos 302, context 128)
TINY = QwenConfig(32, 16, 2, 4, 2, 4, 32, 64, 1e-6, 10000.0, True, 31)
TINY_PARITY = QwenConfig(303, 16, 2, 4, 2, 4, 32, 128, 1e-6, 10000.0, True, 302)
# BASELINE configs
QWEN05B = QwenConfig(151936, 896, 24, 14, 2, 64, 4864, 32768, 1e-6, 1e6, True, 151643)
QWEN7B = QwenConfig(152064, 3584, 28, 28, 4, 128, 18944, 32768, 1e-6, 1e6, False, 151643)
QWEN14B = QwenConfig(152064, 5120, 48, 40, 8, 128, 13824, 32768, 1e-6, 1e6, False, 151643)


class _Config(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "vocab_size", "hidden_size", "num_layers", "num_heads", "num_kv_heads",
        "head_dim", "intermediate_size", "max_context_tokens")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float),
        ("tie_word_embeddings", C.c_int32)]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P, u16, u32, u64, i64 = C.c_void_p, C.c_uint16, C.c_uint32, C.c_uint64, C.c_int64
        sig = {
            "orc_f16_to_f32": (C.c_float, [u16]), "orc_f32_to_f16": (u16, [C.c_float]),
            "orc_bf16_to_f32": (C.c_float, [u16]), "orc_f32_to_bf16": (u16, [C.c_float]),
            "orc_f16_to_f32_array": (None, [P, P, C.c_size_t]),
            "orc_f32_to_f16_array": (None, [P, P, C.c_size_t]),
            "orc_q4_quantize": (None, [P, i64, i64, P, P]),
            "orc_q4_dequantize": (None, [P, P, i64, i64, P]),
            "orc_q8_quantize": (None, [P, i64, i64, P, P]),
            "orc_q8_dequantize": (None, [P, P, i64, i64, P]),
            "orc_quant_scale_f16": (u16, [C.c_float, C.c_float]),
            "orc_matvec": (None, [P, P, P, i64, i64, P]),
            "orc_matvec_mt": (None, [P, P, P, i64, i64, P, C.c_int]),
            "orc_rmsnorm": (None, [P, P, C.c_float, i64, P]),
            "orc_rope": (None, [P, u32, u32, C.c_float]),
            "orc_attention": (None, [P, P, P, u32, u32, u32, u32, P]),
            "orc_attention_mt": (None, [P, P, P, u32, u32, u32, u32, P, C.c_int]),
            "orc_model_new": (P, [C.POINTER(_Config)]),
            "orc_model_free": (None, [P]),
            "orc_model_tensor": (C.POINTER(C.c_float), [P, C.c_int, u32]),
            "orc_model_tensor_numel": (u64, [P, C.c_int]),
            "orc_model_set_threads": (None, [P, C.c_int]),
            "orc_model_set_f16_mirror": (None, [P, C.c_int]),
            "orc_model_set_descending_sums": (None, [P, C.c_int]),
            "orc_seq_new": (P, [P, u32]), "orc_seq_free": (None, [P]),
            "orc_seq_length": (u32, [P]),
            "orc_prefill": (C.c_int, [P, P, P, C.c_size_t, P]),
            "orc_decode": (C.c_int, [P, P, u32, P]),
            "orc_fill_tiny_weights": (None, [P, u64]),
            "orc_sampler_new": (P, [C.c_float, C.c_float, u32, u64]),
            "orc_sampler_free": (None, [P]),
            "orc_sample": (C.c_int, [P, P, C.c_size_t, C.POINTER(u32)]),
            "orc_argmax": (u32, [P, C.c_size_t]),
            "orc_mt64_seed": (None, [P, u64]), "orc_mt64_next": (u64, [P]),
            "orc_mt64_canonical": (C.c_double, [P]),
            "orc_synth_normal": (None, [u64, u64, u64, u64, C.c_float, P]),
            "orc_synth_tokens": (None, [u64, u64, u64, u32, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_LIB_PATH)


def ref_lib():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_LIB_PATH)
        P, u16, u32, u64 = C.c_void_p, C.c_uint16, C.c_uint32, C.c_uint64
        sig = {
            "ref_f16_to_f32": (C.c_float, [u16]), "ref_f32_to_f16": (u16, [C.c_float]),
            "ref_bf16_to_f32": (C.c_float, [u16]), "ref_f32_to_bf16": (u16, [C.c_float]),
            "ref_model_load": (P, [C.c_char_p] + [u32] * 8 + [C.c_double, C.c_double, C.c_int, u32,
                                                             C.POINTER(C.c_int32)]),
            "ref_model_free": (None, [P]), "ref_seq_new": (P, [P, u32]), "ref_seq_free": (None, [P]),
            "ref_prefill": (C.c_int32, [P, P, P, C.c_size_t, P]),
            "ref_decode": (C.c_int32, [P, P, u32, P]),
            "ref_sampler_new": (P, [C.c_float, C.c_float, u32, u64]),
            "ref_sampler_free": (None, [P]),
            "ref_sample": (C.c_int32, [P, P, C.c_size_t, C.POINTER(u32)]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _ref = L
    return _ref


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- codecs
def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def round_f16(x):
    return f16_bits_to_f32(f32_to_f16_bits(x))


# ------------------------------------------------------------ quantizers
def _by_rows(n, k, call):
    """call(a, b) over row blocks [a, b) in parallel; the quantizers work row
    by row, so the result equals one call over all rows."""
    futs = [_pool().submit(call, a, b) for a, b in _split(n, max(1, (1 << 20) // max(1, k))) if b > a]
    for f in futs:
        f.result()


def _rp(x, a):
    """Pointer to row a of x."""
    return C.c_void_p(x.ctypes.data + a * x.strides[0])


def q4_quantize(w):
    """int4 g32 fp16-scale codes [N,K] int8 and scales [N,ceil(K/32)] fp16 bits."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    codes = np.empty((n, k), np.int8)
    scales = np.empty((n, (k + 31) // 32), np.uint16)
    _by_rows(n, k, lambda a, b: lib().orc_q4_quantize(_rp(w, a), b - a, k, _rp(codes, a), _rp(scales, a)))
    return codes, scales


def q4_dequantize(codes, scales):
    n, k = codes.shape
    out = np.empty((n, k), np.float32)
    codes, scales = np.ascontiguousarray(codes), np.ascontiguousarray(scales)
    _by_rows(n, k, lambda a, b: lib().orc_q4_dequantize(_rp(codes, a), _rp(scales, a), b - a, k, _rp(out, a)))
    return out


def q8_quantize(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    codes = np.empty((n, k), np.int8)
    scales = np.empty((n,), np.uint16)
    _by_rows(n, k, lambda a, b: lib().orc_q8_quantize(_rp(w, a), b - a, k, _rp(codes, a), _rp(scales, a)))
    return codes, scales


def q8_dequantize(codes, scales):
    n, k = codes.shape
    out = np.empty((n, k), np.float32)
    codes, scales = np.ascontiguousarray(codes), np.ascontiguousarray(scales)
    _by_rows(n, k, lambda a, b: lib().orc_q8_dequantize(_rp(codes, a), _rp(scales, a), b - a, k, _rp(out, a)))
    return out


def quant_dequant(w, mode):
    if mode == "int4":
        return q4_dequantize(*q4_quantize(w))
    if mode == "int8":
        return q8_dequantize(*q8_quantize(w))
    raise ValueError(mode)


# ------------------------------------------------------------ primitives
def matvec(w, x, bias=None, threads=1):
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, k = w.shape
    out = np.empty(n, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_matvec_mt(_p(w), None if b is None else _p(b), _p(x), k, n, _p(out), threads)
    return out


def rmsnorm(x, weight, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    wt = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(wt), eps, x.size, _p(out))
    return out


def rope(vec, pos, theta):
    v = np.array(vec, dtype=np.float32)
    lib().orc_rope(_p(v), v.size, pos, theta)
    return v


def attention(q, keys, values, heads, kv_heads, head_dim, threads=1):
    q = np.ascontiguousarray(q, dtype=np.float32)
    keys = np.ascontiguousarray(keys, dtype=np.float32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(heads * head_dim, np.float32)
    if threads > 1:
        lib().orc_attention_mt(_p(q), _p(keys), _p(values), keys.shape[0], heads, kv_heads,
                               head_dim, _p(out), threads)
    else:
        lib().orc_attention(_p(q), _p(keys), _p(values), keys.shape[0], heads, kv_heads,
                            head_dim, _p(out))
    return out


_POOL = None


def _pool():
    """Worker threads for the row- or element-independent helpers below
    (ctypes releases the GIL around each C call)."""
    global _POOL
    if _POOL is None:
        from concurrent.futures import ThreadPoolExecutor
        _POOL = ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1)))
    return _POOL


def _split(total, min_piece):
    n = max(1, min(_pool()._max_workers, total // max(1, min_piece)))
    return [(total * i // n, total * (i + 1) // n) for i in range(n)]


def synth_normal(seed, stream, count, sigma, first=0):
    """Value i depends only on (seed, stream, first + i): chunks computed in
    parallel equal the serial stream."""
    out = np.empty(count, np.float32)
    parts = _split(count, 1 << 20)
    futs = [_pool().submit(lib().orc_synth_normal, seed, stream, first + a, b - a, sigma,
                           out[a:b].ctypes.data_as(C.c_void_p)) for a, b in parts if b > a]
    for f in futs:
        f.result()
    return out


def synth_tokens(seed, stream, count, n):
    out = np.empty(count, np.uint32)
    lib().orc_synth_tokens(seed, stream, count, n, _p(out))
    return out


# ----------------------------------------------------------------- model
class OracleModel:
    """The restated QwenModel: fp32 weights, token-by-token forward."""

    def __init__(self, cfg: QwenConfig, threads=1):
        self.cfg = cfg
        c = _Config(cfg.vocab_size, cfg.hidden_size, cfg.num_layers, cfg.num_heads,
                    cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size,
                    cfg.max_context_tokens, cfg.rms_norm_eps, cfg.rope_theta,
                    int(cfg.tie_word_embeddings))
        self._h = lib().orc_model_new(C.byref(c))
        if not self._h:
            raise MemoryError("oracle model allocation failed")
        lib().orc_model_set_threads(self._h, threads)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.orc_model_free(self._h)
            self._h = None

    def tensor(self, kind, layer=0):
        shape = self.cfg.shape(kind)
        if shape is None:
            return None
        ptr = lib().orc_model_tensor(self._h, kind, layer)
        return np.ctypeslib.as_array(ptr, shape=shape)

    def tensors(self):
        """(kind, layer, array view) for every tensor of the model."""
        out = [(T_EMBED, 0, self.tensor(T_EMBED))]
        for l in range(self.cfg.num_layers):
            out += [(k, l, self.tensor(k, l)) for k in LAYER_KINDS]
        out.append((T_FINAL_NORM, 0, self.tensor(T_FINAL_NORM)))
        if not self.cfg.tie_word_embeddings:
            out.append((T_LM_HEAD, 0, self.tensor(T_LM_HEAD)))
        return out

    def fill_tiny(self, seed=42):
        lib().orc_fill_tiny_weights(self._h, seed)

    def set_threads(self, n):
        lib().orc_model_set_threads(self._h, n)

    def set_f16_mirror(self, on):
        lib().orc_model_set_f16_mirror(self._h, int(on))

    def set_descending_sums(self, on):
        lib().orc_model_set_descending_sums(self._h, int(on))

    def new_seq(self, max_tokens):
        return _Seq(self, max_tokens)

    def prefill(self, seq, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros(self.cfg.vocab_size, np.float32)
        code = lib().orc_prefill(self._h, seq._h, _p(t), t.size, _p(logits))
        return code, logits

    def decode(self, seq, token):
        logits = np.zeros(self.cfg.vocab_size, np.float32)
        code = lib().orc_decode(self._h, seq._h, int(token), _p(logits))
        return code, logits


class _Seq:
    def __init__(self, model, max_tokens):
        self._m = model
        self._h = lib().orc_seq_new(model._h, max_tokens)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.orc_seq_free(self._h)
            self._h = None

    @property
    def length(self):
        return lib().orc_seq_length(self._h)


class Sampler:
    """The restated Sampler (core/generation/sampler.cpp:35-106)."""

    def __init__(self, temperature=1.0, top_p=1.0, top_k=0, seed=0):
        self._h = lib().orc_sampler_new(temperature, top_p, top_k, seed)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_sampler_free(self._h)
            self._h = None

    def sample(self, logits):
        l = np.ascontiguousarray(logits, dtype=np.float32)
        out = C.c_uint32(0)
        code = lib().orc_sample(self._h, _p(l), l.size, C.byref(out))
        return code, out.value


def argmax(logits):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().orc_argmax(_p(l), l.size)


# ----------------------------------------------------- safetensors writer
def tensor_name(kind, layer):
    if kind == T_EMBED:
        return "model.embed_tokens.weight"
    if kind == T_FINAL_NORM:
        return "model.norm.weight"
    if kind == T_LM_HEAD:
        return "lm_head.weight"
    return f"model.layers.{layer}.{LAYER_NAMES[kind]}"


def write_safetensors(path, tensors, dtype="F32"):
    """Writes {name: float32 array} in byte-lexicographic name order with
    contiguous offsets (the layout tests/testutil/tiny_model.cpp:80-114 writes
    and model/loader/safetensors.cpp accepts). dtype F32, F16 or BF16."""
    names = sorted(tensors)
    header, off, blobs = {}, 0, []
    for n in names:
        a = np.ascontiguousarray(tensors[n], dtype=np.float32)
        if dtype == "F32":
            b = a.tobytes()
        elif dtype == "F16":
            b = f32_to_f16_bits(a).tobytes()
        elif dtype == "BF16":
            b = np.array([lib().orc_f32_to_bf16(float(v)) for v in a.ravel()],
                         np.uint16).tobytes()
        else:
            raise ValueError(dtype)
        header[n] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    hj = json.dumps(header, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(len(hj).to_bytes(8, "little"))
        f.write(hj)
        for b in blobs:
            f.write(b)


def model_to_safetensors(model: OracleModel, path):
    write_safetensors(path, {tensor_name(k, l): a for k, l, a in model.tensors()})


class RefModel:
    """The reference engine's own QwenModel (oracle/_ref), loaded from a file."""

    def __init__(self, cfg: QwenConfig, path):
        code = C.c_int32(0)
        self.cfg = cfg
        self._h = ref_lib().ref_model_load(
            path.encode(), cfg.vocab_size, cfg.hidden_size, cfg.num_layers, cfg.num_heads,
            cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size, cfg.max_context_tokens,
            cfg.rms_norm_eps, cfg.rope_theta, int(cfg.tie_word_embeddings),
            cfg.eos_token_id, C.byref(code))
        if not self._h:
            raise RuntimeError(f"reference load failed with code {code.value}")

    def __del__(self):
        if getattr(self, "_h", None):
            ref_lib().ref_model_free(self._h)
            self._h = None

    def new_seq(self, max_tokens):
        return _RefSeq(max_tokens, self)

    def prefill(self, seq, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros(self.cfg.vocab_size, np.float32)
        return ref_lib().ref_prefill(self._h, seq._h, _p(t), t.size, _p(logits)), logits

    def decode(self, seq, token):
        logits = np.zeros(self.cfg.vocab_size, np.float32)
        return ref_lib().ref_decode(self._h, seq._h, int(token), _p(logits)), logits


class _RefSeq:
    def __init__(self, max_tokens, model):
        self._h = ref_lib().ref_seq_new(model._h, max_tokens)

    def __del__(self):
        if getattr(self, "_h", None):
            ref_lib().ref_seq_free(self._h)
            self._h = None


class RefSampler:
    def __init__(self, temperature=1.0, top_p=1.0, top_k=0, seed=0):
        self._h = ref_lib().ref_sampler_new(temperature, top_p, top_k, seed)

    def __del__(self):
        if getattr(self, "_h", None):
            ref_lib().ref_sampler_free(self._h)
            self._h = None

    def sample(self, logits):
        l = np.ascontiguousarray(logits, dtype=np.float32)
        out = C.c_uint32(0)
        code = ref_lib().ref_sample(self._h, _p(l), l.size, C.byref(out))
        return code, out.value
