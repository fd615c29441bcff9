"""Python handle over QwenHipModel through include/lykuro_hip_model.h.

Mirrors the engine's GenerativeModel operations (CreateSequence(Ex),
Prefill, Decode, DecodeBatch, GreedyRun) with numpy logits; status codes are
the engine's ErrorCode values."""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np

from . import lib as L

OK, INVALID_REQUEST, UNSUPPORTED_MODEL, ARTIFACT_VERIFICATION_FAILED = 0, 1, 4, 5
CONTEXT_LENGTH_EXCEEDED, CAPACITY_EXHAUSTED = 6, 8
GPU_OOM, GPU_UNHEALTHY, INFERENCE_FAILED, INTERNAL_ERROR = 13, 14, 15, 17


class ModelError(RuntimeError):
    def __init__(self, what, code):
        super().__init__(f"{what}: error code {code}")
        self.code = code


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class QwenConfig:
    """Qwen2 dense decoder shape; model/architectures/qwen/qwen_model.h:22-37
    (one eos id here: the hip model consults none on device)."""
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


# Qwen2.5-7B (config.json of the released checkpoint): 28 layers, 28 query and
# 4 KV heads of 128, SwiGLU 18944, vocab 152064, untied LM head.
QWEN25_7B = QwenConfig(152064, 3584, 28, 28, 4, 128, 18944, 32768, 1e-6, 1e6, False, 151643)
# Qwen2.5-14B: 48 layers, 40 query and 8 KV heads of 128, SwiGLU 13824.
QWEN25_14B = QwenConfig(152064, 5120, 48, 40, 8, 128, 13824, 32768, 1e-6, 1e6, False, 151643)


def _config(cfg):
    return L.ModelConfig(cfg.vocab_size, cfg.hidden_size, cfg.num_layers, cfg.num_heads,
                         cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size,
                         cfg.max_context_tokens, cfg.rms_norm_eps, cfg.rope_theta,
                         int(cfg.tie_word_embeddings), cfg.eos_token_id)


@dataclass
class Options:
    device_id: int = 0
    kv_pool_tokens: int = 0
    kv_block_tokens: int = 16
    quant: str = "int4"
    attn_split_tokens: int = 0   # 0: the kernel's defaults
    attn_max_splits: int = 0
    tile_rows: tuple = (0, 0, 0, 0, 0)   # qkv, o, gate/up, down, head; 0: device choice
    lds_prefetch: int = 0   # gate/up chunks per wave staged in LDS: 0 as many as fit, -1 none
    prefill_chunk: int = 0  # prompt rows per chunk pass: 0 = 2048, -1 = token by token (fused step)

    def c(self):
        return L.ModelOptions(self.device_id, self.kv_pool_tokens, self.kv_block_tokens,
                              1 if self.quant == "int8" else 0, self.attn_split_tokens,
                              self.attn_max_splits, (C.c_int32 * 5)(*self.tile_rows), self.lds_prefetch,
                              self.prefill_chunk)


class HipModel:
    def __init__(self, handle, cfg):
        self._h = handle
        self.cfg = cfg
        self.vocab = cfg.vocab_size
        self._seqs = weakref.WeakSet()

    @classmethod
    def from_safetensors(cls, path, cfg, options: Options = Options()):
        st = C.c_int32(0)
        h = L.model_lib().lyk_model_load_safetensors(path.encode(), C.byref(_config(cfg)),
                                                     C.byref(options.c()), C.byref(st))
        if not h:
            raise ModelError("load", st.value)
        return cls(h, cfg)

    @classmethod
    def synthetic(cls, cfg, seed=0, sigma=0.02, options: Options = Options()):
        st = C.c_int32(0)
        h = L.model_lib().lyk_model_load_synthetic(C.byref(_config(cfg)), seed, sigma,
                                                   C.byref(options.c()), C.byref(st))
        if not h:
            raise ModelError("load", st.value)
        return cls(h, cfg)

    def close(self):
        """Frees the model; sequences still open are freed first."""
        if getattr(self, "_h", None):
            for s in list(self._seqs):
                s.close()
            L.model_lib().lyk_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def new_seq(self, max_tokens, allow_prefix_cache=False, scope_key=""):
        st = C.c_int32(0)
        h = L.model_lib().lyk_model_seq_new(self._h, max_tokens, int(allow_prefix_cache),
                                            scope_key.encode(), C.byref(st))
        if not h:
            raise ModelError("create sequence", st.value)
        seq = Sequence(h, self)
        self._seqs.add(seq)
        return seq

    def prefill(self, seq, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros(self.vocab, np.float32)
        code = L.model_lib().lyk_model_prefill(self._h, seq._h, _p(t), t.size, _p(logits))
        return code, logits

    def decode(self, seq, token):
        logits = np.zeros(self.vocab, np.float32)
        code = L.model_lib().lyk_model_decode(self._h, seq._h, int(token), _p(logits))
        return code, logits

    def decode_batch(self, seqs, tokens):
        n = len(seqs)
        handles = (C.c_void_p * n)(*[s._h for s in seqs])
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros((n, self.vocab), np.float32)
        per = np.zeros(n, np.int32)
        code = L.model_lib().lyk_model_decode_batch(self._h, handles, _p(t), n, _p(logits), _p(per))
        return code, list(per), logits

    def greedy_run(self, seq, token, max_new):
        out = np.zeros(max(1, max_new), np.uint32)
        n = C.c_uint32(0)
        code = L.model_lib().lyk_model_greedy_run(self._h, seq._h, int(token), max_new, _p(out),
                                                  C.byref(n))
        return code, [int(v) for v in out[:n.value]]

    @property
    def kv_blocks_total(self):
        return L.model_lib().lyk_model_kv_blocks_total(self._h)

    @property
    def kv_blocks_free(self):
        return L.model_lib().lyk_model_kv_blocks_free(self._h)

    @property
    def prefix_cache_hit_tokens(self):
        return L.model_lib().lyk_model_prefix_cache_hit_tokens(self._h)

    @property
    def gemv_weight_bytes(self):
        return L.model_lib().lyk_model_gemv_weight_bytes(self._h)

    @property
    def stream_ptr(self):
        """hipStream_t of the model (for torch.cuda.ExternalStream)."""
        return L.model_lib().lyk_model_stream(self._h)

    @property
    def step_launches(self):
        """Fused-step launches since the step workspace was last zeroed."""
        return L.model_lib().lyk_model_step_launches(self._h)

    def set_step_launches(self, n):
        """Zeroes the step workspace and presets its launch count (tests of
        the 2^24 - 1 launch-tag limit)."""
        L.check("lyk_model_set_step_launches", L.model_lib().lyk_model_set_step_launches(self._h, n))

    def set_wait_limit(self, microseconds):
        """Bound of the fused step's waits for other workgroups (0: 2 s)."""
        L.model_lib().lyk_model_set_wait_limit(self._h, microseconds)

    def set_step_tracing(self, on=True):
        L.check("lyk_model_set_step_tracing", L.model_lib().lyk_model_set_step_tracing(self._h, int(on)))

    def step_trace(self, mode="greedy"):
        """Device timestamps (100 MHz ticks) of the latest step, per
        workgroup: [grid][2 + 4*phases] = entry, exit, then per phase
        (entered, inputs ready, main loop done, outputs written). `mode` is
        the mode the buffer was sized for (the largest, greedy)."""
        grid = L.kernels().lyk_hip_step_grid()
        nph = 5 * self.cfg.num_layers + 2
        n = grid * (4 * nph + 2)
        buf = (C.c_uint64 * n)()
        got = L.model_lib().lyk_model_step_trace(self._h, buf, n)
        return np.array(buf, dtype=np.int64)[:got]


class Sequence:
    def __init__(self, handle, model):
        self._h = handle
        self._model = model  # keep the model alive while the sequence lives

    def close(self):
        if getattr(self, "_h", None):
            L.model_lib().lyk_model_seq_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def length(self):
        return L.model_lib().lyk_model_seq_length(self._h)

    @property
    def capacity(self):
        return L.model_lib().lyk_model_seq_capacity(self._h)


def read_tensor_f32(path, name):
    """(status, fp32 array) of one tensor as the loader reads it (no GPU)."""
    n = C.c_uint64(0)
    code = L.model_lib().lyk_model_read_tensor_f32(path.encode(), name.encode(), None, 0, C.byref(n))
    if code != OK:
        return code, None
    out = np.empty(n.value, np.float32)
    code = L.model_lib().lyk_model_read_tensor_f32(path.encode(), name.encode(), _p(out), n.value, C.byref(n))
    return code, out


def synth_normal(seed, stream, count, sigma, first=0):
    out = np.empty(count, np.float32)
    L.model_lib().lyk_synth_normal(seed, stream, first, count, sigma, _p(out))
    return out
