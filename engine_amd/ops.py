"""Torch-facing helpers over the kernel C ABI: device buffers come from
PyTorch, every computation runs in the hip backend's own kernels."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import lib as L


def _p(a):
    if isinstance(a, np.ndarray):
        return a.ctypes.data_as(C.c_void_p)
    if isinstance(a, torch.Tensor):
        return C.c_void_p(a.data_ptr())
    return a


def stream_ptr(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def quantize(w, mode):
    """Host load-time quantizer of the backend: (codes int8 [n,k], scales fp16 bits)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    codes = np.empty((n, k), np.int8)
    lib = L.kernels()
    if mode == "int4":
        scales = np.empty((n, (k + 31) // 32), np.uint16)
        L.check("lyk_q4_quantize", lib.lyk_q4_quantize(_p(w), n, k, _p(codes), _p(scales)))
    elif mode == "int8":
        scales = np.empty((n,), np.uint16)
        L.check("lyk_q8_quantize", lib.lyk_q8_quantize(_p(w), n, k, _p(codes), _p(scales)))
    else:
        raise ValueError(mode)
    return codes, scales


def layout_bytes(n, k, mode, paired=False):
    wb, sb = C.c_uint64(), C.c_uint64()
    fn = L.kernels().lyk_q4_layout if mode == "int4" else L.kernels().lyk_q8_layout
    L.check("layout", fn(n, k, int(paired), C.byref(wb), C.byref(sb)))
    return wb.value, sb.value


def pack(codes, scales, mode, b_codes=None, b_scales=None):
    """Host repack into the device layout; returns (qw, qs) numpy byte arrays."""
    n, k = codes.shape
    wb, sb = layout_bytes(n, k, mode, b_codes is not None)
    qw = np.empty(wb, np.uint8)
    qs = np.empty(sb, np.uint8)
    fn = L.kernels().lyk_q4_pack if mode == "int4" else L.kernels().lyk_q8_pack
    rc = fn(_p(np.ascontiguousarray(codes)), _p(np.ascontiguousarray(scales)),
            None if b_codes is None else _p(np.ascontiguousarray(b_codes)),
            None if b_scales is None else _p(np.ascontiguousarray(b_scales)), n, k, _p(qw), _p(qs))
    L.check("pack", rc)
    return qw, qs


class PackedWeight:
    """A quantized [n, k] matrix (or an A/B pair) resident on the device."""

    def __init__(self, mode, n, k, qw, qs, paired=False, device="cuda"):
        self.mode, self.n, self.k, self.paired = mode, n, k, paired
        self.qw = torch.from_numpy(qw).to(device)
        self.qs = torch.from_numpy(qs).to(device)

    @classmethod
    def from_codes(cls, mode, codes, scales, b_codes=None, b_scales=None, device="cuda"):
        qw, qs = pack(codes, scales, mode, b_codes, b_scales)
        n, k = codes.shape
        return cls(mode, n, k, qw, qs, b_codes is not None, device)

    @classmethod
    def from_float(cls, mode, w, b=None, device="cuda"):
        codes, scales = quantize(w, mode)
        bc = bs = None
        if b is not None:
            bc, bs = quantize(b, mode)
        return cls.from_codes(mode, codes, scales, bc, bs, device)

    @property
    def nbytes(self):
        return self.qw.numel() + self.qs.numel()

    def unpack(self, stream=None):
        rows = self.n * (2 if self.paired else 1)
        codes = torch.empty((rows, self.k), dtype=torch.int8, device=self.qw.device)
        ns = (self.k + 31) // 32 if self.mode == "int4" else 1
        scales = torch.empty((rows, ns), dtype=torch.int16, device=self.qw.device)
        fn = L.kernels().lyk_hip_q4_unpack if self.mode == "int4" else L.kernels().lyk_hip_q8_unpack
        L.check("unpack", fn(_p(self.qw), _p(self.qs), self.n, self.k, int(self.paired), _p(codes),
                             _p(scales), stream_ptr(stream)))
        return codes, scales

    def dequant(self, stream=None):
        rows = self.n * (2 if self.paired else 1)
        w = torch.empty((rows, self.k), dtype=torch.float32, device=self.qw.device)
        fn = L.kernels().lyk_hip_q4_dequant if self.mode == "int4" else L.kernels().lyk_hip_q8_dequant
        L.check("dequant", fn(_p(self.qw), _p(self.qs), self.n, self.k, int(self.paired), _p(w),
                              stream_ptr(stream)))
        return w


class Workspace:
    """Zero-initialised device scratch for split-K partials and counters."""

    def __init__(self, nbytes=64 << 20, device="cuda"):
        self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)

    @property
    def nbytes(self):
        return self.buf.numel()


_ws = {}


def default_workspace(device="cuda"):
    if device not in _ws:
        _ws[device] = Workspace(device=device)
    return _ws[device]


def gemv(pw: PackedWeight, x, epilogue=L.EPI_STORE, y=None, bias=None, splits=0,
         workspace=None, stream=None):
    """y = W x for x fp16 [m, ldx] on the device (see lyk_hip_gemv_q4)."""
    m, ldx = x.shape
    assert x.dtype == torch.float16 and x.is_contiguous()
    if y is None:
        if epilogue == L.EPI_SILU_F16 or epilogue == L.EPI_STORE_F16:
            y = torch.empty((m, pw.n), dtype=torch.float16, device=x.device)
        else:
            y = torch.empty((m, pw.n), dtype=torch.float32, device=x.device)
    ws = workspace or default_workspace(str(x.device))
    fn = L.kernels().lyk_hip_gemv_q4 if pw.mode == "int4" else L.kernels().lyk_hip_gemv_q8
    rc = fn(_p(pw.qw), _p(pw.qs), pw.n, pw.k, _p(x), ldx, m, epilogue, _p(y), y.shape[1],
            None if bias is None else _p(bias), splits, _p(ws.buf), ws.nbytes, stream_ptr(stream))
    L.check("gemv", rc)
    return y


def padded_k(k, mode):
    unit = 32 if mode == "int4" else 16
    return (k + unit - 1) // unit * unit


class Rng:
    """The generator Sampler draws from (core/generation/sampler.cpp:32-33):
    std::mt19937_64 seeded with the request's seed, one
    generate_canonical<double, 53> per non-greedy token."""

    def __init__(self, seed):
        self._h = L.kernels().lyk_rng_new(int(seed))

    def canonical(self):
        return float(L.kernels().lyk_rng_canonical(self._h))

    def close(self):
        if self._h:
            L.kernels().lyk_rng_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


def sample(logits, temperature, top_k, top_p, u, workspace=None):
    """Device sampling of each row of `logits` ([m, n] fp32 on the GPU),
    Sampler::Sample's rule with the given draws u (one per row). Returns the
    tokens as an int32 tensor on the device (-1: a non-finite logit)."""
    assert logits.dtype == torch.float32 and logits.dim() == 2 and logits.is_cuda
    m, n = logits.shape
    ld = logits.stride(0)
    assert logits.stride(1) == 1 and len(u) == m
    k = L.kernels()
    need = k.lyk_hip_sample_workspace_bytes(m, n)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=logits.device)
    out = torch.empty(m, dtype=torch.int32, device=logits.device)
    draws = (C.c_double * m)(*u)
    L.check("lyk_hip_sample", k.lyk_hip_sample(_p(logits), ld, m, n, float(temperature), int(top_k),
                                                float(top_p), draws, _p(out), _p(workspace), need,
                                                stream_ptr()))
    return out


def pack_tiled(codes, scales, mode, tile_rows, b_codes=None, b_scales=None):
    """The fused step's tiled layout of one matrix, or of the pair (codes, b)
    when b_codes is given (gate and up): (qw, qs) uint8 arrays."""
    n, k = codes.shape
    q8 = mode == "int8"
    paired = b_codes is not None
    wb, sb = C.c_uint64(), C.c_uint64()
    lay = L.kernels().lyk_q8_layout_tiled if q8 else L.kernels().lyk_q4_layout_tiled
    L.check("layout_tiled", lay(n, k, 1 if paired else 0, tile_rows, C.byref(wb), C.byref(sb)))
    qw = np.zeros(wb.value, np.uint8)
    qs = np.zeros(sb.value, np.uint8)
    pack = L.kernels().lyk_q8_pack_tiled if q8 else L.kernels().lyk_q4_pack_tiled
    bc = np.ascontiguousarray(b_codes) if paired else None
    bs = np.ascontiguousarray(b_scales) if paired else None
    L.check("pack_tiled", pack(_p(np.ascontiguousarray(codes)), _p(np.ascontiguousarray(scales)),
                               _p(bc) if paired else None, _p(bs) if paired else None, n, k, tile_rows, _p(qw),
                               _p(qs)))
    return qw, qs


GEMM_STORE, GEMM_ADD, GEMM_SILU_PAIRS = 0, 1, 2


def gemm_q(x, qw, qs, n, mode, tile_rows, bias=None, epilogue=GEMM_STORE, y=None):
    """The prefill GEMM on the matrix cores; x fp16 [T, K] on the GPU (row
    stride a multiple of 8), qw / qs the tiled layout on the GPU. STORE: Y[T,
    n] = X . W^T (+ bias), fp32; ADD: y += X . W^T into the given fp32 y;
    SILU_PAIRS: W paired (gate and up, n rows each), fp16 SiLU(gate) * up."""
    assert x.dtype == torch.float16 and x.dim() == 2 and x.stride(1) == 1
    T, K = x.shape
    if y is None:
        assert epilogue != GEMM_ADD
        dt = torch.float16 if epilogue == GEMM_SILU_PAIRS else torch.float32
        y = torch.empty(T, n, dtype=dt, device=x.device)
    assert y.stride(1) == 1 and y.shape[0] == T
    L.check("lyk_hip_gemm_q", L.kernels().lyk_hip_gemm_q(_p(x), x.stride(0), T, K, _p(qw), _p(qs), n, tile_rows,
                                                         1 if mode == "int8" else 0, epilogue,
                                                         _p(bias) if bias is not None else None, _p(y), y.stride(0),
                                                         stream_ptr()))
    return y


def chunk_rope_kv(qkv, pos0, nq, nkv, hd, cos, sin, kcache, vcache, table, block_tokens):
    """Chunk prefill RoPE + KV append (lyk_hip_chunk_rope_kv): qkv fp32 [T,
    (nq+2nkv)*hd] at positions pos0..; returns q rotated, fp32 [T, nq*hd]; K/V
    go into the caches (fp16, [blocks][nkv][bt][hd] and [blocks][nkv][hd][bt])
    through table (int32 block ids). cos/sin fp32 [max_pos, hd/2]."""
    T = qkv.shape[0]
    q = torch.empty(T, nq * hd, dtype=torch.float32, device=qkv.device)
    L.check("lyk_hip_chunk_rope_kv", L.kernels().lyk_hip_chunk_rope_kv(
        _p(qkv), qkv.stride(0), T, pos0, nq, nkv, hd, _p(cos), _p(sin), cos.shape[0], _p(q), _p(kcache),
        _p(vcache), _p(table), table.numel(), block_tokens, kcache.shape[0], stream_ptr()))
    return q


def chunk_attention(q, pos0, nq, nkv, hd, kcache, vcache, table, block_tokens):
    """Chunk prefill causal attention (lyk_hip_chunk_attention): fp16 [T, nq*hd]."""
    T = q.shape[0]
    out = torch.empty(T, nq * hd, dtype=torch.float16, device=q.device)
    L.check("lyk_hip_chunk_attention", L.kernels().lyk_hip_chunk_attention(
        _p(q), _p(kcache), _p(vcache), _p(table), table.numel(), T, pos0, nq, nkv, hd, block_tokens,
        kcache.shape[0], _p(out), out.stride(0), stream_ptr()))
    return out
