"""Prefill GEMM on the matrix cores (lyk_hip_gemm_q) against the CPU product
of the same fp16 activations and the dequantized weights (the oracle's
MatVec per row, model/architectures/qwen/qwen_model.cpp:21-31), with each of
its epilogues: store (+ bias), add into y (the residual), and the paired
gate/up SiLU(gate) * up in fp16.

Bar: every product is exact (fp16 activations times integer codes; int4 group
and int8 row scales multiply the sums), so the result differs from the fp64
product on the dequantized weights by fp32 accumulation only: TOL = 2e-6
norm-relative per row (a few fp32 ulps of a sum of thousands of terms; an
int4 weight rounded to fp16 before the product, 2^-12 relative, fails it).
The SiLU epilogue rounds its product to fp16 once: half an fp16 ulp (plus
the sums' error) per element. Bit-identical run to run."""
import numpy as np
import pytest
import torch

from engine_amd import ops

pytestmark = pytest.mark.gpu

TOL = 2e-6


def dequant(codes, scales, mode):
    s = scales.view(np.float16).astype(np.float64)
    c = codes.astype(np.float64)
    if mode == "int8":
        return c * s[:, None]
    return c * np.repeat(s, 32, axis=1)[:, : c.shape[1]]


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("tr", [16, 32, 64])
@pytest.mark.parametrize("T,n,k", [(1, 64, 32), (17, 70, 100), (128, 256, 512), (300, 96, 3584), (64, 4608, 896)])
def test_gemm_matches_dequantized_product(cuda, mode, tr, T, n, k):
    g = np.random.default_rng(T * 131 + n + k + tr)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    codes, scales = ops.quantize(w, mode)
    qw, qs = ops.pack_tiled(codes, scales, mode, tr)
    kp = (k + 7) // 8 * 8
    x = np.zeros((T, kp), np.float16)
    x[:, :k] = g.standard_normal((T, k)).astype(np.float16)
    bias = g.standard_normal(n).astype(np.float32)
    xd = torch.from_numpy(x).cuda()[:, :k]
    y = ops.gemm_q(xd, torch.from_numpy(qw).cuda(), torch.from_numpy(qs).cuda(), n, mode, tr,
                   torch.from_numpy(bias).cuda()).cpu().numpy()
    ref = x[:, :k].astype(np.float64) @ dequant(codes, scales, mode)[:, :k].T + bias
    err = np.linalg.norm(y - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    assert err.max() < TOL, err.max()
    y2 = ops.gemm_q(xd, torch.from_numpy(qw).cuda(), torch.from_numpy(qs).cuda(), n, mode, tr,
                    torch.from_numpy(bias).cuda()).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def _problem(seed, T, n, k, mode, tr, paired=False):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    codes, scales = ops.quantize(w, mode)
    bc = bs = None
    if paired:
        wb = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
        bc, bs = ops.quantize(wb, mode)
    qw, qs = ops.pack_tiled(codes, scales, mode, tr, bc, bs)
    kp = (k + 7) // 8 * 8
    x = np.zeros((T, kp), np.float16)
    x[:, :k] = g.standard_normal((T, k)).astype(np.float16)
    xd = torch.from_numpy(x).cuda()[:, :k]
    a = x[:, :k].astype(np.float64) @ dequant(codes, scales, mode)[:, :k].T
    b = x[:, :k].astype(np.float64) @ dequant(bc, bs, mode)[:, :k].T if paired else None
    return g, xd, torch.from_numpy(qw).cuda(), torch.from_numpy(qs).cuda(), a, b


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("tr", [16, 32, 64])
@pytest.mark.parametrize("T,n,k", [(17, 70, 100), (130, 256, 896)])
def test_gemm_add_epilogue_accumulates_into_y(cuda, mode, tr, T, n, k):
    """ADD: y += X . W^T over a strided y (ldy > n); the columns past n keep
    their values."""
    g, xd, qw, qs, a, _ = _problem(T * 7 + n + tr, T, n, k, mode, tr)
    y0 = g.standard_normal((T, n + 5)).astype(np.float32)
    y = torch.from_numpy(y0).cuda()
    ops.gemm_q(xd, qw, qs, n, mode, tr, epilogue=ops.GEMM_ADD, y=y[:, :n])
    got = y.cpu().numpy()
    ref = y0[:, :n].astype(np.float64) + a
    err = np.linalg.norm(got[:, :n] - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    assert err.max() < 4 * TOL, err.max()
    assert np.array_equal(got[:, n:], y0[:, n:])


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("tr", [16, 32, 64])
@pytest.mark.parametrize("T,n,k", [(5, 40, 64), (129, 200, 512), (64, 1184, 3584)])
def test_gemm_silu_pairs_epilogue(cuda, mode, tr, T, n, k):
    """SILU_PAIRS over the paired (gate, up) layout against the STORE
    epilogue's fp32 sums of the gate and up matrices packed alone (the same
    sums bit for bit: each output's arithmetic depends only on its own row's
    codes and scales): fp16(SiLU(gate) * up) within half an fp16 ulp of the
    fp64 value of those sums, plus the fp32 evaluation of x / (1 + exp(-x))
    times up, as the fused step's gate/up epilogue computes it."""
    g = np.random.default_rng(T * 11 + n + tr)
    wa = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    ca, sa = ops.quantize(wa, mode)
    cb, sb = ops.quantize(wb, mode)
    dev = lambda a: torch.from_numpy(a).cuda()
    kp = (k + 7) // 8 * 8
    x = np.zeros((T, kp), np.float16)
    x[:, :k] = g.standard_normal((T, k)).astype(np.float16)
    xd = dev(x)[:, :k]
    gate = ops.gemm_q(xd, *map(dev, ops.pack_tiled(ca, sa, mode, tr)), n, mode, tr).cpu().numpy()
    up = ops.gemm_q(xd, *map(dev, ops.pack_tiled(cb, sb, mode, tr)), n, mode, tr).cpu().numpy()
    qw, qs = map(dev, ops.pack_tiled(ca, sa, mode, tr, cb, sb))
    got = ops.gemm_q(xd, qw, qs, n, mode, tr, epilogue=ops.GEMM_SILU_PAIRS).cpu().numpy().astype(np.float64)
    g64, u64 = gate.astype(np.float64), up.astype(np.float64)
    ref = g64 / (1.0 + np.exp(-g64)) * u64
    bound = np.abs(ref) * (2.0 ** -11 + 1e-6) + 3e-8
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))
