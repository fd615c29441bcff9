"""Prefill GEMM on the matrix cores (lyk_hip_gemm_q) against the CPU product
of the same fp16 activations and the dequantized weights (the oracle's
MatVec per row, model/architectures/qwen/qwen_model.cpp:21-31).

Bar (per-op): within 1e-3 norm-relative of the fp32
result on the dequantized weights, per row; bit-identical run to run. The
matrix product is exact in its inputs (fp16 activations, integer codes), so
the difference is fp32 accumulation order only."""
import numpy as np
import pytest
import torch

from engine_amd import ops

pytestmark = pytest.mark.gpu

TOL = 1e-3


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
