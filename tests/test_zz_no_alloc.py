"""The allocation-free sampler entry point (lyk_hip_sample_static, scratch in
a static device array) against the entry point with a caller workspace
(lyk_hip_sample), through the C ABI: the same tokens (integers, so bit for
bit), on two calls in a row, the second with a smaller input; rows past the
static scratch are refused."""
import ctypes as C

import numpy as np
import pytest
import torch

import engine_amd.lib as L
from engine_amd import ops

pytestmark = pytest.mark.gpu


def _p(t):
    return C.c_void_p(t.data_ptr())


def _both(logits, temperature, top_k, top_p, u):
    k = L.kernels()
    m, n = logits.shape
    draws = (C.c_double * m)(*u)
    ws = torch.empty(k.lyk_hip_sample_workspace_bytes(m, n), dtype=torch.uint8, device="cuda")
    a = torch.full((m,), -7, dtype=torch.int32, device="cuda")
    b = torch.full((m,), -7, dtype=torch.int32, device="cuda")
    L.check("lyk_hip_sample", k.lyk_hip_sample(_p(logits), logits.stride(0), m, n, temperature, top_k, top_p,
                                                draws, _p(a), _p(ws), ws.numel(), ops.stream_ptr()))
    L.check("lyk_hip_sample_static", k.lyk_hip_sample_static(_p(logits), logits.stride(0), m, n, temperature,
                                                              top_k, top_p, draws, _p(b), ops.stream_ptr()))
    torch.cuda.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


def test_static_scratch_sampler_equals_workspace_sampler(cuda):
    rng = np.random.default_rng(17)
    # first call: 4 rows at the 7B vocabulary; second: 2 shorter rows (the
    # static scratch still holds the first call's keys)
    for m, n, t, k, p in [(4, 152064, 0.8, 0, 0.9), (2, 40000, 1.0, 40, 0.95)]:
        logits = torch.from_numpy((rng.standard_normal((m, n)) * 2.5).astype(np.float32)).cuda()
        u = [float(v) for v in rng.random(m)]
        a, b = _both(logits, t, k, p, u)
        assert (a >= 0).all() and np.array_equal(a, b), (m, n, a, b)


def test_static_scratch_refuses_rows_beyond_it(cuda):
    k = L.kernels()
    n = (1 << 18) + 1
    logits = torch.zeros((1, n), dtype=torch.float32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    draws = (C.c_double * 1)(0.5)
    rc = k.lyk_hip_sample_static(_p(logits), n, 1, n, 1.0, 0, 0.9, draws, _p(out), ops.stream_ptr())
    assert rc == 2   # LYK_ERR_SHAPE
