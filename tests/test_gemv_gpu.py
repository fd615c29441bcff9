"""GPU parity of the weight-only GEMV kernels against the CPU oracle.

Bar: unpack and dequant bit-exact; GEMV outputs within
1e-3 norm-relative (||y - y_ref|| / ||y_ref||) of the oracle's fp32 MatVec on
the dequantized weights, with the same fp16-rounded activations fed to both
sides; bit-identical run to run."""
import numpy as np
import pytest
import torch

import engine_amd.lib as L
from engine_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3  # norm-relative, north_star per-op bar


def rel_err(y, ref):
    return float(np.linalg.norm(y.astype(np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def weights(seed, n, k, sigma=0.02):
    return (np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32) * sigma)


def acts(seed, m, k, ldx):
    x = np.zeros((m, ldx), np.float32)
    x[:, :k] = np.random.default_rng(seed).standard_normal((m, k), dtype=np.float32)
    return O.round_f16(x)


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("n,k,paired", [(1, 16, False), (70, 100, False), (303, 16, False),
                                        (18944, 3584, False), (96, 18944, False), (33, 72, True),
                                        (4096, 3584, True)])
def test_unpack_and_dequant_bit_exact(cuda, mode, n, k, paired):
    a = weights(n + k, n, k)
    b = weights(n + k + 1, n, k) if paired else None
    ca, sa = O.q4_quantize(a) if mode == "int4" else O.q8_quantize(a)
    cb, sb = (O.q4_quantize(b) if mode == "int4" else O.q8_quantize(b)) if paired else (None, None)
    pw = ops.PackedWeight.from_codes(mode, ca, sa, cb, sb)
    codes, scales = pw.unpack()
    want_c = np.concatenate([ca, cb]) if paired else ca
    want_s = np.concatenate([sa, sb]) if paired else sa
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint16).reshape(want_s.shape), want_s)
    deq = pw.dequant().cpu().numpy()
    want = (O.q4_dequantize if mode == "int4" else O.q8_dequantize)(want_c, want_s)
    assert np.array_equal(deq.view(np.uint32), want.view(np.uint32))


SHAPES = [(1, 16), (70, 100), (303, 16), (129, 40), (4608, 3584), (18944, 3584), (3584, 18944)]


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("n,k", SHAPES)
def test_gemv_matches_oracle(cuda, mode, m, n, k):
    w = weights(7 * n + k, n, k)
    deq = O.quant_dequant(w, mode)
    pw = ops.PackedWeight.from_float(mode, w)
    ldx = ops.padded_k(k, mode) + (32 if k > 1000 else 0)
    x = acts(m * 13 + k, m, k, ldx)
    xd = torch.from_numpy(x.astype(np.float16)).to(cuda)
    y = ops.gemv(pw, xd).cpu().numpy()
    for i in range(m):
        ref = O.matvec(deq, x[i, :k], threads=8)
        e = rel_err(y[i], ref)
        assert e < TOL, f"row {i}: norm-relative error {e:.3e}"


def test_gemv_lm_head_shape(cuda):
    n, k = 152064, 3584
    w = weights(99, n, k)
    deq = O.quant_dequant(w, "int4")
    pw = ops.PackedWeight.from_float("int4", w)
    x = acts(5, 1, k, k)
    y = ops.gemv(pw, torch.from_numpy(x.astype(np.float16)).to(cuda)).cpu().numpy()[0]
    ref = O.matvec(deq, x[0], threads=8)
    assert rel_err(y, ref) < TOL
    assert int(np.argmax(y)) == int(np.argmax(ref))


@pytest.mark.parametrize("mode", ["int4", "int8"])
def test_epilogues(cuda, mode):
    n, k, m = 200, 320, 3
    w = weights(1, n, k)
    g = weights(2, n, k)
    deq, gdeq = O.quant_dequant(w, mode), O.quant_dequant(g, mode)
    x = acts(3, m, k, k)
    xd = torch.from_numpy(x.astype(np.float16)).to(cuda)
    bias = np.random.default_rng(4).standard_normal(n).astype(np.float32)
    pw = ops.PackedWeight.from_float(mode, w)
    refs = [O.matvec(deq, x[i]) for i in range(m)]
    # store + bias (CPU order: bias first, then the products)
    y = ops.gemv(pw, xd, bias=torch.from_numpy(bias).to(cuda)).cpu().numpy()
    for i in range(m):
        assert rel_err(y[i], O.matvec(deq, x[i], bias)) < TOL
    # residual add
    h0 = np.random.default_rng(5).standard_normal((m, n)).astype(np.float32)
    h = torch.from_numpy(h0.copy()).to(cuda)
    ops.gemv(pw, xd, L.EPI_ADD, y=h)
    hh = h.cpu().numpy()
    for i in range(m):
        assert rel_err(hh[i] - h0[i], refs[i]) < TOL
    # fp16 store
    y16 = ops.gemv(pw, xd, L.EPI_STORE_F16).cpu().numpy().astype(np.float32)
    for i in range(m):
        assert rel_err(y16[i], refs[i]) < TOL
    # paired gate/up with SiLU-gate: a = silu(G x) * (W x)
    pp = ops.PackedWeight.from_float(mode, g, w)
    a = ops.gemv(pp, xd, L.EPI_SILU_F16).cpu().numpy().astype(np.float32)
    for i in range(m):
        gv = O.matvec(gdeq, x[i])
        ref = gv / (1.0 + np.exp(-gv)) * refs[i]
        assert rel_err(a[i], ref) < TOL


@pytest.mark.parametrize("mode", ["int4", "int8"])
def test_split_counts_agree_and_runs_are_deterministic(cuda, mode):
    n, k = 3584, 18944
    w = weights(11, n, k)
    pw = ops.PackedWeight.from_float(mode, w)
    x = acts(12, 1, k, k)
    xd = torch.from_numpy(x.astype(np.float16)).to(cuda)
    ref = O.matvec(O.quant_dequant(w, mode), x[0], threads=8)
    base = ops.gemv(pw, xd).cpu().numpy()[0]
    for splits in (1, 2, 3, 4, 8, 64, 1000):
        y = ops.gemv(pw, xd, splits=splits).cpu().numpy()[0]
        assert rel_err(y, ref) < TOL, splits
        again = ops.gemv(pw, xd, splits=splits).cpu().numpy()[0]
        assert np.array_equal(y.view(np.uint32), again.view(np.uint32)), splits
    again = ops.gemv(pw, xd).cpu().numpy()[0]
    assert np.array_equal(base.view(np.uint32), again.view(np.uint32))
