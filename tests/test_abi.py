"""CPU-side checks of the C ABI: the libraries load and export every declared
entry point, the load-time quantizers equal the oracle's bit for bit, and the
packed layouts decode (by the rule written in include/lykuro_hip.h) to the
codes and scales they were made from. No kernel is launched here."""
import ctypes as C
import os

import numpy as np
import pytest

import engine_amd.lib as L
from engine_amd import ops
from oracle import oracle as O


def test_abi_version():
    assert L.kernels().lyk_abi_version() == 1


@pytest.mark.parametrize("header", L.HEADERS)
def test_every_declared_symbol_is_exported(header):
    if not os.path.exists(header):
        pytest.skip("header not present")
    path = L.KERNEL_LIB if header.endswith("lykuro_hip.h") else L.MODEL_LIB
    lib = C.CDLL(path)
    names = L.declared_symbols(header)
    assert names, "no declarations found"
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{os.path.basename(path)} lacks {missing}"


def _weights(rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[0, :] = 0.0                       # all-zero row
    if n > 2:
        w[1, : min(k, 32)] *= 1e-8      # fp16-subnormal scales
        w[2, :] *= 1e5                  # large values
    return w


@pytest.mark.parametrize("n,k", [(1, 1), (3, 16), (70, 100), (130, 3584), (64, 96)])
def test_q4_quantizer_equals_oracle(n, k):
    w = _weights(np.random.default_rng(n * 1000 + k), n, k)
    a_codes, a_scales = ops.quantize(w, "int4")
    b_codes, b_scales = O.q4_quantize(w)
    np.testing.assert_array_equal(a_codes, b_codes)
    np.testing.assert_array_equal(a_scales, b_scales)


@pytest.mark.parametrize("n,k", [(1, 1), (3, 16), (70, 100), (130, 3584)])
def test_q8_quantizer_equals_oracle(n, k):
    w = _weights(np.random.default_rng(n * 1000 + k + 7), n, k)
    a_codes, a_scales = ops.quantize(w, "int8")
    b_codes, b_scales = O.q8_quantize(w)
    np.testing.assert_array_equal(a_codes, b_codes)
    np.testing.assert_array_equal(a_scales, b_scales)


NIBBLE_POS = [0, 16, 4, 20, 8, 24, 12, 28]


def decode_q4(qw, qs, n, k, paired):
    """Reads the int4 layout exactly as include/lykuro_hip.h describes it."""
    tiles = (n + 31) // 32 if paired else (n + 63) // 64
    groups = (k + 31) // 32
    gp = (groups + 7) // 8 * 8
    words = qw.view(np.uint32).reshape(tiles, gp, 64, 4)
    sc = qs.view(np.uint16).reshape(tiles, gp // 8, 64, 8)
    rows = 2 * n if paired else n
    codes = np.zeros((rows, k), np.int8)
    scales = np.zeros((rows, groups), np.uint16)
    for t in range(tiles):
        for lane in range(64):
            if paired:
                r = t * 32 + (lane & 31)
                if r >= n:
                    continue
                r += n if lane >= 32 else 0
            else:
                r = t * 64 + lane
                if r >= n:
                    continue
            for g in range(groups):
                scales[r, g] = sc[t, g // 8, lane, g % 8]
                for d in range(4):
                    wd = int(words[t, g, lane, d])
                    for j in range(8):
                        kk = g * 32 + d * 8 + j
                        if kk < k:
                            codes[r, kk] = ((wd >> NIBBLE_POS[j]) & 0xF) - 8
    return codes, scales


def decode_q8(qw, qs, n, k, paired):
    tiles = (n + 31) // 32 if paired else (n + 63) // 64
    blocks = (k + 15) // 16
    bp = (blocks + 7) // 8 * 8
    by = qw.reshape(tiles, bp, 64, 16)
    sc = qs.view(np.uint16).reshape(tiles, 64)
    rows = 2 * n if paired else n
    codes = np.zeros((rows, k), np.int8)
    scales = np.zeros(rows, np.uint16)
    for t in range(tiles):
        for lane in range(64):
            if paired:
                r = t * 32 + (lane & 31)
                if r >= n:
                    continue
                r += n if lane >= 32 else 0
            else:
                r = t * 64 + lane
                if r >= n:
                    continue
            scales[r] = sc[t, lane]
            flat = by[t, :, lane, :].reshape(-1)[:k].astype(np.int32) - 128
            codes[r] = flat.astype(np.int8)
    return codes, scales


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("n,k,paired", [(5, 40, False), (70, 300, False), (33, 64, True), (7, 16, True)])
def test_pack_layout_round_trip(mode, n, k, paired):
    rng = np.random.default_rng(n + k)
    a = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.02).astype(np.float32) if paired else None
    ca, sa = ops.quantize(a, mode)
    cb, sb = ops.quantize(b, mode) if paired else (None, None)
    qw, qs = ops.pack(ca, sa, mode, cb, sb)
    dec = decode_q4 if mode == "int4" else decode_q8
    codes, scales = dec(qw, qs, n, k, paired)
    want_c = np.concatenate([ca, cb]) if paired else ca
    want_s = np.concatenate([sa, sb]) if paired else sa
    np.testing.assert_array_equal(codes, want_c)
    np.testing.assert_array_equal(scales, want_s.reshape(scales.shape))


def test_pack_padding_is_zero_code_zero_scale():
    """Padded groups/rows must contribute exactly 0 in the GEMV."""
    codes, scales = ops.quantize(np.ones((3, 40), np.float32), "int4")
    qw, qs = ops.pack(codes, scales, "int4")
    words = qw.view(np.uint32).reshape(1, 8, 64, 4)
    sc = qs.view(np.uint16).reshape(1, 1, 64, 8)
    assert np.all(sc[0, 0, 3:, :] == 0) and np.all(sc[0, 0, :3, 2:] == 0)
    assert np.all(words[0, 2:, :, :] == 0x88888888)
    assert np.all(words[0, :, 3:, :] == 0x88888888)


def test_invalid_arguments_rejected():
    lib = L.kernels()
    wb, sb = C.c_uint64(), C.c_uint64()
    assert lib.lyk_q4_layout(0, 10, 0, C.byref(wb), C.byref(sb)) == 1
    assert lib.lyk_q4_quantize(None, 1, 1, None, None) == 1
    # device entry points validate before touching memory
    x = np.zeros(64, np.uint16)
    assert lib.lyk_hip_gemv_q4(None, None, 64, 64, x.ctypes.data, 64, 1, 0, None, 64,
                               None, 0, None, 0, None) == 1
    assert lib.lyk_hip_gemv_q4(1, 1, 64, 64, 8, 64, 5, 0, 8, 64, None, 0, None, 0, None) == 1
    assert lib.lyk_hip_gemv_q4(1, 1, 64, 64, 8, 48, 1, 0, 8, 64, None, 0, None, 0, None) == 1


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("tr", [16, 32, 64])
@pytest.mark.parametrize("n,k,paired", [(1, 16, False), (70, 100, False), (45, 300, True), (96, 512, False),
                                        (33, 4160, True)])
def test_tiled_pack_round_trip(mode, tr, n, k, paired):
    """The fused step's tiled layouts: pack then unpack returns the codes and
    scales exactly, for every tile height, ragged n and k, paired or not."""
    lib = L.kernels()
    rng = np.random.default_rng(n * 7 + k + tr)
    q8 = mode == "int8"
    ns = 1 if q8 else (k + 31) // 32
    mats = []
    for _ in range(2 if paired else 1):
        w = rng.standard_normal((n, k)).astype(np.float32) * 0.02
        codes = np.zeros((n, k), np.int8)
        scales = np.zeros((n, ns), np.uint16)
        quant = lib.lyk_q8_quantize if q8 else lib.lyk_q4_quantize
        assert quant(w.ctypes.data, n, k, codes.ctypes.data, scales.ctypes.data) == 0
        mats.append((codes, scales))
    wb, sb = C.c_uint64(), C.c_uint64()
    layout = lib.lyk_q8_layout_tiled if q8 else lib.lyk_q4_layout_tiled
    assert layout(n, k, int(paired), tr, C.byref(wb), C.byref(sb)) == 0
    qw = np.full(wb.value, 0xAB, np.uint8)
    qs = np.full(sb.value, 0xCD, np.uint8)
    pack = lib.lyk_q8_pack_tiled if q8 else lib.lyk_q4_pack_tiled
    b = mats[1] if paired else (None, None)
    assert pack(mats[0][0].ctypes.data, mats[0][1].ctypes.data,
                b[0].ctypes.data if paired else None, b[1].ctypes.data if paired else None,
                n, k, tr, qw.ctypes.data, qs.ctypes.data) == 0
    rows = 2 * n if paired else n
    out_c = np.zeros((rows, k), np.int8)
    out_s = np.zeros((rows, ns), np.uint16)
    unpack = lib.lyk_q8_unpack_tiled if q8 else lib.lyk_q4_unpack_tiled
    assert unpack(qw.ctypes.data, qs.ctypes.data, n, k, int(paired), tr,
                  out_c.ctypes.data, out_s.ctypes.data) == 0
    want_c = np.concatenate([m[0] for m in mats])
    want_s = np.concatenate([m[1] for m in mats])
    assert np.array_equal(out_c, want_c)
    assert np.array_equal(out_s, want_s)
    # every byte of both buffers is written: packing over another fill
    # pattern gives the same bytes
    qw2 = np.full(wb.value, 0x12, np.uint8)
    qs2 = np.full(sb.value, 0x34, np.uint8)
    assert pack(mats[0][0].ctypes.data, mats[0][1].ctypes.data,
                b[0].ctypes.data if paired else None, b[1].ctypes.data if paired else None,
                n, k, tr, qw2.ctypes.data, qs2.ctypes.data) == 0
    assert np.array_equal(qw, qw2) and np.array_equal(qs, qs2)


def test_tiled_layout_rejects_bad_tile_rows():
    lib = L.kernels()
    wb, sb = C.c_uint64(), C.c_uint64()
    for tr in (0, 8, 48, 128):
        assert lib.lyk_q4_layout_tiled(64, 64, 0, tr, C.byref(wb), C.byref(sb)) == 1
