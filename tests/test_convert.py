"""Offline-quantized artifacts (engine_amd/convert.py) on the CPU: the
converter stores the loader's own codes and scales in the on-wire form, and
the hip backend's safetensors reader takes the U8 / I8 tensors (the allowlist
extension of model/loader/safetensors.h:21) while refusing them as floating
point weights."""
import os

import numpy as np
import pytest

from engine_amd import convert as CV
from engine_amd import model as M
from engine_amd import ops
from oracle import oracle as O
from tests.model_pairs import fill_synthetic

SMALL = O.QwenConfig(256, 64, 2, 4, 2, 16, 96, 64, 1e-6, 1e6, False, 255)


def _unpack4(qw, n, k):
    b = np.frombuffer(qw, np.uint8).reshape(n, (k + 1) // 2)
    nib = np.empty((n, 2 * b.shape[1]), np.int16)
    nib[:, 0::2] = b & 15
    nib[:, 1::2] = b >> 4
    return (nib[:, :k] - 8).astype(np.int8)


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("dtype", ["F32", "BF16"])
def test_converted_codes_are_the_loaders(tmp_path, mode, dtype):
    src = O.OracleModel(SMALL)
    fill_synthetic(src, seed=3)
    path = str(tmp_path / "m.safetensors")
    O.write_safetensors(path, {O.tensor_name(k, l): a for k, l, a in src.tensors()}, dtype=dtype)
    dst = str(tmp_path / "q.safetensors")
    CV.convert(path, dst, mode)
    tensors, meta = CV.read_safetensors(dst)
    orig, _ = CV.read_safetensors(path)
    assert meta["lykuro_quant"] == ("int4_g32" if mode == "int4" else "int8_row")
    gemv = [n for n in orig if CV._GEMV.match(n)]
    assert len(gemv) == 7 * SMALL.num_layers + 1
    for name in gemv:
        base = name[: -len(".weight")]
        assert name not in tensors
        w = CV.as_f32(*orig[name])
        codes, scales = ops.quantize(w, mode)
        dt, shape, raw = tensors[base + ".qweight"]
        n, k = w.shape
        if mode == "int4":
            assert dt == "U8" and shape == [n, (k + 1) // 2]
            got = _unpack4(raw, n, k)
        else:
            assert dt == "I8" and shape == [n, k]
            got = np.frombuffer(raw, np.int8).reshape(n, k)
        assert np.array_equal(got, codes)
        sdt, sshape, sraw = tensors[base + ".qscale"]
        assert sdt == "F16" and sshape == list(scales.shape)
        assert np.array_equal(np.frombuffer(sraw, np.uint16).reshape(scales.shape), scales)
    for name in orig:
        if not CV._GEMV.match(name):
            assert tensors[name] == orig[name]
    # the reader takes the file; the quantized tensors are not float weights
    assert M.read_tensor_f32(dst, "model.norm.weight")[0] == M.OK
    assert M.read_tensor_f32(dst, "lm_head.qweight")[0] == M.ARTIFACT_VERIFICATION_FAILED


def test_odd_k_int4_pads_the_last_nibble(tmp_path):
    w = (np.random.default_rng(0).standard_normal((5, 37)) * 0.02).astype(np.float32)
    t = CV.quantized_tensors("x", w, "int4")
    dt, shape, raw = t["x.qweight"]
    assert shape == [5, 19]
    assert np.array_equal(_unpack4(raw, 5, 37), ops.quantize(w, "int4")[0])
    assert all(b >> 4 == 8 for b in np.frombuffer(raw, np.uint8).reshape(5, 19)[:, -1])


def test_reader_accepts_u8_i8_and_checks_their_size(tmp_path):
    from tests.test_loader import write
    ok = {"a": {"dtype": "U8", "shape": [3, 5], "data_offsets": [0, 15]},
          "b": {"dtype": "I8", "shape": [4], "data_offsets": [15, 19]},
          "c": {"dtype": "F32", "shape": [1], "data_offsets": [19, 23]}}
    p = write(tmp_path / "u8.safetensors", ok, bytes(23))
    assert M.read_tensor_f32(p, "c")[0] == M.OK
    assert M.read_tensor_f32(p, "a")[0] == M.ARTIFACT_VERIFICATION_FAILED
    bad = {"a": {"dtype": "U8", "shape": [3, 5], "data_offsets": [0, 16]}}
    assert M.read_tensor_f32(write(tmp_path / "bad.safetensors", bad, bytes(16)), "a")[0] == \
        M.ARTIFACT_VERIFICATION_FAILED
