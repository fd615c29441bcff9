"""The hip backend's safetensors reader and dtype widening, on the CPU
(through lyk_model_read_tensor_f32: the loader's own reader and widening,
no device).

Cases follow the reference reader's tests (tests/unit/safetensors_test.cpp:
23-166) and the checks of model/loader/safetensors.cpp:160-297 (regular file,
no symlink, rank <= 8, a non-empty tensor map); widening of F16/BF16 is
checked exhaustively against the oracle's codecs, themselves pinned by the
reference's KATs (tests/unit/dtype_test.cpp:10-55)."""
import json
import os
import struct

import numpy as np
import pytest

from engine_amd import model as M
from oracle import oracle as O

TWO = {"a": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]},
       "b": {"dtype": "F32", "shape": [4], "data_offsets": [16, 32]},
       "__metadata__": {"format": "pt"}}


def write(path, header, data: bytes, raw_header=None):
    h = raw_header if raw_header is not None else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        f.write(data)
    return str(path)


def read(path, name="a"):
    return M.read_tensor_f32(str(path), name)


def test_opens_valid_file(tmp_path):
    data = bytearray(32)
    data[0:4] = struct.pack("<f", 1.5)
    p = write(tmp_path / "ok.safetensors", TWO, bytes(data))
    code, a = read(p)
    assert code == M.OK and a.tolist() == [1.5, 0.0, 0.0, 0.0]
    assert read(p, "missing")[0] == M.ARTIFACT_VERIFICATION_FAILED


@pytest.mark.parametrize("header,size", [
    ({"a": {"dtype": "I64", "shape": [2], "data_offsets": [0, 16]}}, 16),           # dtype allow-list
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, 8),            # out of bounds
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]},
      "b": {"dtype": "F32", "shape": [4], "data_offsets": [8, 24]}}, 24),           # overlap
    ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
      "b": {"dtype": "F32", "shape": [2], "data_offsets": [16, 24]}}, 24),          # gap
    ({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, 16),           # size mismatch
    ({"a": {"dtype": "F32", "shape": [4294967295] * 3, "data_offsets": [0, 16]}}, 16),  # overflow
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16], "extra": 1}}, 16),   # extra field
    ({}, 0),                                                                         # no tensors
    ({"__metadata__": {"format": "pt"}}, 0),                                         # still none
    ({"a": {"dtype": "F32", "shape": [1] * 8 + [4], "data_offsets": [0, 16]}}, 16),  # rank 9 > 8
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, 32),           # trailing data
], ids=["dtype", "out_of_bounds", "overlap", "gap", "size_mismatch", "overflow", "extra_field",
        "empty", "metadata_only", "rank9", "trailing"])
def test_rejects_bad_headers(tmp_path, header, size):
    p = write(tmp_path / "bad.safetensors", header, bytes(size))
    assert read(p)[0] == M.ARTIFACT_VERIFICATION_FAILED


def test_rank_eight_is_accepted(tmp_path):
    p = write(tmp_path / "r8.safetensors",
              {"a": {"dtype": "F32", "shape": [1] * 7 + [4], "data_offsets": [0, 16]}}, bytes(16))
    assert read(p)[0] == M.OK


def test_rejects_truncated_data_and_header_length(tmp_path):
    assert read(write(tmp_path / "t.safetensors", TWO, bytes(16)))[0] == M.ARTIFACT_VERIFICATION_FAILED
    p = tmp_path / "h.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 20))
    assert read(p)[0] == M.ARTIFACT_VERIFICATION_FAILED
    q = tmp_path / "short.safetensors"
    q.write_bytes(b"\x01\x02")
    assert read(q)[0] == M.ARTIFACT_VERIFICATION_FAILED


def test_rejects_missing_file_symlink_fifo_and_directory(tmp_path):
    assert read(tmp_path / "does_not_exist.st")[0] == M.ARTIFACT_VERIFICATION_FAILED
    good = write(tmp_path / "ok.safetensors", TWO, bytes(32))
    link = tmp_path / "link.safetensors"
    os.symlink(good, link)
    assert read(link)[0] == M.ARTIFACT_VERIFICATION_FAILED      # symlinks refused
    fifo = tmp_path / "fifo.safetensors"
    os.mkfifo(fifo)
    assert read(fifo)[0] == M.ARTIFACT_VERIFICATION_FAILED      # and it does not block
    assert read(tmp_path)[0] == M.ARTIFACT_VERIFICATION_FAILED  # a directory


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
def test_widening_is_exhaustive_bit_exact(tmp_path, dtype):
    """Every 16-bit pattern (subnormals, infinities, NaNs, -0 included) widens
    to the oracle codec's fp32 bits."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    p = write(tmp_path / f"{dtype}.safetensors",
              {"a": {"dtype": dtype, "shape": [256, 256], "data_offsets": [0, 1 << 17]}}, bits.tobytes())
    code, got = read(p)
    assert code == M.OK
    if dtype == "F16":
        want = O.f16_bits_to_f32(bits)
    else:
        want = (bits.astype(np.uint32) << 16).view(np.float32)
        # the oracle's scalar codec agrees on a sample (it is pinned by the KATs)
        for b in (0x0000, 0x8000, 0x3F80, 0x7F80, 0xFF80, 0x7FC0, 0x0001, 0x807F, 0x4049):
            assert np.float32(O.lib().orc_bf16_to_f32(b)).view(np.uint32) == np.uint32(b) << 16
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
