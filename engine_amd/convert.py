"""Offline quantization of a Qwen2 safetensors checkpoint for the hip backend.

  python -m engine_amd.convert IN.safetensors OUT.safetensors --quant int4|int8 [--head]

Every GEMV matrix (q/k/v/o projections, gate/up/down, the untied LM head) is
quantized with the backend's own load-time quantizer (lyk_q4_quantize /
lyk_q8_quantize, the same codes and scales the loader would compute) and
stored as two tensors in place of `<name>.weight`:

  int4  `<name>.qweight` U8 [n, ceil(k/2)]: code + 8 per nibble, even k in the
        low nibble; `<name>.qscale` F16 [n, ceil(k/32)] (groups of 32 along k)
  int8  `<name>.qweight` I8 [n, k]; `<name>.qscale` F16 [n] (per row)

Everything else (embedding, norms, biases) is copied as it is. With --head, a
model whose LM head is tied to the embedding also gets `lm_head.qweight` /
`lm_head.qscale` (the embedding stays, for the token gather). QwenHipModel
loads either form, matrix by matrix, and a converted file gives the logits of
its source bit for bit; the loader checks the codes' dtype against the model's
quantization option. This is the offline-quantized artifact of the reference's
next step (model/loader/safetensors.h:21 allowlist,
model/convert/hf_convert.cpp:266 precision), which skips load-time quantization.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import re
import struct

import numpy as np

from engine_amd import lib as L

_NP = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "U8": np.uint8, "I8": np.int8}
_GEMV = re.compile(r"^(model\.layers\.\d+\.(self_attn\.[qkvo]_proj|mlp\.(gate|up|down)_proj)|lm_head)\.weight$")


def read_safetensors(path):
    """{name: (dtype string, shape, raw bytes)} and the metadata of a file."""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        data = f.read()
    meta = header.pop("__metadata__", {})
    out = {}
    for name, info in header.items():
        a, b = info["data_offsets"]
        out[name] = (info["dtype"], list(info["shape"]), data[a:b])
    return out, meta


def write_safetensors(path, tensors, meta):
    """tensors: {name: (dtype string, shape, raw bytes)}, written in name order."""
    header, off = {}, 0
    for name in sorted(tensors):
        dt, shape, raw = tensors[name]
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    if meta:
        header["__metadata__"] = meta
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for name in sorted(tensors):
            f.write(tensors[name][2])


def as_f32(dt, shape, raw):
    a = np.frombuffer(raw, dtype=_NP[dt]).reshape(shape)
    if dt == "BF16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def quantize(w, mode):
    """The loader's quantizer: (codes int8 [n, k], fp16 scale bits)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    codes = np.empty((n, k), np.int8)
    scales = np.empty((n, (k + 31) // 32) if mode == "int4" else (n,), np.uint16)
    fn = L.kernels().lyk_q4_quantize if mode == "int4" else L.kernels().lyk_q8_quantize
    p = lambda a: a.ctypes.data_as(C.c_void_p)
    L.check(fn.__name__, fn(p(w), n, k, p(codes), p(scales)))
    return codes, scales


def quantized_tensors(base, w, mode):
    """{base.qweight, base.qscale} in the on-wire form above."""
    codes, scales = quantize(w, mode)
    n, k = codes.shape
    if mode == "int4":
        nib = (codes.astype(np.int16) + 8).astype(np.uint8)
        if k % 2:
            nib = np.concatenate([nib, np.full((n, 1), 8, np.uint8)], axis=1)
        packed = nib[:, 0::2] | (nib[:, 1::2] << 4)
        qw = ("U8", [n, (k + 1) // 2], np.ascontiguousarray(packed).tobytes())
    else:
        qw = ("I8", [n, k], codes.tobytes())
    return {f"{base}.qweight": qw, f"{base}.qscale": ("F16", list(scales.shape), scales.tobytes())}


def convert(src, dst, mode, head=False):
    tensors, meta = read_safetensors(src)
    out = {}
    for name, (dt, shape, raw) in tensors.items():
        if _GEMV.match(name):
            out.update(quantized_tensors(name[: -len(".weight")], as_f32(dt, shape, raw), mode))
        else:
            out[name] = (dt, shape, raw)
    if head and "lm_head.weight" not in tensors and "model.embed_tokens.weight" in tensors:
        out.update(quantized_tensors("lm_head", as_f32(*tensors["model.embed_tokens.weight"]), mode))
    meta = dict(meta)
    meta["lykuro_quant"] = "int4_g32" if mode == "int4" else "int8_row"
    write_safetensors(dst, out, meta)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("src")
    ap.add_argument("dst")
    ap.add_argument("--quant", choices=["int4", "int8"], default="int4")
    ap.add_argument("--head", action="store_true", help="also store a tied LM head's quantized form")
    a = ap.parse_args()
    out = convert(a.src, a.dst, a.quant, a.head)
    print(f"wrote {a.dst}: {len(out)} tensors ({a.quant})")


if __name__ == "__main__":
    main()
