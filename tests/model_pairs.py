"""Builds a hip-backend model and the CPU oracle model that computes with the
same weights: the oracle holds every GEMV weight dequantized from the
backend's own quantization (bit-exact by construction and by the unpack
tests), and the embedding, norms and biases exactly."""
import dataclasses
import os
import tempfile

import numpy as np

from engine_amd import model as M
from oracle import oracle as O

GEMV_KINDS = (O.T_Q_W, O.T_K_W, O.T_V_W, O.T_O_W, O.T_GATE_W, O.T_UP_W, O.T_DOWN_W)
NORM_KINDS = (O.T_INPUT_NORM, O.T_POST_NORM, O.T_FINAL_NORM)


def fill_synthetic(model, seed=0, sigma=0.02):
    """The backend's synthetic source restated with the oracle generator:
    stream kind*1000 + layer, norms 1.0."""
    for kind, layer, arr in model.tensors():
        if kind in NORM_KINDS:
            arr[...] = 1.0
        else:
            arr[...] = O.synth_normal(seed, kind * 1000 + layer, arr.size, sigma).reshape(arr.shape)


def oracle_for(src: O.OracleModel, mode, threads=8):
    """Untied oracle with dequantized GEMV weights (lm_head = the quantized
    head the backend uses; embedding exact)."""
    cfg = dataclasses.replace(src.cfg, tie_word_embeddings=False)
    m = O.OracleModel(cfg, threads)
    for kind, layer, arr in src.tensors():
        dst = m.tensor(kind, layer)
        dst[...] = O.quant_dequant(arr, mode) if kind in GEMV_KINDS else arr
    head = src.tensor(O.T_EMBED) if src.cfg.tie_word_embeddings else src.tensor(O.T_LM_HEAD)
    m.tensor(O.T_LM_HEAD)[...] = O.quant_dequant(head, mode)
    return m


def tiny_pair(mode, cfg=O.TINY_PARITY, options=None, seed=42):
    """Reference tiny fixture (LCG weights) through a safetensors file."""
    src = O.OracleModel(cfg)
    src.fill_tiny(seed)
    path = os.path.join(tempfile.mkdtemp(), "tiny.safetensors")
    O.model_to_safetensors(src, path)
    opts = options or M.Options(quant=mode)
    hip = M.HipModel.from_safetensors(path, cfg, opts)
    os.remove(path)
    return src, oracle_for(src, mode), hip


def synthetic_pair(cfg, mode, seed=0, threads=8, options=None):
    src = O.OracleModel(cfg, threads)
    fill_synthetic(src, seed)
    opts = options or M.Options(quant=mode)
    hip = M.HipModel.synthetic(cfg, seed=seed, sigma=0.02, options=opts)
    return src, oracle_for(src, mode, threads), hip


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def top2_gap(logits):
    s = np.sort(np.asarray(logits, np.float64))
    return float(s[-1] - s[-2])


def dequant_oracle(cfg, mode, seed=0, threads=16, sigma=0.02):
    """The oracle the synthetic hip model is checked against, built in place
    (no fp32 copy of the source weights): untied, every GEMV weight (and the
    LM head, the embedding when tied) the dequantized product of the
    backend's quantizer on the seeded synthetic weights; embedding, norms and
    biases exact."""
    ucfg = dataclasses.replace(cfg, tie_word_embeddings=False)
    m = O.OracleModel(ucfg, threads)
    for kind, layer, arr in m.tensors():
        if kind in NORM_KINDS:
            arr[...] = 1.0
            continue
        src_kind = O.T_EMBED if (kind == O.T_LM_HEAD and cfg.tie_word_embeddings) else kind
        arr[...] = O.synth_normal(seed, src_kind * 1000 + layer, arr.size, sigma).reshape(arr.shape)
        if kind in GEMV_KINDS or kind == O.T_LM_HEAD:
            arr[...] = O.quant_dequant(arr, mode)
    return m


def oracle_run(ref, prompt, steps, mirror, forced=None, descending=False):
    """Logits after the prompt and after each of `steps` tokens (greedy on
    the oracle's own logits, or the `forced` tokens), and the tokens fed.
    descending: the noise-floor twin (matvec products added in descending
    order)."""
    ref.set_f16_mirror(mirror)
    ref.set_descending_sums(descending)
    s = ref.new_seq(len(prompt) + steps + 1)
    code, b = ref.prefill(s, prompt)
    assert code == 0
    traj, toks = [b], []
    for i in range(steps):
        toks.append(O.argmax(b) if forced is None else forced[i])
        code, b = ref.decode(s, toks[-1])
        assert code == 0
        traj.append(b)
    ref.set_f16_mirror(False)
    ref.set_descending_sums(False)
    return traj, toks
