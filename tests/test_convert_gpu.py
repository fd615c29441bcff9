"""QwenHipModel from an offline-quantized artifact (engine_amd/convert.py)
against the same model quantized at load: the converter stores the loader's
own codes and scales, so the logits are equal bit for bit, through the chunk
prefill, Decode and GreedyRun; an artifact quantized for the other mode is
refused (kUnsupportedModel). The artifact side of the reference's next step:
model/loader/safetensors.h:21, model/convert/hf_convert.cpp:266."""
import os
import tempfile

import numpy as np
import pytest

from engine_amd import convert as CV
from engine_amd import model as M
from oracle import oracle as O
from tests.model_pairs import fill_synthetic

pytestmark = pytest.mark.gpu

UNTIED = O.QwenConfig(1024, 256, 2, 4, 2, 64, 512, 256, 1e-6, 1e6, False, 1023)


def _files(cfg, seed, mode, head=False, tiny=False):
    src = O.OracleModel(cfg)
    if tiny:
        src.fill_tiny(seed)
    else:
        fill_synthetic(src, seed=seed)
    d = tempfile.mkdtemp()
    path = os.path.join(d, "m.safetensors")
    O.model_to_safetensors(src, path)
    qpath = os.path.join(d, f"q_{mode}.safetensors")
    CV.convert(path, qpath, mode, head=head)
    return path, qpath


def _run(hip, prompt, steps):
    s = hip.new_seq(len(prompt) + steps + 2)
    code, a = hip.prefill(s, prompt)
    assert code == 0
    out = [a]
    for _ in range(steps):
        code, a = hip.decode(s, O.argmax(a))
        assert code == 0
        out.append(a)
    g = hip.new_seq(len(prompt) + steps + 2)
    code, first = hip.prefill(g, prompt)
    code, toks = hip.greedy_run(g, O.argmax(first), steps)
    assert code == 0
    return out, toks


@pytest.mark.parametrize("mode", ["int4", "int8"])
@pytest.mark.parametrize("case", ["untied_hd64", "tied_tiny_head"])
def test_quantized_artifact_equals_load_time_quantization(cuda, mode, case):
    if case == "untied_hd64":
        cfg, paths = UNTIED, _files(UNTIED, 4, mode)
        prompt = list(O.synth_tokens(5, 0, 40, cfg.vocab_size))
    else:
        cfg, paths = O.TINY_PARITY, _files(O.TINY_PARITY, 42, mode, head=True, tiny=True)
        prompt = [1, 5, 9, 2, 17, 250]
    runs = []
    for p in paths:
        hip = M.HipModel.from_safetensors(p, cfg, M.Options(quant=mode))
        try:
            runs.append(_run(hip, prompt, 8))
        finally:
            hip.close()
    (la, ta), (lb, tb) = runs
    for x, y in zip(la, lb):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    assert ta == tb


def test_artifact_of_the_other_mode_is_refused(cuda):
    _, q = _files(UNTIED, 4, "int4")
    with pytest.raises(M.ModelError) as e:
        M.HipModel.from_safetensors(q, UNTIED, M.Options(quant="int8"))
    assert e.value.code == M.UNSUPPORTED_MODEL
