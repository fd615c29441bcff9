"""QwenHipModel's host-side contract on the device path, through the model C
ABI:

  * non-finite logits -> inference_failed on Prefill, Decode, DecodeBatch
    (per item, the others advance) and GreedyRun, with nothing advanced or
    published (tests/unit/qwen_model_test.cpp:268-282 poisons the embedding
    the same way; qwen_cuda_model.cu:2386-2392, 3085-3096);
  * BF16 and F16 checkpoints load and compute as the oracle does on the same
    widened values (backends/cpu/cpu_backend.cpp:8-50,
    model/loader/safetensors.cpp:26-29);
  * a step that cannot finish (its bounded waits forced to give up from the
    host) -> gpu_unhealthy with no sequence advanced, even for the second
    group of a DecodeBatch (generative_model.h:76-78), and the next call
    works on a reset workspace;
  * the launch-tag epoch: crossing the 2^24 - 1 launch limit of a workspace
    changes no result.
"""
import os
import tempfile

import numpy as np
import pytest

from engine_amd import model as M
from oracle import oracle as O
from tests.model_pairs import oracle_for, rel_err

pytestmark = pytest.mark.gpu

E2E_TOL = 5e-3
# the reference's tiny parity fixture, untied here so that one poisoned
# embedding row leaves the LM head finite
UNTIED = O.QwenConfig(303, 16, 2, 4, 2, 4, 32, 128, 1e-6, 10000.0, False, 302)


def _poisoned_pair(cfg):
    src = O.OracleModel(cfg)
    src.fill_tiny(42)
    if not cfg.tie_word_embeddings:
        src.tensor(O.T_LM_HEAD)[...] = np.resize(src.tensor(O.T_EMBED), src.tensor(O.T_LM_HEAD).shape)
    src.tensor(O.T_EMBED)[0, 0] = np.inf      # token 0's row, as the reference's fixture
    path = os.path.join(tempfile.mkdtemp(), "poison.safetensors")
    O.model_to_safetensors(src, path)
    hip = M.HipModel.from_safetensors(path, cfg, M.Options(quant="int4"))
    os.remove(path)
    return src, hip


def test_poisoned_embedding_fails_prefill_like_the_reference(cuda):
    """The reference's fixture exactly (tied): prompt {0} -> inference_failed
    on the oracle and on the hip model alike; the sequence stays empty."""
    src, hip = _poisoned_pair(O.TINY_PARITY)
    try:
        assert src.prefill(src.new_seq(8), [0])[0] == O.INFERENCE_FAILED
        s = hip.new_seq(8)
        assert hip.prefill(s, [0])[0] == M.INFERENCE_FAILED
        assert s.length == 0 and hip.kv_blocks_free == hip.kv_blocks_total
    finally:
        hip.close()


def test_non_finite_paths_advance_nothing(cuda):
    _, hip = _poisoned_pair(UNTIED)
    try:
        a, b, c = (hip.new_seq(64) for _ in range(3))
        for s in (a, b, c):
            assert hip.prefill(s, [5, 6, 7])[0] == M.OK
        # Decode: the poisoned token fails and leaves the sequence as it was
        assert hip.decode(a, 0)[0] == M.INFERENCE_FAILED and a.length == 3
        assert hip.decode(a, 9)[0] == M.OK and a.length == 4
        # DecodeBatch: per item; the overall call succeeds and the rest advance
        code, per, _ = hip.decode_batch([a, b, c], [9, 0, 11])
        assert code == M.OK and per == [M.OK, M.INFERENCE_FAILED, M.OK]
        assert (a.length, b.length, c.length) == (5, 3, 4)
        # GreedyRun from the poisoned token: nothing advances
        code, toks = hip.greedy_run(b, 0, 4)
        assert code == M.INFERENCE_FAILED and toks == [] and b.length == 3
        # Prefill ending on the poisoned token: rolled back, nothing published
        p = [3] * 32 + [0]
        s = hip.new_seq(64, True, "scope")
        assert hip.prefill(s, p)[0] == M.INFERENCE_FAILED and s.length == 0
        t = hip.new_seq(64, True, "scope")
        assert hip.prefill(t, p[:-1] + [4])[0] == M.OK
        assert hip.prefix_cache_hit_tokens == 0
    finally:
        hip.close()


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
@pytest.mark.parametrize("mode", ["int4", "int8"])
def test_half_precision_checkpoint_matches_oracle(cuda, dtype, mode):
    """A checkpoint stored in F16/BF16 loads into the hip model and computes
    as the oracle does on the same values widened by the oracle's codecs."""
    cfg = O.QwenConfig(512, 128, 2, 2, 1, 64, 256, 128, 1e-6, 1e6, False, 511)
    src = O.OracleModel(cfg)
    from tests.model_pairs import fill_synthetic
    fill_synthetic(src, seed=9)
    tensors = {O.tensor_name(k, l): a for k, l, a in src.tensors()}
    path = os.path.join(tempfile.mkdtemp(), f"m_{dtype}.safetensors")
    O.write_safetensors(path, tensors, dtype=dtype)
    for _, _, arr in src.tensors():     # the values the file holds, widened
        if dtype == "F16":
            arr[...] = O.round_f16(arr)
        else:
            arr[...] = (np.vectorize(O.lib().orc_f32_to_bf16, otypes=[np.uint16])(arr).astype(np.uint32)
                        << 16).view(np.float32)
    ref = oracle_for(src, mode)
    hip = M.HipModel.from_safetensors(path, cfg, M.Options(quant=mode))
    os.remove(path)
    try:
        prompt = [7, 100, 3, 45, 9]
        s, rs = hip.new_seq(64), ref.new_seq(64)
        (c1, a), (c2, b) = hip.prefill(s, prompt), ref.prefill(rs, prompt)
        assert c1 == c2 == 0
        for step in range(12):
            assert rel_err(a, b) < E2E_TOL, step
            t = O.argmax(b)
            assert O.argmax(a) == t, step
            (c1, a), (c2, b) = hip.decode(s, t), ref.decode(rs, t)
            assert c1 == c2 == 0
    finally:
        hip.close()


def test_unfinished_step_returns_unhealthy_and_recovers(cuda):
    """Waits forced to give up after 1 us: the six-item batch (two groups of
    rows) returns gpu_unhealthy and no sequence advances; with the limit
    restored the same batch runs and matches sequential decoding."""
    from tests.model_pairs import tiny_pair
    _, _, hip = tiny_pair("int4")
    _, _, twin = tiny_pair("int4")
    try:
        prompts = [[1, 2], [3, 4, 5], [6], [7, 8, 9, 10], [11, 12], [13]]
        seqs = [hip.new_seq(64) for _ in prompts]
        twins = [twin.new_seq(64) for _ in prompts]
        for s, t, p in zip(seqs, twins, prompts):
            assert hip.prefill(s, p)[0] == M.OK and twin.prefill(t, p)[0] == M.OK
        toks = [20, 21, 22, 23, 24, 25]
        hip.set_wait_limit(1)
        code, per, _ = hip.decode_batch(seqs, toks)
        assert code == M.GPU_UNHEALTHY
        assert [s.length for s in seqs] == [len(p) for p in prompts]
        hip.set_wait_limit(0)
        code, per, got = hip.decode_batch(seqs, toks)
        assert code == M.OK and per == [M.OK] * 6
        assert [s.length for s in seqs] == [len(p) + 1 for p in prompts]
        for i, (t, tok) in enumerate(zip(twins, toks)):
            c, want = twin.decode(t, tok)
            assert c == 0 and rel_err(got[i], want) < 1e-3, i
    finally:
        hip.close()
        twin.close()


def test_launch_tag_epoch_changes_no_result(cuda):
    """A workspace 4 launches short of the 2^24 - 1 limit: the prefill and
    greedy run that cross it (the host re-zeroes the workspace on the way)
    give the logits and tokens of a workspace far from it, bit for bit."""
    from tests.model_pairs import tiny_pair
    _, _, hip = tiny_pair("int4")
    try:
        prompt = [1, 5, 9, 2, 17, 250]
        runs = []
        for preset in (None, (1 << 24) - 1 - 4):
            if preset is not None:
                hip.set_step_launches(preset)
                assert hip.step_launches == preset
            s = hip.new_seq(64)
            code, logits = hip.prefill(s, prompt)
            assert code == 0
            code, toks = hip.greedy_run(s, O.argmax(logits), 10)
            assert code == 0
            runs.append((logits, toks))
            s.close()
        assert hip.step_launches < 16     # the epoch restarted
        assert np.array_equal(runs[0][0].view(np.uint32), runs[1][0].view(np.uint32))
        assert runs[0][1] == runs[1][1]
    finally:
        hip.close()
