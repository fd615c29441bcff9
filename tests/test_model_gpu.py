"""QwenHipModel against the CPU oracle, through the model C ABI.

The case list follows the reference's backend parity suite
(tests/cuda/cuda_parity_test.cpp:85-558): prefill / long-prompt / decode
trajectory parity, run-to-run determinism, capacity and vocab errors, batched
vs sequential decode, per-item error isolation, paged-pool exhaustion, the
prefix cache, quantized-vs-fp32 closeness, plus GreedyRun == sequential
Decode + argmax (tests/metal/metal_fast_parity_test.cpp:123-163).

Bars: greedy tokens equal the oracle's for 32 decode
steps; logits within the stated norm-relative tolerance of the fp32 oracle on
the dequantized weights; bit-identical repeats."""
import numpy as np
import pytest

from engine_amd import model as M
from oracle import oracle as O
from tests.model_pairs import rel_err, synthetic_pair, tiny_pair, top2_gap

pytestmark = pytest.mark.gpu

# End-to-end logits tolerance (norm-relative) against the fp32 oracle: the
# backend rounds GEMV inputs and K/V to fp16, ~2^-12 relative per element.
E2E_TOL = 5e-3
MODES = ["int4", "int8"]


@pytest.fixture(scope="module", params=MODES)
def tiny(request):
    src, ref, hip = tiny_pair(request.param)
    yield request.param, src, ref, hip
    hip.close()


def test_prefill_logits_match_oracle(tiny):
    mode, _, ref, hip = tiny
    prompt = [1, 5, 9, 2, 17, 250]
    s, rs = hip.new_seq(128), ref.new_seq(128)
    c1, a = hip.prefill(s, prompt)
    c2, b = ref.prefill(rs, prompt)
    assert c1 == c2 == 0
    assert rel_err(a, b) < E2E_TOL
    assert np.argmax(a) == np.argmax(b)


def test_long_prompt_prefill_matches_oracle(tiny):
    """cuda_parity_test.cpp:99-110 (60-token prompt)."""
    mode, _, ref, hip = tiny
    prompt = [1 + i * 5 % 300 for i in range(60)]
    s, rs = hip.new_seq(128), ref.new_seq(128)
    c1, a = hip.prefill(s, prompt)
    c2, b = ref.prefill(rs, prompt)
    assert c1 == c2 == 0 and rel_err(a, b) < E2E_TOL


def test_decode_trajectory_matches_oracle(tiny):
    """32 greedy steps, each side sampling its own logits."""
    mode, _, ref, hip = tiny
    s, rs = hip.new_seq(128), ref.new_seq(128)
    _, a = hip.prefill(s, [3, 7, 11])
    _, b = ref.prefill(rs, [3, 7, 11])
    for step in range(32):
        assert rel_err(a, b) < E2E_TOL, step
        ta, tb = O.argmax(a), O.argmax(b)
        assert ta == tb, f"greedy divergence at step {step} (oracle top-2 gap {top2_gap(b):.2e})"
        c1, a = hip.decode(s, ta)
        c2, b = ref.decode(rs, tb)
        assert c1 == c2 == 0


def test_output_is_deterministic_across_runs(tiny):
    mode, _, _, hip = tiny

    def run():
        s = hip.new_seq(128)
        _, logits = hip.prefill(s, [1, 2, 3])
        for i in range(10):
            c, logits = hip.decode(s, i * 7 % 300)
            assert c == 0
        return logits

    a, b = run(), run()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rejects_capacity_overrun_and_bad_tokens(tiny):
    mode, _, _, hip = tiny
    s = hip.new_seq(4)
    assert hip.prefill(s, [1] * 5)[0] == M.CONTEXT_LENGTH_EXCEEDED
    assert hip.prefill(s, [9999])[0] == M.INVALID_REQUEST
    assert hip.prefill(s, [])[0] == M.INVALID_REQUEST
    assert hip.prefill(s, [1, 2, 3, 4])[0] == M.OK
    assert hip.prefill(s, [1])[0] == M.INTERNAL_ERROR
    assert hip.decode(s, 1)[0] == M.CONTEXT_LENGTH_EXCEEDED
    assert hip.decode(hip.new_seq(8), 303)[0] == M.INVALID_REQUEST


# Batches of up to two rows fold the quantization offsets out of the GEMV
# loop exactly as single rows do, so their rows' logits equal sequential
# decoding bit for bit; wider batches subtract the offsets per code and agree
# to rounding (BATCH_TOL), with equal greedy tokens as the reference requires.
BATCH_TOL = 1e-3


@pytest.mark.parametrize("prompts", [[[1, 5, 9], [17, 4, 22, 8, 30]],
                                     [[1, 5, 9], [17, 4, 22, 8, 30], [7, 7, 25], [300, 2]]],
                         ids=["rows2_bit_exact", "rows4"])
def test_batched_decode_matches_sequential(tiny, prompts):
    """cuda_parity_test.cpp:206-256 (greedy tokens equal), and for batches
    of two the stronger bar: logits equal bit for bit."""
    mode, _, _, hip = tiny
    exact = len(prompts) <= 2
    seq = [hip.new_seq(64) for _ in prompts]
    bat = [hip.new_seq(64) for _ in prompts]
    sl = [hip.prefill(s, p)[1] for s, p in zip(seq, prompts)]
    bl = [hip.prefill(s, p)[1] for s, p in zip(bat, prompts)]
    for step in range(12):
        toks = [O.argmax(l) for l in sl]
        assert toks == [O.argmax(l) for l in bl]
        for i in range(len(prompts)):
            if exact:
                assert np.array_equal(sl[i].view(np.uint32), bl[i].view(np.uint32)), (step, i)
            else:
                assert rel_err(bl[i], sl[i]) < BATCH_TOL, (step, i)
        sl = [hip.decode(s, t)[1] for s, t in zip(seq, toks)]
        code, per, logits = hip.decode_batch(bat, toks)
        assert code == 0 and per == [0] * len(prompts)
        bl = list(logits)
    for x in seq + bat:
        x.close()


def test_batched_decode_isolates_invalid_items(tiny):
    """cuda_parity_test.cpp:258-276."""
    mode, _, _, hip = tiny
    good, full = hip.new_seq(64), hip.new_seq(3)
    assert hip.prefill(good, [1, 2])[0] == 0
    assert hip.prefill(full, [1, 2, 3])[0] == 0
    code, per, _ = hip.decode_batch([good, full, good], [5, 6, 99999])
    assert code == 0
    assert per == [0, M.CONTEXT_LENGTH_EXCEEDED, M.INVALID_REQUEST]
    assert good.length == 3 and full.length == 3


def test_greedy_run_equals_sequential_decode(tiny):
    """GreedyRun (on-device argmax chaining) == Decode + host argmax, bit for
    bit (metal_fast_parity_test.cpp:123-163)."""
    mode, _, _, hip = tiny
    a, b = hip.new_seq(128), hip.new_seq(128)
    _, la = hip.prefill(a, [4, 9, 16])
    hip.prefill(b, [4, 9, 16])
    first = O.argmax(la)
    code, run = hip.greedy_run(b, first, 40)
    assert code == 0 and len(run) == 40 and b.length == 43
    seqt, t = [], first
    for _ in range(40):
        _, l = hip.decode(a, t)
        t = O.argmax(l)
        seqt.append(t)
    assert run == seqt
    # state continues identically afterwards
    assert np.array_equal(hip.decode(a, 5)[1].view(np.uint32), hip.decode(b, 5)[1].view(np.uint32))


def test_greedy_run_argument_errors(tiny):
    mode, _, _, hip = tiny
    s = hip.new_seq(8)
    hip.prefill(s, [1, 2, 3])
    assert hip.greedy_run(s, 303, 4)[0] == M.INVALID_REQUEST
    assert hip.greedy_run(s, 1, 0)[0] == M.INVALID_REQUEST
    code, toks = hip.greedy_run(s, 1, 100)      # capped by capacity
    assert code == 0 and len(toks) == 5 and s.length == 8
    assert hip.greedy_run(s, 1, 1)[0] == M.CONTEXT_LENGTH_EXCEEDED


def test_quantized_close_to_fp32_model(tiny):
    """cuda_parity_test.cpp:424-453: quantization error bound against the
    unquantized model (0.05 int8, 0.4 int4 max-abs on logits)."""
    mode, src, _, hip = tiny
    prompt = [1, 5, 9, 2, 17, 250]
    _, a = hip.prefill(hip.new_seq(128), prompt)
    _, b = src.prefill(src.new_seq(128), prompt)
    tol = 0.05 if mode == "int8" else 0.4
    assert np.abs(a - b).max() <= tol


# ------------------------------------------------------- paged pool / prefix
def _pool_model(mode, pool_tokens):
    _, _, hip = tiny_pair(mode, options=M.Options(quant=mode, kv_pool_tokens=pool_tokens,
                                                  kv_block_tokens=16))
    return hip


@pytest.mark.parametrize("mode", MODES)
def test_paged_pool_exhaustion_reports_capacity(cuda, mode):
    """cuda_parity_test.cpp:280-305."""
    hip = _pool_model(mode, 32)  # 2 blocks of 16
    s = hip.new_seq(128)
    assert hip.prefill(s, [1] * 40)[0] == M.CAPACITY_EXHAUSTED
    s.close()
    assert hip.kv_blocks_free == hip.kv_blocks_total == 2
    hip.close()


def test_prefix_cache_reuses_blocks_within_scope(cuda):
    """cuda_parity_test.cpp:307-367."""
    hip = _pool_model("int4", 512)
    prompt = [1 + i % 250 for i in range(40)]
    first = hip.new_seq(128, True, "tn_a/prj_1")
    _, l1 = hip.prefill(first, prompt)
    assert hip.prefix_cache_hit_tokens == 0
    second = hip.new_seq(128, True, "tn_a/prj_1")
    _, l2 = hip.prefill(second, prompt)
    assert hip.prefix_cache_hit_tokens == 32
    assert np.array_equal(l1, l2)
    pristine = l1.copy()
    for _ in range(8):
        t1, t2 = O.argmax(l1), O.argmax(l2)
        assert t1 == t2
        _, l1 = hip.decode(first, t1)
        _, l2 = hip.decode(second, t2)
    third = hip.new_seq(128, True, "tn_b/prj_9")
    _, l3 = hip.prefill(third, prompt)
    assert hip.prefix_cache_hit_tokens == 32
    assert np.array_equal(pristine, l3)
    hip.close()


def test_prefix_cache_disabled_by_default(cuda):
    hip = _pool_model("int4", 512)
    for _ in range(2):
        s = hip.new_seq(128)
        assert hip.prefill(s, [7] * 40)[0] == 0
    assert hip.prefix_cache_hit_tokens == 0
    hip.close()


def test_prefix_cache_eviction_reclaims_unreferenced_blocks(cuda):
    """cuda_parity_test.cpp:388-420."""
    hip = _pool_model("int4", 64)  # 4 blocks
    a = hip.new_seq(128, True, "tn_a")
    assert hip.prefill(a, [3] * 40)[0] == 0
    a.close()
    assert hip.kv_blocks_free == hip.kv_blocks_total
    b = hip.new_seq(128, True, "tn_a")
    assert hip.prefill(b, [9] * 48)[0] == 0
    b.close()
    hip.close()


# ---------------------------------------------------- synthetic, larger
MID = O.QwenConfig(2048, 512, 3, 8, 2, 64, 1408, 512, 1e-6, 1e6, False, 2047)
MID128 = O.QwenConfig(4096, 1024, 2, 8, 2, 128, 2816, 512, 1e-6, 1e6, True, 4095)


@pytest.mark.parametrize("cfg", [MID, MID128], ids=["hd64", "hd128"])
@pytest.mark.parametrize("mode", MODES)
def test_synthetic_model_greedy_32_steps(cuda, cfg, mode):
    src, ref, hip = synthetic_pair(cfg, mode, seed=3)
    prompt = list(O.synth_tokens(1, 0, 24, cfg.vocab_size))
    s, rs = hip.new_seq(cfg.max_context_tokens), ref.new_seq(cfg.max_context_tokens)
    _, a = hip.prefill(s, prompt)
    _, b = ref.prefill(rs, prompt)
    errs = []
    for step in range(32):
        errs.append(rel_err(a, b))
        ta, tb = O.argmax(a), O.argmax(b)
        assert ta == tb, f"step {step}: {ta} != {tb}, oracle top-2 gap {top2_gap(b):.3e}"
        _, a = hip.decode(s, ta)
        _, b = ref.decode(rs, tb)
    assert max(errs) < E2E_TOL, errs
    hip.close()


# ------------------------------------------- long contexts, attention splits
# G = 7 query heads per kv head, as Qwen2.5-0.5B / 7B.
LONG64 = O.QwenConfig(2048, 512, 2, 14, 2, 64, 1408, 1536, 1e-6, 1e6, False, 2047)
LONG128 = O.QwenConfig(4096, 896, 2, 7, 1, 128, 2048, 1536, 1e-6, 1e6, True, 4095)
LONG_PROMPT, LONG_STEPS = 1100, 6
# (attn_split_tokens, attn_max_splits): the defaults (many splits merged
# across workgroups), one split per kv head (a unit runs five 256-token
# softmax chunks), three splits, splits of at least 256 tokens, and 35 splits
# of 32 tokens (more splits than half a wave of lanes in the merge).
POLICIES = {"default": (0, 0), "one_split": (0, 1), "three_splits": (16, 3), "min256": (256, 32),
            "split35": (32, 64)}


@pytest.fixture(scope="module", params=[LONG64, LONG128], ids=["hd64", "hd128"])
def long_case(request):
    """The oracle's teacher-forced trajectory: logits after a 1100-token
    prompt and after each of 6 greedy tokens."""
    cfg = request.param
    src = O.OracleModel(cfg, 8)
    from tests.model_pairs import fill_synthetic, oracle_for
    fill_synthetic(src, 5)
    ref = oracle_for(src, "int4")
    prompt = list(O.synth_tokens(2, 0, LONG_PROMPT, cfg.vocab_size))
    rs = ref.new_seq(cfg.max_context_tokens)
    _, b = ref.prefill(rs, prompt)
    traj, toks = [b], []
    for _ in range(LONG_STEPS):
        toks.append(O.argmax(b))
        _, b = ref.decode(rs, toks[-1])
        traj.append(b)
    return cfg, prompt, toks, traj


@pytest.mark.parametrize("policy", list(POLICIES), ids=list(POLICIES))
def test_long_context_attention_splits(cuda, long_case, policy):
    cfg, prompt, toks, traj = long_case
    tok, ms = POLICIES[policy]
    hip = M.HipModel.synthetic(cfg, seed=5, sigma=0.02,
                               options=M.Options(quant="int4", attn_split_tokens=tok, attn_max_splits=ms))
    s = hip.new_seq(cfg.max_context_tokens)
    code, a = hip.prefill(s, prompt)
    assert code == 0
    for step in range(LONG_STEPS + 1):
        err = rel_err(a, traj[step])
        assert err < E2E_TOL, (step, err)
        if step < LONG_STEPS:
            assert O.argmax(a) == toks[step], f"step {step}, oracle top-2 gap {top2_gap(traj[step]):.3e}"
            code, a = hip.decode(s, toks[step])
            assert code == 0
    hip.close()


def test_long_context_split_policies_agree(cuda, long_case):
    """Every split policy computes the same attention up to rounding: the
    split changes the fp32 summation order, and fp16 rounding of the GEMV
    inputs and cached K/V (2^-11 relative per flipped element) carries the
    difference to the logits, so policies agree to well inside E2E_TOL but
    not bit for bit."""
    cfg, prompt, toks, traj = long_case
    outs = []
    for tok, ms in POLICIES.values():
        hip = M.HipModel.synthetic(cfg, seed=5, sigma=0.02,
                                   options=M.Options(quant="int4", attn_split_tokens=tok, attn_max_splits=ms))
        s = hip.new_seq(cfg.max_context_tokens)
        outs.append(hip.prefill(s, prompt)[1])
        hip.close()
    to_oracle = [rel_err(o, traj[0]) for o in outs]
    between = [rel_err(o, outs[0]) for o in outs[1:]]
    assert max(between) < 1.5e-3, (between, to_oracle)


@pytest.mark.parametrize("lens", [[LONG_PROMPT, 37], [LONG_PROMPT, 37, 600, 260]], ids=["rows2", "rows4"])
def test_batched_long_rows_match_sequential(cuda, long_case, lens):
    """Rows of different context lengths (different split counts) in one
    batch: each row's logits equal its own sequential decode (bit for bit
    for batches of two, to BATCH_TOL for four)."""
    cfg, prompt, _, _ = long_case
    hip = M.HipModel.synthetic(cfg, seed=5, sigma=0.02, options=M.Options(quant="int4"))
    exact = len(lens) <= 2
    seq = [hip.new_seq(cfg.max_context_tokens) for _ in lens]
    bat = [hip.new_seq(cfg.max_context_tokens) for _ in lens]
    sl = [hip.prefill(s, prompt[:n])[1] for s, n in zip(seq, lens)]
    bl = [hip.prefill(s, prompt[:n])[1] for s, n in zip(bat, lens)]
    for step in range(3):
        toks = [O.argmax(l) for l in sl]
        assert toks == [O.argmax(l) for l in bl]
        for i in range(len(lens)):
            if exact:
                assert np.array_equal(sl[i].view(np.uint32), bl[i].view(np.uint32)), (step, i)
            else:
                assert rel_err(bl[i], sl[i]) < BATCH_TOL, (step, i)
        sl = [hip.decode(s, t)[1] for s, t in zip(seq, toks)]
        code, per, logits = hip.decode_batch(bat, toks)
        assert code == 0 and per == [0] * len(lens)
        bl = list(logits)
    hip.close()


@pytest.mark.parametrize("kw", [dict(attn_split_tokens=24), dict(attn_max_splits=65),
                                dict(attn_split_tokens=-16), dict(kv_block_tokens=8), dict(lds_prefetch=-2)],
                         ids=["tokens_not_tile_multiple", "too_many_splits", "negative", "block_not_16",
                              "bad_lds_prefetch"])
def test_attention_options_rejected(cuda, kw):
    with pytest.raises(M.ModelError) as e:
        M.HipModel.synthetic(MID, seed=1, options=M.Options(quant="int4", **kw))
    assert e.value.code in (M.UNSUPPORTED_MODEL, M.INVALID_REQUEST)


# ------------------------------------------------- gate/up staging in LDS
def staged_run(cfg, mode, lds_prefetch, rows, seed=3, steps=6):
    """Logits of a prefill and `steps` greedy batched decode steps of `rows`
    sequences (prompts of different lengths)."""
    hip = M.HipModel.synthetic(cfg, seed=seed, sigma=0.02,
                               options=M.Options(quant=mode, kv_pool_tokens=4096, lds_prefetch=lds_prefetch))
    seqs = [hip.new_seq(min(cfg.max_context_tokens, 512)) for _ in range(rows)]
    outs = [hip.prefill(s, list(O.synth_tokens(4, i, 20 + 7 * i, cfg.vocab_size)))[1] for i, s in enumerate(seqs)]
    got = [np.stack(outs)]
    for _ in range(steps):
        toks = [O.argmax(l) for l in outs]
        if rows == 1:
            code, l = hip.decode(seqs[0], toks[0])
            outs = [l]
        else:
            code, per, logits = hip.decode_batch(seqs, toks)
            assert per == [0] * rows
            outs = list(logits)
        assert code == 0
        got.append(np.stack(outs))
    hip.close()
    return np.stack(got)


@pytest.mark.parametrize("rows", [1, 2, 4])
@pytest.mark.parametrize("cfg", [MID, MID128], ids=["hd64", "hd128"])
@pytest.mark.parametrize("mode", MODES)
def test_lds_staging_is_bit_exact(cuda, cfg, mode, rows):
    """Staging the gate/up weights in LDS changes where the GEMV reads them
    from, not the arithmetic: every amount of staging (as many chunks as fit,
    one, two) gives the logits of none, bit for bit."""
    base = staged_run(cfg, mode, -1, rows)
    for pf in (0, 1, 2):
        got = staged_run(cfg, mode, pf, rows)
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), pf


def test_lds_staging_bit_exact_at_7b_shape(cuda):
    """The same at Qwen2.5-7B geometry (int4), where the staging region holds
    about half of each wave's gate/up chunks."""
    cfg = M.QWEN25_7B
    base = staged_run(cfg, "int4", -1, 1, steps=3)
    got = staged_run(cfg, "int4", 0, 1, steps=3)
    assert np.array_equal(got.view(np.uint32), base.view(np.uint32))
