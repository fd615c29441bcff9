"""The fused decode step (QwenHipModel through the model C ABI) against the
CPU oracle at the BASELINE geometries, not only at small shapes:

  * Qwen2.5-7B layers (hidden 3584, 28/4 heads of 128, MLP 18944, untied
    152064 head), int4 -- the tile heights, K pieces, 4752-tile LM head and
    greedy pick the 7B model runs with;
  * Qwen2.5-14B layers (hidden 5120 = the register-window limit, 40/8 heads,
    MLP 13824), int8;
  * Qwen2.5-0.5B whole (24 layers, 14/2 heads of 64, tied 151936 head);
  * config 3's attention geometry (28/4 heads of 128) over four ragged rows
    with contexts drawn from U[512, 8192] and block tables scrambled by
    freeing blocks in a permuted order;
  * config 4's four-sequence leg at 7B geometry, batched against sequential.

The GEMV-heavy layers are few (2) so the CPU oracle finishes in seconds; the
layer count does not change what one layer computes. Pattern of the
reference's backend parity suite (tests/cuda/cuda_parity_test.cpp:85-136,
206-256; tests/metal/metal_fast_parity_test.cpp:123-163, 210-).

Bars:
  floor       the oracle's fp16 mirror mode (the fp32 reference forward with
              fp16 rounding exactly where this backend stores fp16) against
              itself with its matvec sums taken in the other (descending)
              order: both are correct fp32 evaluations, and they differ only
              because a ~1e-6 change of order flips some fp16 roundings,
              whose 2^-11 steps propagate. The backend sums in yet another
              order (trees of partial sums), so it is held to that floor:
              logits within FLOOR_FACTOR x the floor of the mirrored oracle
              (both modes pinned in test_oracle.py).
  E2E_TOL     against the plain fp32 oracle (the backend's fp16 storage
              points differ from it by ~2^-12 relative per element).
  greedy      the backend's greedy tokens equal the oracle's for 32 steps
              (teacher-forced), except where the oracle's own two orders
              disagree by more than the logit gap between the two tokens (a
              tie at the floor's resolution); GreedyRun gives the backend's
              Decode + argmax tokens bit for bit.
"""
import dataclasses

import numpy as np
import pytest

from engine_amd import model as M
from oracle import oracle as O
from tests.model_pairs import dequant_oracle, oracle_run, rel_err, top2_gap

pytestmark = pytest.mark.gpu

FLOOR_FACTOR = 2.5
E2E_TOL = 5e-3
BATCH_TOL = 1e-3
STEPS = 32


def _geom(cfg, layers, ctx=512):
    return dataclasses.replace(cfg, num_layers=layers, max_context_tokens=ctx)


Q7B = _geom(O.QWEN7B, 2)
Q14B = _geom(O.QWEN14B, 2)
Q05B = _geom(O.QWEN05B, 24)


def _report(tag, errs):
    print(f"{tag}: max rel err {max(errs):.3e} mean {np.mean(errs):.3e}", flush=True)


def _floor(ref, prompt, toks, mir):
    """The mirrored oracle's trajectory `mir` (ascending sums) against its
    descending twin along the same tokens: (mir, per-step relative gap,
    per-step max |gap|)."""
    rev, _ = oracle_run(ref, prompt, len(toks), mirror=True, forced=toks, descending=True)
    rel = [rel_err(r, m) for r, m in zip(rev, mir)]
    gap = [float(np.max(np.abs(r - m))) for r, m in zip(rev, mir)]
    return mir, rel, gap


def _greedy_ok(logits, ref_logits, tok, gap):
    """The backend's choice is the oracle's token, or a tie at the floor's
    resolution: the oracle scores the two within 4x its own order gap."""
    got = O.argmax(logits)
    return got == tok or ref_logits[tok] - ref_logits[got] <= 4 * gap


@pytest.mark.parametrize("cfg,mode", [(Q7B, "int4"), (Q14B, "int8"), (Q05B, "int4"), (Q05B, "int8")],
                         ids=["7b_int4", "14b_int8", "05b_int4", "05b_int8"])
def test_geometry_decode_and_greedy_run_match_oracle(cuda, cfg, mode):
    """Prefill + 32 teacher-forced Decode steps along the mirrored oracle's
    greedy tokens: logits within FLOOR_FACTOR x the oracle's own order floor
    of the mirrored oracle and within E2E_TOL of the plain one; greedy
    choices equal up to floor-resolution ties. Then GreedyRun from the same
    prompt reproduces the backend's own Decode + argmax run bit for bit."""
    print(f"[geometry] {cfg.hidden_size} hidden x {cfg.num_layers} layers, {mode}", flush=True)
    ref = dequant_oracle(cfg, mode, seed=11)
    prompt = list(O.synth_tokens(12, 0, 9, cfg.vocab_size))
    mir, toks = oracle_run(ref, prompt, STEPS, mirror=True)
    _, floor, gap = _floor(ref, prompt, toks, mir)
    plain, _ = oracle_run(ref, prompt, STEPS, mirror=False, forced=toks)
    del ref
    hip = M.HipModel.synthetic(cfg, seed=11, sigma=0.02, options=M.Options(quant=mode))
    try:
        s = hip.new_seq(cfg.max_context_tokens)
        code, a = hip.prefill(s, prompt)
        assert code == 0
        em, ep, ties = [], [], 0
        for step in range(STEPS + 1):
            em.append(rel_err(a, mir[step]))
            ep.append(rel_err(a, plain[step]))
            if step == STEPS:
                break
            assert _greedy_ok(a, mir[step], toks[step], gap[step]), \
                f"step {step}: greedy {O.argmax(a)} != oracle {toks[step]} (top-2 gap {top2_gap(mir[step]):.3e})"
            ties += O.argmax(a) != toks[step]
            code, a = hip.decode(s, toks[step])
            assert code == 0
        _report(f"{mode} H{cfg.hidden_size} vs mirrored oracle", em)
        _report(f"{mode} H{cfg.hidden_size} oracle order floor", floor)
        _report(f"{mode} H{cfg.hidden_size} vs plain oracle", ep)
        print(f"  greedy: {STEPS - ties}/{STEPS} equal, {ties} floor-resolution ties", flush=True)
        assert max(em) <= FLOOR_FACTOR * max(floor), (em, floor)
        assert max(ep) < E2E_TOL, ep
        # GreedyRun (on-device argmax chaining, the LM head's tile
        # candidates) against the backend's own Decode + argmax
        g, d = hip.new_seq(cfg.max_context_tokens), hip.new_seq(cfg.max_context_tokens)
        code, first = hip.prefill(g, prompt)
        assert code == 0 and hip.prefill(d, prompt)[0] == 0
        code, run = hip.greedy_run(g, O.argmax(first), STEPS)
        assert code == 0
        want, t = [], O.argmax(first)
        for _ in range(STEPS):
            code, l = hip.decode(d, t)
            t = O.argmax(l)
            want.append(t)
        assert run == want
    finally:
        hip.close()


# ------------------------------------------------ config 3: ragged, long
ATT = O.QwenConfig(1024, 512, 1, 28, 4, 128, 1024, 8300, 1e-6, 1e6, False, 1023)
ATT_STEPS = 6


def _scramble_pool(hip, nblocks, seed):
    """Takes every block of the pool with one-block sequences, then frees
    them in a seeded random order, so later sequences get physical blocks in
    a permuted order."""
    seqs = []
    for i in range(nblocks):
        s = hip.new_seq(16)
        assert hip.prefill(s, [i % 1000 + 1])[0] == 0
        seqs.append(s)
    assert hip.kv_blocks_free == 0
    for i in np.random.default_rng(seed).permutation(nblocks):
        seqs[i].close()
    assert hip.kv_blocks_free == nblocks


def test_config3_ragged_long_context_attention(cuda):
    """Four rows with contexts from U[512, 8192] (seeded), 28 query / 4 kv
    heads of 128, fp16 KV in 16-token blocks placed in a scrambled order;
    DecodeBatch over the four rows, teacher-forced, against the oracle's
    per-row trajectories."""
    rng = np.random.default_rng(3)
    lens = [int(v) for v in rng.integers(512, 8193, 4)]
    print(f"[config3] contexts {lens}", flush=True)
    ref = dequant_oracle(ATT, "int4", seed=21)
    prompts = [list(O.synth_tokens(30 + i, 0, n, ATT.vocab_size)) for i, n in enumerate(lens)]
    runs = [oracle_run(ref, p, ATT_STEPS, mirror=True) for p in prompts]
    floors = [_floor(ref, p, toks, traj)[1:] for p, (traj, toks) in zip(prompts, runs)]
    del ref
    pool_tokens = sum(lens) + 4 * (ATT_STEPS + 16) + 64
    hip = M.HipModel.synthetic(ATT, seed=21, sigma=0.02,
                               options=M.Options(quant="int4", kv_pool_tokens=pool_tokens))
    try:
        _scramble_pool(hip, hip.kv_blocks_total, seed=5)
        seqs = [hip.new_seq(n + ATT_STEPS + 1) for n in lens]
        logits = []
        for s, p in zip(seqs, prompts):
            code, a = hip.prefill(s, p)
            assert code == 0
            logits.append(a)
        errs = []
        for step in range(ATT_STEPS + 1):
            for r in range(4):
                traj, toks = runs[r]
                floor, gap = floors[r]
                errs.append(rel_err(logits[r], traj[step]))
                assert errs[-1] <= FLOOR_FACTOR * max(floor), (step, r, lens[r], errs[-1], floor)
                if step < ATT_STEPS:
                    assert _greedy_ok(logits[r], traj[step], toks[step], gap[step]), \
                        (step, r, top2_gap(traj[step]))
            if step == ATT_STEPS:
                break
            code, per, out = hip.decode_batch(seqs, [runs[r][1][step] for r in range(4)])
            assert code == 0 and per == [0] * 4
            logits = list(out)
        _report("config3 attention vs mirrored oracle", errs)
    finally:
        hip.close()


# ------------------------------------------ config 4: four sequences at 7B
def test_7b_four_sequences_batched_equals_sequential(cuda):
    """max_sequences=4 at 7B geometry: DecodeBatch of four rows of different
    lengths against each row decoded alone (BATCH_TOL, equal greedy tokens),
    and against the mirrored oracle."""
    cfg = Q7B
    ref = dequant_oracle(cfg, "int4", seed=13)
    prompts = [list(O.synth_tokens(40 + i, 0, n, cfg.vocab_size)) for i, n in enumerate([5, 17, 40, 96])]
    steps = 8
    runs = [oracle_run(ref, p, steps, mirror=True) for p in prompts]
    floors = [_floor(ref, p, toks, traj)[1:] for p, (traj, toks) in zip(prompts, runs)]
    del ref
    hip = M.HipModel.synthetic(cfg, seed=13, sigma=0.02, options=M.Options(quant="int4"))
    try:
        seq = [hip.new_seq(cfg.max_context_tokens) for _ in prompts]
        bat = [hip.new_seq(cfg.max_context_tokens) for _ in prompts]
        sl = [hip.prefill(s, p)[1] for s, p in zip(seq, prompts)]
        bl = [hip.prefill(s, p)[1] for s, p in zip(bat, prompts)]
        errs = []
        for step in range(steps + 1):
            for i in range(4):
                traj, toks = runs[i]
                floor, gap = floors[i]
                errs.append(rel_err(bl[i], traj[step]))
                assert errs[-1] <= FLOOR_FACTOR * max(floor), (step, i, errs[-1], floor)
                assert rel_err(bl[i], sl[i]) < BATCH_TOL, (step, i)
                if step < steps:
                    assert O.argmax(bl[i]) == O.argmax(sl[i]), (step, i)
                    assert _greedy_ok(bl[i], traj[step], toks[step], gap[step]), (step, i)
            if step == steps:
                break
            toks = [runs[i][1][step] for i in range(4)]
            sl = [hip.decode(s, t)[1] for s, t in zip(seq, toks)]
            code, per, out = hip.decode_batch(bat, toks)
            assert code == 0 and per == [0] * 4
            bl = list(out)
        _report("7b batch-4 vs mirrored oracle", errs)
    finally:
        hip.close()
