"""Device top-p / temperature / top-k sampling against the oracle's
restatement of Sampler::Sample (core/generation/sampler.cpp:35-106), which is
itself checked against the reference's own sampler cases (sampler_test.cpp)
and, where oracle/_ref is built, against the reference Sampler.

Bar: the same token as the oracle for every draw, the draws u coming from
the product's generator (std::mt19937_64 + generate_canonical<double, 53>),
which the CPU tests pin to the oracle's mt19937_64 restatement and to the
published 10000th output. The device's double exp may differ from the
host's in the last bit, which could move a token only when u lands within
about 1e-16 of a boundary; the seeded cases here do not."""
import ctypes as C

import numpy as np
import pytest
import torch

import engine_amd.lib as L
from engine_amd import ops
from oracle import oracle as O


# ------------------------------------------------------------- generator (CPU)
@pytest.mark.parametrize("seed", [0, 1, 42, 5489, 2**63 + 11])
def test_rng_matches_oracle_mt19937_64(seed):
    g = (C.c_uint64 * 313)()
    O.lib().orc_mt64_seed(g, seed)
    r = ops.Rng(seed)
    for _ in range(2000):
        assert r.canonical() == O.lib().orc_mt64_canonical(g)
    r.close()


def test_rng_published_output(golden):
    """The 10000th output of mt19937_64 with the default seed, as a draw:
    generate_canonical divides the 64-bit output by 2^64 in double."""
    c = golden["mt19937_64"]
    r = ops.Rng(c["seed"])
    for _ in range(9999):
        r.canonical()
    assert r.canonical() == float(np.float64(c["output_10000"]) / np.float64(2.0**64))


# ------------------------------------------------------------------ device
def device_tokens(logits, temperature, top_k, top_p, seed, draws):
    """`draws` tokens of one row, the product's generator giving u."""
    x = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).reshape(1, -1).cuda()
    r = ops.Rng(seed)
    ws = torch.empty(L.kernels().lyk_hip_sample_workspace_bytes(1, x.shape[1]), dtype=torch.uint8,
                     device="cuda")
    out = []
    for _ in range(draws):
        u = r.canonical() if temperature != 0.0 else 0.0
        out.append(int(ops.sample(x, temperature, top_k, top_p, [u], ws).cpu()[0]))
    r.close()
    return out


def oracle_tokens(logits, temperature, top_k, top_p, seed, draws):
    s = O.Sampler(temperature, top_p, top_k, seed)
    out = []
    for _ in range(draws):
        code, tok = s.sample(np.ascontiguousarray(logits, np.float32))
        out.append(tok if code == 0 else -1)
    return out


def logits_of(kind, n, seed):
    g = np.random.default_rng(seed)
    if kind == "normal":
        return g.standard_normal(n).astype(np.float32) * 3.0
    if kind == "peaked":   # a model-like head: a few large logits over a wide low tail
        x = g.standard_normal(n).astype(np.float32) * 2.0
        x[g.integers(0, n, 5)] += 12.0
        return x
    if kind == "ties":     # many equal logits: the stable order by index decides
        return g.integers(-3, 3, n).astype(np.float32)
    raise ValueError(kind)


PARAMS = [(0.0, 0, 1.0), (0.7, 0, 0.9), (1.0, 0, 1.0), (1.0, 40, 0.95), (1.3, 5, 0.5), (0.5, 1, 1.0),
          (2.0, 0, 0.3)]


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["normal", "peaked", "ties"])
@pytest.mark.parametrize("n", [7, 1000, 152064])
@pytest.mark.parametrize("params", PARAMS, ids=[f"T{t}_k{k}_p{p}" for t, k, p in PARAMS])
def test_sample_matches_oracle(cuda, kind, n, params):
    t, k, p = params
    x = logits_of(kind, n, n + len(kind))
    seed = 1234 + n
    assert device_tokens(x, t, k, p, seed, 12) == oracle_tokens(x, t, k, p, seed, 12)


@pytest.mark.gpu
def test_sample_wide_candidate_set(cuda):
    """Near-flat logits at temperature 1: every one of the 152064 terms
    counts, so the candidates are sorted in global memory (more than the LDS
    holds) and the running sums run over all of them."""
    x = (np.random.default_rng(7).standard_normal(152064) * 1e-3).astype(np.float32)
    for t, k, p in [(1.0, 0, 1.0), (1.0, 0, 0.5), (1.0, 20000, 0.9)]:
        assert device_tokens(x, t, k, p, 99, 4) == oracle_tokens(x, t, k, p, 99, 4)


@pytest.mark.gpu
def test_sample_reference_cases(cuda, golden):
    """sampler_test.cpp's cases (tests/golden), through the device."""
    s = golden["sampler"]
    for case in ("greedy_argmax", "greedy_tie"):
        assert device_tokens(s[case]["logits"], 0.0, 0, 1.0, 0, 1) == [s[case]["expected"]]
    c = s["top_k"]
    got = device_tokens(c["logits"], c["temperature"], c["top_k"], 1.0, c["seed"], c["draws"])
    assert all(tok in c["allowed"] for tok in got)
    c = s["small_top_p"]
    got = device_tokens(c["logits"], c["temperature"], 0, c["top_p"], c["seed"], c["draws"])
    assert all(tok == c["expected"] for tok in got)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1000, 152064])
@pytest.mark.parametrize("bad", [float("inf"), float("-inf"), float("nan")])
def test_sample_non_finite_fails_the_row(cuda, bad, n):
    """Both paths: one launch (n = 1000) and the wide rows' prep / sort /
    finish (n = 152064 without top_k)."""
    x = logits_of("normal", n, 3)
    x[n // 2] = bad
    assert device_tokens(x, 0.8, 0, 0.9, 1, 1) == [-1]
    assert device_tokens(x, 0.0, 0, 1.0, 1, 1) == [-1]


@pytest.mark.gpu
@pytest.mark.parametrize("n", [5000, 40000])
def test_sample_rows_are_independent(cuda, n):
    """Four rows in one call give each row's single-row token (n = 40000:
    the wide rows' path)."""
    rows = np.stack([logits_of(kind, n, i) for i, kind in enumerate(["normal", "peaked", "ties", "normal"])])
    x = torch.from_numpy(rows).cuda()
    u = [0.1, 0.5, 0.9, 0.999]
    got = ops.sample(x, 0.9, 0, 0.95, u).cpu().tolist()
    for r in range(4):
        assert got[r] == int(ops.sample(x[r:r + 1], 0.9, 0, 0.95, [u[r]]).cpu()[0])


@pytest.mark.gpu
def test_sample_rejects_bad_arguments(cuda):
    x = torch.zeros(1, 10, device="cuda")
    for t, k, p, u in [(-1.0, 0, 1.0, 0.5), (1.0, 0, 0.0, 0.5), (1.0, 0, 1.5, 0.5), (1.0, -1, 1.0, 0.5),
                       (1.0, 0, 1.0, 1.0), (float("nan"), 0, 1.0, 0.5)]:
        with pytest.raises(L.LykError):
            ops.sample(x, t, k, p, [u])
