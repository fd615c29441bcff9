"""Chunk prefill on the matrix cores: the chunk kernels against exact
restatements, and QwenHipModel's chunked Prefill against its token-by-token
Prefill (every prompt token through the fused decode step) and the oracle.

Reference: ForwardChunk / ChunkAttentionKernel and the chunk loop
(backends/cuda/qwen_cuda_model.cu:981-1030, 2398-2516, 2578-2590); parity
pattern of tests/cuda/cuda_parity_test.cpp:85-110 (prefill and long-prompt
logits against the CPU path).

Bars:
  * RoPE + KV append: bit-exact (the CPU's separately rounded rotation on the
    same cos/sin tables; fp16 K/V at the fused step's cache layout).
  * chunk attention: against fp64 softmax attention on the same fp32 q and
    fp16 K/V, per element within half an fp16 ulp of the result (the output
    rounding) plus 2e-5 of the largest |v| (q and the weights carried as two
    fp16 parts, ~2^-22; fp32 sums and exp).
  * chunked Prefill: bit-identical logits for every chunk size (no row's
    arithmetic depends on the chunk it falls in), and within CHUNK_TOL of the
    token-by-token Prefill, with equal greedy continuations (the two sum in
    different orders, and fp16 storage points carry those ~1e-7 differences
    on as whole fp16 steps)."""
import numpy as np
import pytest
import torch

from engine_amd import model as M, ops
from oracle import oracle as O
from tests.model_pairs import rel_err, top2_gap

pytestmark = pytest.mark.gpu

CHUNK_TOL = 2e-3


def _tables(max_pos, hd, theta=1e6):
    half = hd // 2
    freq = theta ** (-2.0 * np.arange(half) / hd)
    ang = np.arange(max_pos)[:, None] * freq[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _rot(x, c, s):
    """The CPU rotation in fp32, each product rounded (qwen_model.cpp:49-52)."""
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1).astype(np.float32)


class Cache:
    """A paged fp16 K/V pool of the fused step's layout and a scrambled
    block table for one sequence of `tokens` positions."""

    def __init__(self, nkv, hd, bt, tokens, seed):
        self.nkv, self.hd, self.bt = nkv, hd, bt
        nblk = (tokens + bt - 1) // bt
        self.blocks = nblk + 3
        rng = np.random.default_rng(seed)
        self.table_np = rng.permutation(self.blocks)[:nblk].astype(np.int32)
        self.table = torch.from_numpy(self.table_np).cuda()
        # NaN fill: a read of a slot nothing wrote shows in the results
        self.k = torch.full((self.blocks, nkv, bt, hd), float("nan"), dtype=torch.float16, device="cuda")
        self.v = torch.full((self.blocks, nkv, hd, bt), float("nan"), dtype=torch.float16, device="cuda")

    def positions(self, n):
        """K and V of positions 0..n-1, [n, nkv, hd] each (host copies)."""
        k, v = self.k.cpu().numpy(), self.v.cpu().numpy()
        blk = self.table_np[np.arange(n) // self.bt]
        slot = np.arange(n) % self.bt
        return k[blk, :, slot, :], v[blk, :, :, slot]


def _append(cache, qkv, pos0, nq, cs, sn):
    return ops.chunk_rope_kv(torch.from_numpy(qkv).cuda(), pos0, nq, cache.nkv, cache.hd,
                             torch.from_numpy(cs).cuda(), torch.from_numpy(sn).cuda(), cache.k, cache.v,
                             cache.table, cache.bt)


@pytest.mark.parametrize("hd,bt", [(64, 16), (128, 32)])
def test_chunk_rope_kv_bit_exact(cuda, hd, bt):
    nq, nkv, T, pos0 = 6, 2, 37, 21
    cs, sn = _tables(128, hd)
    rng = np.random.default_rng(hd + bt)
    qkv = rng.standard_normal((T, (nq + 2 * nkv) * hd)).astype(np.float32)
    cache = Cache(nkv, hd, bt, pos0 + T, seed=3)
    q = _append(cache, qkv, pos0, nq, cs, sn).cpu().numpy()
    k_all = cache.k.cpu().numpy()
    v_all = cache.v.cpu().numpy()
    for t in range(T):
        p = pos0 + t
        c, s = cs[p], sn[p]
        x = qkv[t].reshape(nq + 2 * nkv, hd)
        assert np.array_equal(q[t].reshape(nq, hd).view(np.uint32), _rot(x[:nq], c, s).view(np.uint32))
        blk, slot = cache.table_np[p // bt], p % bt
        want_k = _rot(x[nq:nq + nkv], c, s).astype(np.float16)
        want_v = x[nq + nkv:].astype(np.float16)
        assert np.array_equal(k_all[blk, :, slot, :].view(np.uint16), want_k.view(np.uint16)), t
        assert np.array_equal(v_all[blk, :, :, slot].view(np.uint16), want_v.view(np.uint16)), t
    # positions before pos0 were not touched
    assert np.isnan(cache.positions(pos0)[0].astype(np.float32)).all()


def _reference_attention(q, cache, pos0, nq):
    """fp64 causal softmax attention of q (fp32 [T, nq*hd]) over the cache."""
    T, hd, nkv = q.shape[0], cache.hd, cache.nkv
    G = nq // nkv
    K, V = (a.astype(np.float64) for a in cache.positions(pos0 + T))   # [P, nkv, hd]
    out = np.empty((T, nq, hd))
    for t in range(T):
        n = pos0 + t + 1
        for h in range(nq):
            g = h // G
            s = K[:n, g, :] @ q[t, h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
            w = np.exp(s - s.max())
            out[t, h] = (w / w.sum()) @ V[:n, g, :]
    return out.reshape(T, nq * hd), np.abs(V).max()


@pytest.mark.parametrize("nq,nkv", [(4, 2), (7, 1), (28, 4)])
@pytest.mark.parametrize("hd,bt", [(64, 16), (128, 16), (128, 32)])
@pytest.mark.parametrize("T,pos0", [(1, 0), (16, 0), (37, 5), (70, 300)])
def test_chunk_attention_matches_fp64(cuda, nq, nkv, hd, bt, T, pos0):
    cs, sn = _tables(512, hd)
    rng = np.random.default_rng(nq * 1000 + hd + T + pos0)
    cache = Cache(nkv, hd, bt, pos0 + T, seed=nq + T)
    width = (nq + 2 * nkv) * hd
    if pos0:   # earlier positions through the same kernel, as earlier chunks
        _append(cache, rng.standard_normal((pos0, width)).astype(np.float32), 0, nq, cs, sn)
    q = _append(cache, rng.standard_normal((T, width)).astype(np.float32), pos0, nq, cs, sn)
    got = ops.chunk_attention(q, pos0, nq, nkv, hd, cache.k, cache.v, cache.table, bt).cpu().numpy()
    ref, vmax = _reference_attention(q.cpu().numpy(), cache, pos0, nq)
    got = got.astype(np.float64)
    bound = np.abs(ref) * 2.0 ** -11 + 2e-5 * vmax
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))


def test_chunk_attention_rejects_unsupported_shapes(cuda):
    from engine_amd import lib as L
    k = L.kernels()
    shape = 2   # LYK_ERR_SHAPE
    dummy = torch.zeros(64, dtype=torch.float32, device="cuda")
    p = dummy.data_ptr()
    # head dim 96; block tokens 8; positions past the table
    assert k.lyk_hip_chunk_attention(p, p, p, p, 1, 1, 0, 2, 1, 96, 16, 1, p, 192, None) == shape
    assert k.lyk_hip_chunk_attention(p, p, p, p, 1, 1, 0, 2, 1, 64, 8, 1, p, 128, None) == shape
    assert k.lyk_hip_chunk_attention(p, p, p, p, 1, 1, 16, 2, 1, 64, 16, 1, p, 128, None) == shape
    assert k.lyk_hip_chunk_rope_kv(p, 64, 1, 16, 1, 1, 16, p, p, 8, p, p, p, p, 1, 16, 1, None) == shape


# --------------------------------------------------------------- model level
MID = O.QwenConfig(2048, 512, 3, 8, 2, 64, 1408, 1024, 1e-6, 1e6, False, 2047)
MID128 = O.QwenConfig(4096, 896, 2, 7, 1, 128, 2048, 1024, 1e-6, 1e6, True, 4095)


def _prefill_and_follow(hip, prompt, follow):
    """Prefill logits, then teacher-forced Decode logits along `follow`."""
    s = hip.new_seq(len(prompt) + len(follow) + 1)
    code, a = hip.prefill(s, prompt)
    assert code == 0
    out = [a]
    for t in follow:
        code, a = hip.decode(s, t)
        assert code == 0
        out.append(a)
    return out


@pytest.mark.parametrize("cfg", [MID, MID128], ids=["hd64", "hd128"])
@pytest.mark.parametrize("mode", ["int4", "int8"])
def test_chunked_prefill_matches_token_by_token(cuda, cfg, mode):
    """Prompts of 2, 17 and 300 tokens: chunk sizes 2048 (the default, one
    pass), 16 and 37 (many passes, the last one short) give bit-identical
    logits, before and after 6 Decode steps; each within CHUNK_TOL of the
    token-by-token Prefill, greedy tokens equal where the top-2 gap is not a
    tie."""
    runs = {}
    for chunk in (0, 16, 37, -1):
        hip = M.HipModel.synthetic(cfg, seed=5, sigma=0.02, options=M.Options(quant=mode, prefill_chunk=chunk))
        try:
            runs[chunk] = [_prefill_and_follow(hip, list(O.synth_tokens(60 + n, 0, n, cfg.vocab_size)),
                                               [7, 100, 3, 45, 9, 12]) for n in (2, 17, 300)]
        finally:
            hip.close()
    for chunk in (16, 37):
        for a, b in zip(runs[0], runs[chunk]):
            for x, y in zip(a, b):
                assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), chunk
    for a, b in zip(runs[0], runs[-1]):
        for x, y in zip(a, b):
            assert rel_err(x, y) < CHUNK_TOL
            assert O.argmax(x) == O.argmax(y) or top2_gap(y) < 1e-2


def test_chunked_prefill_with_prefix_cache_is_bit_exact(cuda):
    """A prompt whose first 4 blocks come from the prefix cache starts its
    chunk pass at position 64 and gives the logits of the same prompt
    prefilled from position 0, bit for bit."""
    cfg = MID
    hip = M.HipModel.synthetic(cfg, seed=8, sigma=0.02, options=M.Options(quant="int4", prefill_chunk=32))
    try:
        shared = list(O.synth_tokens(9, 0, 70, cfg.vocab_size))
        p1 = shared + [5, 6, 7]
        p2 = shared + [8, 9, 10, 11, 12]
        a = hip.new_seq(128, True, "s")
        assert hip.prefill(a, p1)[0] == 0
        hits = hip.prefix_cache_hit_tokens
        b = hip.new_seq(128, True, "s")
        code, got = hip.prefill(b, p2)
        assert code == 0 and hip.prefix_cache_hit_tokens - hits == 64
        c = hip.new_seq(128)
        code, want = hip.prefill(c, p2)
        assert code == 0
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        hip.close()


def test_prefill_chunk_option_rejected_below_minus_one(cuda):
    with pytest.raises(M.ModelError):
        M.HipModel.synthetic(MID, seed=0, sigma=0.02, options=M.Options(quant="int4", prefill_chunk=-2))
