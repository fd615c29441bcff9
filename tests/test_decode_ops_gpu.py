"""GPU parity of the decode-step kernels (RMSNorm, RoPE + paged KV append,
paged GQA decode attention, greedy argmax) against the CPU oracle, called
through the C ABI of include/lykuro_hip.h."""
import ctypes as C

import numpy as np
import pytest
import torch

import engine_amd.lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def P(t):
    return C.c_void_p(t.data_ptr())


def S():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def rel_err(y, ref):
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def rope_tables(cap, hd, theta):
    """cos/sin exactly as the oracle's ApplyRope computes them."""
    half = hd // 2
    cs = np.zeros((cap, half), np.float32)
    sn = np.zeros((cap, half), np.float32)
    for p in range(cap):
        v = np.zeros(hd, np.float32)
        v[:half] = 1.0
        r = O.rope(v, p, theta)          # rotating (1, 0) gives (cos, sin)
        cs[p], sn[p] = r[:half], r[half:]
    return cs, sn


@pytest.mark.parametrize("m,n", [(1, 16), (3, 896), (4, 3584), (2, 5120)])
def test_rmsnorm_f16(cuda, m, n):
    rng = np.random.default_rng(n)
    h = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    ldx = (n + 31) // 32 * 32
    xn = torch.zeros((m, ldx), dtype=torch.float16, device=cuda)
    hd_, gd = torch.from_numpy(h).to(cuda), torch.from_numpy(g).to(cuda)
    assert L.kernels().lyk_hip_rmsnorm_f16(P(hd_), n, P(gd), 1e-6, m, n, P(xn), ldx, S()) == 0
    out = xn.cpu().numpy()[:, :n].astype(np.float32)
    for i in range(m):
        ref = O.rmsnorm(h[i], g, 1e-6)
        # the sum of squares is a tree on the GPU: allow 1 fp16 ulp
        np.testing.assert_allclose(out[i], O.round_f16(ref), rtol=2 ** -10, atol=1e-7)
    assert torch.all(xn[:, n:] == 0)


def test_embed_rmsnorm(cuda):
    rng = np.random.default_rng(1)
    V, n = 300, 896
    table = rng.standard_normal((V, n)).astype(np.float32)
    g = np.ones(n, np.float32)
    toks = np.array([5, 299, 0], np.int32)
    td, gd, tk = (torch.from_numpy(a).to(cuda) for a in (table, g, toks))
    h = torch.zeros((3, n), device=cuda)
    xn = torch.zeros((3, n), dtype=torch.float16, device=cuda)
    assert L.kernels().lyk_hip_embed_rmsnorm(P(td), V, P(tk), 3, n, P(h), n, P(gd), 1e-6,
                                             P(xn), n, S()) == 0
    np.testing.assert_array_equal(h.cpu().numpy(), table[toks])
    for i, t in enumerate(toks):
        np.testing.assert_allclose(xn[i].cpu().numpy().astype(np.float32),
                                   O.round_f16(O.rmsnorm(table[t], g, 1e-6)), rtol=2 ** -10)


def _paged_pool(rng, ctxs, nkv, hd, bt, extra_blocks=5):
    """Random fp16 K/V for ragged sequences in a pool whose block ids are a
    random permutation."""
    nblk = [(c + bt - 1) // bt for c in ctxs]
    total = sum(nblk) + extra_blocks
    perm = rng.permutation(total).astype(np.int32)
    stride = max(nblk)
    table = np.full((len(ctxs), stride), -1, np.int32)
    at = 0
    for i, nb in enumerate(nblk):
        table[i, :nb] = perm[at:at + nb]
        at += nb
    kc = rng.standard_normal((total, nkv, bt, hd)).astype(np.float16)
    vc = rng.standard_normal((total, nkv, bt, hd)).astype(np.float16)
    return table, kc, vc, total


def _gather(cache, table_row, ctx, bt):
    """[ctx][nkv*hd] fp32 rows of one sequence, the oracle's KV layout."""
    rows = []
    for t in range(ctx):
        rows.append(cache[table_row[t // bt], :, t % bt, :].reshape(-1))
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("nq,nkv,hd,ctxs,splits", [
    (28, 4, 128, None, 16),            # config 3: ragged 4 x U[512, 8192]
    (28, 4, 128, [1, 17, 64, 300], 8),
    (14, 2, 64, [33, 2, 129], 1),      # 0.5B geometry, no split
    (40, 8, 128, [700, 1500], 32),     # 14B geometry
    (4, 2, 4, [1, 5, 20], 3),          # tiny fixture geometry (hd 4)
])
def test_attention_matches_oracle(cuda, nq, nkv, hd, ctxs, splits):
    rng = np.random.default_rng(nq * 7 + hd)
    if ctxs is None:
        ctxs = [int(c) for c in rng.integers(512, 8193, 4)]
    bt = 16
    m = len(ctxs)
    table, kc, vc, total = _paged_pool(rng, ctxs, nkv, hd, bt)
    q = rng.standard_normal((m, nq * hd)).astype(np.float32)
    pos = np.array([c - 1 for c in ctxs], np.int32)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(cuda) for k, v in
         dict(q=q, kc=kc.view(np.uint16), vc=vc.view(np.uint16), table=table, pos=pos).items()}
    out = torch.zeros((m, nq * hd), dtype=torch.float16, device=cuda)
    wsb = L.kernels().lyk_hip_attn_workspace_bytes(m, nq, nkv, hd, splits)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=cuda)
    rc = L.kernels().lyk_hip_attn_decode(P(d["q"]), P(d["kc"]), P(d["vc"]), P(d["table"]),
                                         table.shape[1], P(d["pos"]), m, nq, nkv, hd, bt, total,
                                         splits, P(out), nq * hd, P(ws), wsb, S())
    assert rc == 0
    got = out.cpu().numpy().astype(np.float32)
    for i, c in enumerate(ctxs):
        keys = _gather(kc, table[i], c, bt)
        vals = _gather(vc, table[i], c, bt)
        ref = O.attention(q[i], keys, vals, nq, nkv, hd)
        e = rel_err(got[i], ref)
        assert e < 1e-3, f"seq {i} ctx {c}: {e:.2e}"
    assert torch.count_nonzero(ws) == 0, "workspace must be left zeroed"
    # deterministic
    out2 = torch.zeros_like(out)
    L.kernels().lyk_hip_attn_decode(P(d["q"]), P(d["kc"]), P(d["vc"]), P(d["table"]),
                                    table.shape[1], P(d["pos"]), m, nq, nkv, hd, bt, total, splits,
                                    P(out2), nq * hd, P(ws), wsb, S())
    assert torch.equal(out, out2)


@pytest.mark.parametrize("nq,nkv,hd", [(28, 4, 128), (14, 2, 64), (4, 2, 4)])
def test_rope_kv_append_bit_exact(cuda, nq, nkv, hd):
    rng = np.random.default_rng(hd)
    m, bt, cap, theta = 3, 16, 300, 1e6
    pos = np.array([0, 17, 299], np.int32)
    nblocks = 64
    table = rng.permutation(nblocks)[: m * 19].reshape(m, 19).astype(np.int32)
    qkv = rng.standard_normal((m, (nq + 2 * nkv) * hd)).astype(np.float32)
    cs, sn = rope_tables(cap, hd, theta)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(cuda)
         for k, v in dict(qkv=qkv, pos=pos, cs=cs, sn=sn, table=table).items()}
    qo = torch.zeros((m, nq * hd), device=cuda)
    kc = torch.zeros((nblocks, nkv, bt, hd), dtype=torch.int16, device=cuda)
    vc = torch.zeros_like(kc)
    rc = L.kernels().lyk_hip_rope_kv_append(P(d["qkv"]), qkv.shape[1], m, nq, nkv, hd, P(d["pos"]),
                                            P(d["cs"]), P(d["sn"]), cap, P(qo), P(kc), P(vc),
                                            P(d["table"]), 19, bt, nblocks, S())
    assert rc == 0
    qo, kc, vc = qo.cpu().numpy(), kc.cpu().numpy().view(np.uint16), vc.cpu().numpy().view(np.uint16)
    for i in range(m):
        p = int(pos[i])
        blk, slot = table[i, p // bt], p % bt
        for h in range(nq):
            ref = O.rope(qkv[i, h * hd:(h + 1) * hd], p, theta)
            np.testing.assert_array_equal(qo[i, h * hd:(h + 1) * hd].view(np.uint32), ref.view(np.uint32))
        for h in range(nkv):
            k = qkv[i, (nq + h) * hd:(nq + h + 1) * hd]
            v = qkv[i, (nq + nkv + h) * hd:(nq + nkv + h + 1) * hd]
            np.testing.assert_array_equal(kc[blk, h, slot], O.f32_to_f16_bits(O.rope(k, p, theta)))
            np.testing.assert_array_equal(vc[blk, h, slot], O.f32_to_f16_bits(v))


@pytest.mark.parametrize("m,n", [(1, 32), (1, 152064), (3, 151936), (4, 4097), (2, 1)])
def test_argmax_greedy_rule(cuda, m, n):
    rng = np.random.default_rng(n + m)
    logits = rng.standard_normal((m, n)).astype(np.float32)
    if n > 10:
        logits[0, [7, n - 3]] = 50.0                 # tie: lowest index wins
        logits[-1, 2] = np.nan                       # NaN never wins
        logits[-1, 3] = np.inf                       # +inf wins and is counted
    ld = torch.from_numpy(logits).to(cuda)
    toks = torch.zeros(m, dtype=torch.int32, device=cuda)
    bad = torch.zeros(m, dtype=torch.int32, device=cuda)
    wsb = L.kernels().lyk_hip_argmax_workspace_bytes(m, n)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=cuda)
    rc = L.kernels().lyk_hip_argmax(P(ld), n, m, n, P(toks), P(bad), None, None, None, P(ws), wsb, S())
    assert rc == 0
    t = toks.cpu().numpy()
    for i in range(m):
        row = logits[i].copy()
        if np.isfinite(row).all():
            assert t[i] == O.argmax(row)
        else:
            assert t[i] == 3
    if n > 10:
        assert t[0] == (3 if m == 1 else 7)
        assert bad.cpu().numpy()[-1] == 2
    assert torch.count_nonzero(ws) == 0


def test_argmax_greedy_chain_history(cuda):
    """Single-row chaining used by GreedyRun: token, position advance,
    history append at *step."""
    n = 1000
    rng = np.random.default_rng(9)
    tokens = torch.zeros(1, dtype=torch.int32, device=cuda)
    pos = torch.tensor([10], dtype=torch.int32, device=cuda)
    hist = torch.zeros(8, dtype=torch.int32, device=cuda)
    step = torch.zeros(1, dtype=torch.int32, device=cuda)
    wsb = L.kernels().lyk_hip_argmax_workspace_bytes(1, n)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=cuda)
    want = []
    for s in range(5):
        logits = rng.standard_normal(n).astype(np.float32)
        want.append(O.argmax(logits))
        ld = torch.from_numpy(logits).to(cuda)
        assert L.kernels().lyk_hip_argmax(P(ld), n, 1, n, P(tokens), None, P(pos), P(hist), P(step),
                                          P(ws), wsb, S()) == 0
    assert hist.cpu().numpy()[:5].tolist() == want
    assert int(step.item()) == 5 and int(pos.item()) == 15 and int(tokens.item()) == want[-1]
