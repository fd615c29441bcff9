"""Pins the CPU oracle (oracle/qwen_oracle.c) before anything is checked
against it: the reference's own golden values and KATs, the published
mt19937_64 output, closed-form properties, and bit equality with the
reference CPU path compiled from its sources (oracle/_ref) where it is built."""
import math
import os
import tempfile

import numpy as np
import pytest

from oracle import oracle as O

MID = O.QwenConfig(512, 128, 2, 4, 2, 32, 256, 96, 1e-6, 1e6, False, 511)


def fill_synthetic(model, seed=0, sigma=0.02):
    """Seeded N(0, sigma) weights, norms 1.0, biases N(0, sigma)."""
    for kind, layer, arr in model.tensors():
        if kind in (O.T_INPUT_NORM, O.T_POST_NORM, O.T_FINAL_NORM):
            arr[...] = 1.0
        else:
            stream = kind * 1000 + layer
            arr[...] = O.synth_normal(seed, stream, arr.size, sigma).reshape(arr.shape)


# ------------------------------------------------------------- golden values
def test_golden_prefill_then_greedy(golden):
    g = golden["prefill_then_10_greedy"]
    m = O.OracleModel(O.TINY)
    m.fill_tiny(golden["tiny_model"]["seed"])
    s = m.new_seq(64)
    code, logits = m.prefill(s, g["prompt"])
    assert code == O.OK
    for _ in range(g["steps"]):
        code, logits = m.decode(s, O.argmax(logits))
        assert code == O.OK
    np.testing.assert_allclose(logits[:5], g["logits_0_to_4"], atol=g["tolerance"], rtol=0)


def test_golden_greedy_sequences(golden):
    m = O.OracleModel(O.TINY)
    m.fill_tiny(golden["tiny_model"]["seed"])
    for case in golden["greedy_sequences"]["cases"]:
        s = m.new_seq(64)
        code, logits = m.prefill(s, case["prompt"])
        out = []
        for _ in case["expected"]:
            t = O.argmax(logits)
            out.append(t)
            code, logits = m.decode(s, t)
            assert code == O.OK
        assert out == case["expected"]


def test_error_semantics():
    """qwen_model.cpp:336-352, 400-407."""
    m = O.OracleModel(O.TINY)
    m.fill_tiny(42)
    assert m.prefill(m.new_seq(4), [])[0] == O.INVALID_REQUEST
    assert m.prefill(m.new_seq(4), [1] * 5)[0] == O.CONTEXT_LENGTH_EXCEEDED
    assert m.prefill(m.new_seq(4), [40])[0] == O.INVALID_REQUEST
    s = m.new_seq(2)
    assert m.prefill(s, [1, 2])[0] == O.OK
    assert m.prefill(s, [1])[0] == O.INTERNAL_ERROR
    assert m.decode(s, 3)[0] == O.CONTEXT_LENGTH_EXCEEDED
    assert m.decode(m.new_seq(8), 99)[0] == O.INVALID_REQUEST


def test_non_finite_logits_fail():
    """qwen_model.cpp:322-329: a NaN weight surfaces as inference_failed."""
    m = O.OracleModel(O.TINY)
    m.fill_tiny(42)
    m.tensor(O.T_FINAL_NORM)[3] = np.nan
    assert m.prefill(m.new_seq(8), [1, 2])[0] == O.INFERENCE_FAILED


def test_incremental_decode_equals_prefill():
    """qwen_model_test.cpp:171-186 pattern: prefill(p + [t]) == prefill(p) + decode(t)."""
    m = O.OracleModel(O.TINY)
    m.fill_tiny(42)
    _, a = m.prefill(m.new_seq(16), [4, 8, 15, 16])
    s = m.new_seq(16)
    m.prefill(s, [4, 8, 15])
    _, b = m.decode(s, 16)
    np.testing.assert_allclose(a, b, atol=1e-4)


# ------------------------------------------------------------------- codecs
def test_dtype_kats(golden):
    d = golden["dtype"]
    L = O.lib()
    for v in d["bf16_exact"]:
        assert L.orc_bf16_to_f32(L.orc_f32_to_bf16(v)) == v
    for v in d["fp16_exact"]:
        assert L.orc_f16_to_f32(L.orc_f32_to_f16(v)) == v
    sub = d["fp16_smallest_subnormal"]
    assert L.orc_f16_to_f32(L.orc_f32_to_f16(sub)) == np.float32(sub)
    halfway = 1.0 + 2.0 ** -9
    assert L.orc_bf16_to_f32(L.orc_f32_to_bf16(halfway)) == d["bf16_halfway_1_plus_2m9_rounds_to"]
    assert math.isinf(L.orc_f16_to_f32(L.orc_f32_to_f16(1e6)))
    assert math.isnan(L.orc_f16_to_f32(L.orc_f32_to_f16(float("nan"))))
    assert math.isinf(L.orc_bf16_to_f32(L.orc_f32_to_bf16(float("inf"))))


def test_fp16_exhaustive_against_numpy():
    """All 2^16 halves decode like numpy's IEEE float16; encoding every decoded
    value and its neighbours midway rounds like numpy (round-half-even)."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = O.f16_bits_to_f32(bits)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    # encode: random float32 bit patterns plus exact midpoints
    rng = np.random.default_rng(0)
    xs = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    a = ref[finite & (np.abs(ref) < 65504)].astype(np.float64)
    mids = ((a[:-1] + a[1:]) / 2).astype(np.float32)
    xs = np.concatenate([xs, mids, ref[finite]])
    xs = xs[~np.isnan(xs)]
    enc = O.f32_to_f16_bits(xs)
    with np.errstate(over="ignore"):
        expect = xs.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(enc, expect)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_codecs_equal_reference_build():
    R = O.ref_lib()
    L = O.lib()
    rng = np.random.default_rng(1)
    for u in rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64):
        f = float(np.uint32(u).view(np.float32))
        if math.isnan(f):
            continue
        assert L.orc_f32_to_f16(f) == R.ref_f32_to_f16(f)
        assert L.orc_f32_to_bf16(f) == R.ref_f32_to_bf16(f)
    for h in range(1 << 16):
        a, b = L.orc_f16_to_f32(h), R.ref_f16_to_f32(h)
        assert (a == b) or (math.isnan(a) and math.isnan(b))


# ------------------------------------------------------------------ sampler
def test_mt19937_64_published_output(golden):
    import ctypes as C
    g = (C.c_uint64 * 313)()
    L = O.lib()
    L.orc_mt64_seed(g, golden["mt19937_64"]["seed"])
    for _ in range(9999):
        L.orc_mt64_next(g)
    assert L.orc_mt64_next(g) == golden["mt19937_64"]["output_10000"]


def test_sampler_reference_cases(golden):
    s = golden["sampler"]
    assert O.Sampler(0.0).sample(s["greedy_argmax"]["logits"]) == (0, s["greedy_argmax"]["expected"])
    assert O.Sampler(0.0).sample(s["greedy_tie"]["logits"]) == (0, s["greedy_tie"]["expected"])
    c = s["top_k"]
    sm = O.Sampler(c["temperature"], 1.0, c["top_k"], c["seed"])
    assert all(sm.sample(c["logits"])[1] in c["allowed"] for _ in range(c["draws"]))
    c = s["small_top_p"]
    sm = O.Sampler(c["temperature"], c["top_p"], 0, c["seed"])
    assert all(sm.sample(c["logits"])[1] == c["expected"] for _ in range(c["draws"]))
    c = s["reproducible"]
    a = O.Sampler(c["temperature"], 1.0, 0, c["seed"])
    b = O.Sampler(c["temperature"], 1.0, 0, c["seed"])
    assert [a.sample(c["logits"])[1] for _ in range(20)] == [b.sample(c["logits"])[1] for _ in range(20)]
    assert O.Sampler().sample([1.0, float("inf")])[0] == O.INFERENCE_FAILED
    assert O.Sampler().sample([1.0, float("nan")])[0] == O.INFERENCE_FAILED
    assert O.Sampler().sample(np.zeros(0, np.float32))[0] == O.INFERENCE_FAILED


def test_sampler_distribution_matches_softmax():
    """Closed form: with top_p=1, top_k=0 the token frequencies follow
    softmax(logits/T)."""
    logits = np.array([0.5, 1.5, -0.3, 1.0], np.float32)
    sm = O.Sampler(0.7, 1.0, 0, 99)
    counts = np.bincount([sm.sample(logits)[1] for _ in range(40000)], minlength=4)
    p = np.exp(logits / 0.7) / np.exp(logits / 0.7).sum()
    np.testing.assert_allclose(counts / counts.sum(), p, atol=0.01)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_sampler_equals_reference_build():
    rng = np.random.default_rng(0)
    for trial in range(200):
        n = int(rng.integers(1, 2000))
        logits = (rng.standard_normal(n) * 3).astype(np.float32)
        if trial % 4 == 0:
            logits = np.round(logits).astype(np.float32)  # many ties
        T = float(rng.choice([0.0, 0.3, 1.0, 1.7]))
        p = float(rng.choice([1.0, 0.9, 0.5, 0.01]))
        k = int(rng.choice([0, 1, 5, 1024]))
        seed = int(rng.integers(0, 2 ** 63))
        a, b = O.Sampler(T, p, k, seed), O.RefSampler(T, p, k, seed)
        for _ in range(4):
            assert a.sample(logits) == b.sample(logits)


# --------------------------------------------------------------- quantizers
def test_q4_closed_form_properties():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((37, 100)) * 0.02).astype(np.float32)
    w[5, 32:64] = 0.0                      # all-zero group -> scale 1.0
    w[6, :] *= 1e-9                        # tiny scale (fp16 subnormal)
    codes, scales = O.q4_quantize(w)
    assert codes.min() >= -8 and codes.max() <= 7
    s = O.f16_bits_to_f32(scales)
    assert scales[5, 1] == 0x3C00 and np.all(codes[5, 32:64] == 0)
    deq = O.q4_dequantize(codes, scales)
    # exactness: q*s with |q|<=8 and an fp16 s is exact in fp32
    sexp = np.repeat(s, 32, axis=1)[:, :100]
    np.testing.assert_array_equal(deq, codes.astype(np.float64) * sexp)
    # error bound: |w - q s| <= s/2 unless clamped at -8 (never for |w|<=7s)
    assert np.all(np.abs(w - deq) <= sexp * 0.5 + 1e-12)
    # brute force: each code is the nearest integer in [-8,7] to w/s
    for r in range(0, 37, 7):
        for c in range(100):
            cand = np.arange(-8, 8)
            best = cand[np.argmin(np.abs(w[r, c] - cand * sexp[r, c]))]
            assert abs(codes[r, c] - best) <= 0 or np.isclose(
                abs(w[r, c] - codes[r, c] * sexp[r, c]), abs(w[r, c] - best * sexp[r, c]))


def test_q8_closed_form_properties():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((20, 77)) * 0.02).astype(np.float32)
    codes, scales = O.q8_quantize(w)
    assert codes.min() >= -127 and codes.max() <= 127
    s = O.f16_bits_to_f32(scales)
    deq = O.q8_dequantize(codes, scales)
    np.testing.assert_array_equal(deq, codes.astype(np.float64) * s[:, None])
    assert np.all(np.abs(w - deq) <= s[:, None] * 0.5 * (1 + 1e-6))
    # the scale is fp16(absmax/127): the absmax element maps to +-127 or +-126
    amax = np.abs(w).argmax(axis=1)
    assert np.all(np.abs(codes[np.arange(20), amax]) >= 126)


# ------------------------------------------------------ synthetic generator
def test_synth_normal_moments():
    v = O.synth_normal(7, 3, 1_000_000, 1.0)
    assert abs(v.mean()) < 0.005 and abs(v.std() - 1.0) < 0.005
    assert abs((v ** 4).mean() - 3.0) < 0.05  # kurtosis of a normal
    # counter-based: any window equals the same slice of the full stream
    np.testing.assert_array_equal(O.synth_normal(7, 3, 1000, 1.0, first=12345), v[12345:13345])


# ------------------------------------------ oracle vs compiled reference
def _model_pair(cfg, fill):
    m = O.OracleModel(cfg)
    fill(m)
    path = os.path.join(tempfile.mkdtemp(), "m.safetensors")
    O.model_to_safetensors(m, path)
    return m, O.RefModel(cfg, path), path


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("which", ["tiny_parity", "mid"])
def test_oracle_bit_equal_to_reference_build(which):
    if which == "tiny_parity":
        cfg, fill = O.TINY_PARITY, (lambda m: m.fill_tiny(42))
        prompt = [1, 5, 9, 2, 17, 250]
    else:
        cfg, fill = MID, (lambda m: fill_synthetic(m, seed=1))
        prompt = list(O.synth_tokens(0, 1, 20, cfg.vocab_size))
    m, r, path = _model_pair(cfg, fill)
    try:
        s, rs = m.new_seq(64), r.new_seq(64)
        a, b = m.prefill(s, prompt), r.prefill(rs, prompt)
        assert a[0] == b[0] == 0 and np.array_equal(a[1], b[1])
        logits = a[1]
        for _ in range(30):
            t = O.argmax(logits)
            a, b = m.decode(s, t), r.decode(rs, t)
            assert a[0] == b[0] == 0 and np.array_equal(a[1], b[1])
            logits = a[1]
        # error paths agree too
        assert m.decode(s, cfg.vocab_size)[0] == r.decode(rs, cfg.vocab_size)[0]
    finally:
        os.remove(path)


def test_threaded_matvec_bit_identical():
    rng = np.random.default_rng(5)
    w = rng.standard_normal((1000, 700)).astype(np.float32)
    x = rng.standard_normal(700).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(O.matvec(w, x, b, threads=1), O.matvec(w, x, b, threads=7))


def test_threaded_attention_bit_identical():
    rng = np.random.default_rng(6)
    heads, kvh, hd, ctx = 28, 4, 128, 300
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal((ctx, kvh * hd)).astype(np.float32)
    v = rng.standard_normal((ctx, kvh * hd)).astype(np.float32)
    np.testing.assert_array_equal(O.attention(q, k, v, heads, kvh, hd),
                                  O.attention(q, k, v, heads, kvh, hd, threads=5))


def test_model_threads_bit_identical():
    """The forward with matvec rows and attention heads spread over threads
    equals the single-threaded forward (which equals oracle/_ref) bit for bit;
    the context is long enough for the threaded attention path."""
    cfg = O.QwenConfig(512, 256, 1, 8, 2, 64, 512, 700, 1e-6, 1e6, False, 511)
    outs = []
    for threads in (1, 6):
        m = O.OracleModel(cfg, threads)
        fill_synthetic(m, seed=4)
        s = m.new_seq(cfg.max_context_tokens)
        code, logits = m.prefill(s, list(O.synth_tokens(3, 0, 600, cfg.vocab_size)))
        assert code == 0
        outs.append(logits)
    np.testing.assert_array_equal(outs[0], outs[1])


# ------------------------------------------------------------ fp16 mirror
_LIBM = None


def _expf(x):
    """glibc's expf, the function the oracle's SiLU calls."""
    global _LIBM
    import ctypes
    if _LIBM is None:
        _LIBM = ctypes.CDLL("libm.so.6")
        _LIBM.expf.restype, _LIBM.expf.argtypes = ctypes.c_float, [ctypes.c_float]
    return np.array([_LIBM.expf(float(v)) for v in x], np.float32)


def _descending(w, x, b=None):
    """orc_matvec with the products added in descending index order: the
    pinned primitive on reversed columns and input."""
    return O.matvec(np.ascontiguousarray(w[:, ::-1]), np.ascontiguousarray(x[::-1]), b)


def _mirror_composition(m, tokens, matvec=O.matvec, mirror=True):
    """One sequence through qwen_model.cpp:212-331, composed from the pinned
    primitives (orc_matvec, orc_rmsnorm, orc_rope, orc_attention), with the
    pinned fp16 codec applied at exactly the five mirror points (none when
    mirror is False). Logits after every token."""
    c = m.cfg
    r16 = O.round_f16 if mirror else (lambda v: v)
    O_matvec = matvec
    hd, nq, nkv = c.head_dim, c.num_heads, c.num_kv_heads
    T = lambda kind, l=0: m.tensor(kind, l)
    keys = [np.zeros((len(tokens), nkv * hd), np.float32) for _ in range(c.num_layers)]
    vals = [np.zeros((len(tokens), nkv * hd), np.float32) for _ in range(c.num_layers)]
    out = []
    for pos, tok in enumerate(tokens):
        hidden = T(O.T_EMBED)[tok].copy()
        for l in range(c.num_layers):
            x = r16(O.rmsnorm(hidden, T(O.T_INPUT_NORM, l), c.rms_norm_eps))
            q = O_matvec(T(O.T_Q_W, l), x, T(O.T_Q_B, l))
            k = O_matvec(T(O.T_K_W, l), x, T(O.T_K_B, l))
            v = O_matvec(T(O.T_V_W, l), x, T(O.T_V_B, l))
            q = np.concatenate([O.rope(q[h * hd:(h + 1) * hd], pos, c.rope_theta) for h in range(nq)])
            k = np.concatenate([O.rope(k[h * hd:(h + 1) * hd], pos, c.rope_theta) for h in range(nkv)])
            keys[l][pos], vals[l][pos] = r16(k), r16(v)
            attn = r16(O.attention(q, keys[l][:pos + 1], vals[l][:pos + 1], nq, nkv, hd))
            hidden = (hidden + O_matvec(T(O.T_O_W, l), attn)).astype(np.float32)
            x = r16(O.rmsnorm(hidden, T(O.T_POST_NORM, l), c.rms_norm_eps))
            g = O_matvec(T(O.T_GATE_W, l), x)
            u = O_matvec(T(O.T_UP_W, l), x)
            act = r16(g / (np.float32(1.0) + _expf(-g)) * u)
            hidden = (hidden + O_matvec(T(O.T_DOWN_W, l), act)).astype(np.float32)
        x = r16(O.rmsnorm(hidden, T(O.T_FINAL_NORM), c.rms_norm_eps))
        head = T(O.T_EMBED) if c.tie_word_embeddings else T(O.T_LM_HEAD)
        out.append(O_matvec(head, x))
    return out


@pytest.mark.parametrize("cfg", [MID, O.QwenConfig(300, 96, 2, 6, 2, 16, 160, 64, 1e-6, 1e4, True, 299)],
                         ids=["untied", "tied"])
def test_f16_mirror_equals_composition_of_pinned_primitives(cfg):
    """Pins the oracle's fp16 mirror mode: token by token, its logits equal a
    composition of the already-pinned primitives with fp16 rounding (the
    pinned codec) at the RMSNorm outputs, the cached K and V, the attention
    output and SiLU(gate)*up -- bit for bit. Mirror and plain forwards differ
    (so rounding really happens there) by no more than fp16 rounding can
    explain."""
    m = O.OracleModel(cfg, 3)
    fill_synthetic(m, seed=7)
    tokens = list(O.synth_tokens(8, 0, 12, cfg.vocab_size))
    want = _mirror_composition(m, tokens)
    m.set_f16_mirror(True)
    s = m.new_seq(64)
    got = [m.prefill(s, tokens[:1])[1]] + [m.decode(s, t)[1] for t in tokens[1:]]
    for i, (a, b) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(a, b, err_msg=f"token {i}")
    m.set_f16_mirror(False)
    s = m.new_seq(64)
    plain = [m.prefill(s, tokens[:1])[1]] + [m.decode(s, t)[1] for t in tokens[1:]]
    d = max(float(np.linalg.norm(a - b) / np.linalg.norm(b)) for a, b in zip(got, plain))
    assert 0 < d < 1e-2, d


def test_parallel_helpers_equal_serial_calls():
    """The wrapper spreads synthesis and quantization over threads; each
    equals one serial call of the C function."""
    import ctypes as C
    n = (3 << 20) + 77
    serial = np.empty(n, np.float32)
    O.lib().orc_synth_normal(9, 1234, 5, n, 0.02, serial.ctypes.data_as(C.c_void_p))
    np.testing.assert_array_equal(O.synth_normal(9, 1234, n, 0.02, first=5), serial)
    w = O.synth_normal(1, 2, 700 * 3000, 0.02).reshape(700, 3000)
    for q, dq, ns in ((O.lib().orc_q4_quantize, O.lib().orc_q4_dequantize, (3000 + 31) // 32),
                      (O.lib().orc_q8_quantize, O.lib().orc_q8_dequantize, None)):
        codes = np.empty(w.shape, np.int8)
        scales = np.empty((700, ns) if ns else (700,), np.uint16)
        q(w.ctypes.data_as(C.c_void_p), 700, 3000, codes.ctypes.data_as(C.c_void_p),
          scales.ctypes.data_as(C.c_void_p))
        out = np.empty(w.shape, np.float32)
        dq(codes.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p), 700, 3000,
           out.ctypes.data_as(C.c_void_p))
        mode = "int4" if ns else "int8"
        c2, s2 = O.q4_quantize(w) if ns else O.q8_quantize(w)
        np.testing.assert_array_equal(c2, codes)
        np.testing.assert_array_equal(s2, scales)
        np.testing.assert_array_equal(O.quant_dequant(w, mode), out)


@pytest.mark.parametrize("mirror", [False, True], ids=["plain", "mirror"])
def test_descending_sums_equal_composition_on_reversed_inputs(mirror):
    """Pins the noise-floor mode: with descending sums the forward equals the
    composition whose every matvec is the pinned orc_matvec on reversed
    columns and input, bit for bit; and it differs from the ascending
    (reference-order) forward by no more than fp32 summation order (plain)
    or fp16 rounding flips (mirror) can explain."""
    cfg = MID
    m = O.OracleModel(cfg, 3)
    fill_synthetic(m, seed=8)
    tokens = list(O.synth_tokens(8, 1, 10, cfg.vocab_size))
    want = _mirror_composition(m, tokens, _descending, mirror)
    m.set_f16_mirror(mirror)
    m.set_descending_sums(True)
    s = m.new_seq(64)
    got = [m.prefill(s, tokens[:1])[1]] + [m.decode(s, t)[1] for t in tokens[1:]]
    for i, (a, b) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(a, b, err_msg=f"token {i}")
    m.set_descending_sums(False)
    s = m.new_seq(64)
    asc = [m.prefill(s, tokens[:1])[1]] + [m.decode(s, t)[1] for t in tokens[1:]]
    d = max(float(np.linalg.norm(a - b) / np.linalg.norm(b)) for a, b in zip(got, asc))
    assert 0 < d < (5e-3 if mirror else 1e-5), d
