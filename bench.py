"""Decode throughput of the hip backend: Qwen2.5-7B-architecture INT4
weight-only decode at batch 1 on one MI355X (BASELINE.json metric, config 4).

  python bench.py [--steps K] [--warmup W] [--prompt P] [--quant int4|int8]

A step is one decode token of one sequence: one launch of the fused decode
step kernel (every layer, the LM head and the on-device greedy argmax),
chained by GreedyRun. Weights are random-init N(0, 0.02) (synthetic, no
checkpoint) quantized at load; the prompt is P uniform random token ids.
One JSON line is printed:
  value        decode tokens/s (whole job; one GPU)
  prefill      time to first token of the P-token prompt (chunk passes on the
               matrix cores, then the last token through the fused step)
  phases       one traced step after the timed ones: per layer-phase span (us,
               mean over the middle layers) and GB/s of its weights, and the
               GEMV time-weighted fraction of peak (sum of the GEMV phases'
               weight bytes / sum of their spans / 8 TB/s)
  roofline     the dominant (only) kernel of a step, decode_step_kernel:
               algorithmic HBM bytes of one launch (packed GEMV weights and
               scales + K/V of the context, fp16) / its average duration,
               from HIP events on the model's stream around the timed steps
  cpu_baseline the reference engine's own CPU QwenModel (oracle/_ref), single
               thread as the reference runs it, on a bounded sample (see
               cpu_baseline.sample) at the GPU run's mean context; the C
               restatement (oracle) if _ref is absent
  roofline.traffic  HBM bytes per launch measured by rocprofv3 (FETCH_SIZE +
               WRITE_SIZE, calibrated on a plain copy), read from
               profiles/decode_step_traffic.json when that file was measured on
               the same kernel and workload (bench_profile.py writes it); else null
Only N=1 is supported: this build targets one GPU.

  python bench.py --gemv
times the isolated INT4 GEMV kernel (gemv.hip) at the four Qwen2.5-7B shapes
of BASELINE config 2, M = 1, 2, 4, rotating over >= 512 MB of weight copies
(2x the 256 MB MALL) so that every call reads HBM; one JSON line.

  python bench.py --rows 4 [--model 7b|14b] [--quant int4|int8]
BASELINE config 4's max_sequences=4 leg (config 5's decode leg with --model
14b --quant int8 --prompts 256,1024,2048,4096): R sequences prefilled with
their prompts, then K DecodeBatch steps of all R rows (logits to the host,
greedy picks on the host, as a DecodeBatch caller does); one JSON line with
aggregate tokens/s, the step kernel's time per launch from HIP events, and
each prompt's time to first token.

  python bench.py --copy-calibration
copies 1 GiB device to device 4 times (the runtime's plain copy kernel): the
known-size reference that bench_profile.py scales the HBM counters by.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, published
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_step_traffic.json")
COPY_BYTES = 1 << 30


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ decode
def run_decode(args):
    import torch
    from engine_amd import model as M

    cfg = M.QWEN25_7B
    t0 = time.time()
    opts = M.Options(quant=args.quant, kv_pool_tokens=args.prompt + args.warmup + args.steps + 512,
                     prefill_chunk=args.prefill_chunk)
    hip = M.HipModel.synthetic(cfg, seed=0, sigma=0.02, options=opts)
    log(f"[bench] load (synthetic 7B, {args.quant}) {time.time() - t0:.1f}s, "
        f"GEMV bytes/token {hip.gemv_weight_bytes / 1e9:.3f} GB")
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, cfg.vocab_size, args.prompt).astype(np.uint32)
    seq = hip.new_seq(args.prompt + args.warmup + args.steps + 8)
    # a warm-up prefill of another sequence first (first-launch costs)
    warm = hip.new_seq(64)
    assert hip.prefill(warm, prompt[:40])[0] == 0
    warm.close()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    code, logits = hip.prefill(seq, prompt)
    torch.cuda.synchronize()
    ttft = time.perf_counter() - t0
    assert code == 0, f"prefill failed with code {code}"
    log(f"[bench] prefill {args.prompt} tokens {ttft * 1e3:.1f} ms ({args.prompt / ttft:.0f} tok/s)")
    tok = int(np.argmax(logits))

    def greedy(n, tok):
        out = []
        while len(out) < n:
            code, toks = hip.greedy_run(seq, tok, min(256, n - len(out)))
            assert code == 0 and toks, f"greedy run failed with code {code}"
            out += toks
            tok = toks[-1]
        return out, tok

    if args.warmup:
        _, tok = greedy(args.warmup, tok)
    stream = torch.cuda.ExternalStream(hip.stream_ptr)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ctx0 = seq.length
    t0 = time.perf_counter()
    e0.record(stream)
    toks, tok = greedy(args.steps, tok)
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    kernel_us = e0.elapsed_time(e1) * 1e3 / args.steps
    ctx = seq.length
    # algorithmic bytes of one step: the packed GEMV weights + scales, plus
    # K and V (fp16) of the mean context over the timed steps
    kv_per_ctx = cfg.num_layers * 2 * cfg.num_kv_heads * cfg.head_dim * 2
    step_bytes = hip.gemv_weight_bytes + kv_per_ctx * (ctx0 + ctx + 1) / 2
    gemv_bytes = hip.gemv_weight_bytes
    phases = phase_breakdown(hip, seq, tok, cfg, args.quant)
    hip.close()
    return dict(tok_s=args.steps / dt, ms=dt * 1e3 / args.steps, ctx_end=ctx, ctx_mean=(ctx0 + ctx) / 2,
                kernel_us=kernel_us, step_bytes=step_bytes, gemv_bytes=gemv_bytes, tokens=toks,
                ttft_ms=ttft * 1e3, phases=phases)


def phase_breakdown(hip, seq, tok, cfg, quant):
    """One traced GreedyRun step: per phase kind, the mean span over the
    middle layers (from the previous phase done on every workgroup to this
    one done on every workgroup; the spans of a step add up to the step),
    the bytes the phase must read (its packed weights and scales; attention:
    K and V of the context) and their rate; the LM head alone."""
    from engine_amd import lib as L
    import ctypes as C
    k = L.kernels()
    q8 = 1 if quant == "int8" else 0
    H, In, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    kq, kvd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim

    def packed(n, kk, paired, normed):
        tr = k.lyk_hip_step_tile_rows(n, kk, paired, q8, normed)
        wb, sb = C.c_uint64(), C.c_uint64()
        lay = k.lyk_q8_layout_tiled if q8 else k.lyk_q4_layout_tiled
        L.check("layout_tiled", lay(n, kk, paired, tr, C.byref(wb), C.byref(sb)))
        return wb.value + sb.value

    ctx = seq.length + 1
    nbytes = {"qkv": packed(kq + 2 * kvd, H, 0, 1), "attn": 2 * ctx * kvd * 2, "o": packed(H, kq, 0, 0),
              "gate_up": packed(In, H, 1, 1), "down": packed(H, In, 0, 0), "lm_head": packed(V, H, 0, 1)}
    hip.set_step_tracing(True)
    code, _ = hip.greedy_run(seq, tok, 1)
    assert code == 0
    grid = k.lyk_hip_step_grid()
    Lyr = cfg.num_layers
    nph = 5 * Lyr + 2
    tr = hip.step_trace()[: grid * (4 * nph + 2)].reshape(grid, 4 * nph + 2).astype(np.int64)
    hip.set_step_tracing(False)
    t0 = tr[:, 0].min()
    done = (tr[:, 2:].reshape(grid, nph, 4)[:, :, 3].max(0) - t0) / 100.0   # us (100 MHz)
    names = ["qkv", "attn", "o", "gate_up", "down"]
    out = {}
    for j, n in enumerate(names):
        spans = [done[5 * l + j] - done[5 * l + j - 1] for l in range(2, Lyr - 1)]
        us = float(np.mean(spans))
        out[n] = {"us": round(us, 2), "bytes": nbytes[n], "gbs": round(nbytes[n] / (us * 1e3), 1)}
    us = float(done[5 * Lyr] - done[5 * Lyr - 1])
    out["lm_head"] = {"us": round(us, 2), "bytes": nbytes["lm_head"], "gbs": round(nbytes["lm_head"] / (us * 1e3), 1)}
    gemv = ["qkv", "o", "gate_up", "down"]
    gb = sum(out[n]["bytes"] for n in gemv) * Lyr + out["lm_head"]["bytes"]
    gt = sum(out[n]["us"] for n in gemv) * Lyr + out["lm_head"]["us"]
    return {"per_layer": out, "step_us_traced": round(float(done[nph - 1]), 1),
            "gemv_time_weighted_gbs": round(gb / (gt * 1e3), 1),
            "gemv_time_weighted_frac": round(gb / (gt * 1e3) / PEAK_HBM_GBS, 4),
            "note": "spans from the in-kernel trace of one traced step (mean of layers 2..L-2); "
                    "the GEMV fraction weights each GEMV phase by its time"}


def copy_calibration():
    """A plain device-to-device copy of COPY_BYTES, four times."""
    import torch
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "copies": 4}), flush=True)


def measured_traffic(kernel, workload):
    """Bytes per launch from profiles/decode_step_traffic.json, if it was
    measured on this kernel and workload."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel or t.get("workload") != workload:
        return None
    return t.get("traffic_bytes_per_launch")


# ----------------------------------------------------------- CPU baseline
def cpu_info():
    """The host CPU's model string and the cores this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return model, usable


def _ref_or_port(cfg, tensors_fn, use_ref):
    """The reference QwenModel (oracle/_ref) on weights tensors_fn() writes
    to a safetensors file (fp16: values do not change CPU time), or the C
    restatement with the same fill when _ref is absent."""
    from oracle import oracle as O
    if use_ref:
        path = os.path.join(tempfile.gettempdir(), f"lyk_cpu_baseline_{os.getpid()}.safetensors")
        O.write_safetensors(path, tensors_fn(), dtype="F16")
        m = O.RefModel(cfg, path)
        os.remove(path)
        return m
    m = O.OracleModel(cfg, threads=1)
    t = tensors_fn()
    for kind, layer, arr in m.tensors():
        arr[...] = t[O.tensor_name(kind, layer)]
    return m


def cpu_baseline(context, tokens=3):
    """Reference QwenModel (oracle/_ref) on the 7B architecture, single
    thread, per decode token at `context`:
      * the per-token time at a short context, from 1- and 2-layer models
        extrapolated to 28 layers as t(1) + 27 * (t(2) - t(1)) (the head is
        tied to the embedding: the same [152064, 3584] matvec as the untied
        7B head);
      * plus 28 x the attention time that `context` cached tokens add to one
        layer, measured on a 1-layer model with the 7B attention geometry (28
        q / 4 kv heads of 128) and a narrow residual (hidden 64, MLP 16,
        vocab 256), prefilled to `context` tokens: decode at `context`
        minus decode at a short context.
    Weights are random fp16; the prompt tokens are random."""
    from oracle import oracle as O
    from engine_amd.model import QWEN25_7B
    import dataclasses

    use_ref = O.ref_available()
    rng = np.random.default_rng(2)
    block = (rng.standard_normal(1 << 24).astype(np.float32) * 0.02)

    def weights(cfg):
        def fn():
            out = {}
            names = [("model.embed_tokens.weight", cfg.shape(O.T_EMBED)),
                     ("model.norm.weight", cfg.shape(O.T_FINAL_NORM))]
            for l in range(cfg.num_layers):
                for kind, suffix in O.LAYER_NAMES.items():
                    names.append((f"model.layers.{l}.{suffix}", cfg.shape(kind)))
            for name, shape in names:
                cnt = int(np.prod(shape))
                out[name] = np.ones(shape, np.float32) if "norm" in name else \
                    np.tile(block, -(-cnt // block.size))[:cnt].reshape(shape)
            return out
        return fn

    def per_token(m, max_tokens, prompt):
        s = m.new_seq(max_tokens)
        code, _ = m.prefill(s, prompt)
        assert code == 0
        t0 = time.perf_counter()
        for i in range(tokens):
            code, _ = m.decode(s, 2 + i)
            assert code == 0
        return (time.perf_counter() - t0) / tokens

    base = O.QwenConfig(**{**dataclasses.asdict(QWEN25_7B), "max_context_tokens": 64, "tie_word_embeddings": True})
    times = {}
    for layers in (1, 2):
        cfg = dataclasses.replace(base, num_layers=layers)
        m = _ref_or_port(cfg, weights(cfg), use_ref)
        times[layers] = per_token(m, 16, [1])
        del m
    t_short = times[1] + 27 * (times[2] - times[1])
    narrow = dataclasses.replace(base, num_layers=1, hidden_size=64, intermediate_size=16, vocab_size=256,
                                 eos_token_id=255, max_context_tokens=context + tokens + 8)
    m = _ref_or_port(narrow, weights(narrow), use_ref)
    a_short = per_token(m, 16, [1])
    a_long = per_token(m, context + tokens + 8, [int(t) for t in rng.integers(0, 256, context)])
    del m
    t_token = t_short + QWEN25_7B.num_layers * max(a_long - a_short, 0.0)
    model, usable = cpu_info()
    return dict(value=round(1.0 / t_token, 4), unit="tok/s", cores=1,
                kind="reference" if use_ref else "port", cpu=model, nproc=usable, context=context,
                sample=(f"Qwen2.5-7B-architecture decode on the {'reference QwenModel (oracle/_ref)' if use_ref else 'C restatement (oracle)'}, "
                        f"single thread, {tokens} tokens each: 1- and 2-layer models at context 2 "
                        f"({times[1]:.2f}s, {times[2]:.2f}s per token; 28 layers extrapolated: {t_short:.2f}s), "
                        f"plus 28 x the attention cost of {context} cached tokens per layer "
                        f"({(a_long - a_short) * 1e3:.1f} ms, narrow 1-layer model with the 7B heads): "
                        f"{t_token:.2f}s per token at context {context}"))


def batch_bench(args):
    """DecodeBatch throughput of R rows (config 4 / config 5 decode legs)."""
    import torch
    from engine_amd import model as M
    cfg = M.QWEN25_7B if args.model == "7b" else M.QWEN25_14B
    prompts = [int(p) for p in args.prompts.split(",")] if args.prompts else [args.prompt] * args.rows
    assert len(prompts) == args.rows and 1 <= args.rows <= 4
    pool = sum(prompts) + args.rows * (args.warmup + args.steps + 64)
    t0 = time.time()
    hip = M.HipModel.synthetic(cfg, seed=0, sigma=0.02, options=M.Options(quant=args.quant, kv_pool_tokens=pool))
    log(f"[batch] load (synthetic {args.model}, {args.quant}) {time.time() - t0:.1f}s")
    rng = np.random.default_rng(1)
    seqs, toks, ttft = [], [], []
    warm = hip.new_seq(64)
    assert hip.prefill(warm, list(range(1, 41)))[0] == 0
    warm.close()
    for n in prompts:
        s = hip.new_seq(n + args.warmup + args.steps + 8)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        code, logits = hip.prefill(s, rng.integers(0, cfg.vocab_size, n).astype(np.uint32))
        torch.cuda.synchronize()
        ttft.append(round((time.perf_counter() - t1) * 1e3, 1))
        assert code == 0
        seqs.append(s)
        toks.append(int(np.argmax(logits)))

    def steps(k):
        nonlocal toks
        for _ in range(k):
            code, per, out = hip.decode_batch(seqs, toks)
            assert code == 0 and per == [0] * len(seqs)
            toks = [int(v) for v in np.argmax(out, axis=1)]

    steps(args.warmup)
    stream = torch.cuda.ExternalStream(hip.stream_ptr)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    e0.record(stream)
    steps(args.steps)
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t1
    stream_us = e0.elapsed_time(e1) * 1e3 / args.steps
    hip.close()
    line = {"metric": f"DecodeBatch tok/s, {args.rows} sequences, Qwen2.5-{args.model.upper()} {args.quant.upper()} on 1 MI355X",
            "value": round(args.rows * args.steps / dt, 2), "unit": "tok/s", "rows": args.rows,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3 / args.steps, 4),
            "stream_us_per_step": round(stream_us, 1), "prompts": prompts, "ttft_ms": ttft,
            "note": "each step: one fused-step launch for all rows, logits copied to the host, greedy on the host"}
    print(json.dumps(line), flush=True)


def gemv_bench(quant):
    """Isolated GEMV (gemv.hip, lyk_hip_gemv_q4/q8) at BASELINE config 2's
    Qwen2.5-7B shapes, M = 1, 2, 4, fp16 N(0, 1) activations, weights N(0,
    0.02) quantized; each call reads the next of R weight copies totalling
    >= 512 MB (2x the MALL), so the rate is HBM's. >= 100 timed calls per
    case with HIP events; GB/s = packed weight + scale bytes per call / its
    average time."""
    import torch
    from engine_amd import ops
    shapes = {"gate_up": (18944, 3584), "down": (3584, 18944), "qkv": (4608, 3584), "lm_head": (152064, 3584)}
    rng = np.random.default_rng(0)
    cases = []
    for name, (n, k) in shapes.items():
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        base = ops.PackedWeight.from_float(quant, w)
        del w
        reps = max(2, -(-(512 << 20) // base.nbytes))
        copies = [base] + [ops.PackedWeight(quant, n, k, base.qw.cpu().numpy(), base.qs.cpu().numpy())
                           for _ in range(reps - 1)]
        for m in (1, 2, 4):
            x = torch.randn(m, ops.padded_k(k, quant), dtype=torch.float16, device="cuda")
            y = torch.empty(m, n, dtype=torch.float32, device="cuda")
            for c in copies[:2]:
                ops.gemv(c, x, y=y)
            iters = max(100, 2 * reps)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(iters):
                ops.gemv(copies[i % reps], x, y=y)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / iters
            gbs = base.nbytes / (us * 1e3)
            cases.append({"shape": name, "n": n, "k": k, "m": m, "us": round(us, 2), "bytes": base.nbytes,
                          "gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4), "copies": reps})
            log(f"[gemv] {name} n={n} k={k} M={m}: {us:.1f} us, {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS * 100:.1f}%)")
        del copies, base
        torch.cuda.empty_cache()
    print(json.dumps({"metric": f"isolated {quant.upper()} GEMV HBM GB/s (BASELINE config 2, Qwen2.5-7B shapes)",
                      "unit": "GB/s", "peak": PEAK_HBM_GBS, "kernel": "gemv.hip (lyk_hip_gemv_q4/q8)",
                      "rotation_bytes_min": 512 << 20, "cases": cases}), flush=True)


def prefill_gemm(quant):
    """Times the prefill GEMM (lyk_hip_gemm_q) on the 7B gate projection of a
    2048-token chunk, Y[2048, 18944] = X[2048, 3584] . W^T, and prints one JSON
    line (not the decode bench line): MFMA TFLOP/s against the fp16 dense peak."""
    import numpy as np
    import torch
    from engine_amd import ops
    T, n, k, tr = 2048, 18944, 3584, 32
    w = (np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32)
    codes, scales = ops.quantize(w, quant)
    qw, qs = ops.pack_tiled(codes, scales, quant, tr)
    qw, qs = torch.from_numpy(qw).cuda(), torch.from_numpy(qs).cuda()
    x = torch.randn(T, k, dtype=torch.float16, device="cuda")
    for _ in range(3):
        ops.gemm_q(x, qw, qs, n, quant, tr)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    e0.record()
    for _ in range(reps):
        ops.gemm_q(x, qw, qs, n, quant, tr)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    tflops = 2.0 * T * n * k / (us * 1e-6) / 1e12
    print(json.dumps({"metric": "prefill GEMM TFLOP/s (7B gate projection, 2048-token chunk)", "value": round(tflops, 1),
                      "unit": "TFLOP/s", "us_per_call": round(us, 1), "quant": quant,
                      "shape": {"T": T, "n": n, "k": k, "tile_rows": tr},
                      "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
                                   "frac": round(tflops / 2500.0, 4)}}), flush=True)


def sample_bench():
    """Times device sampling (lyk_hip_sample) of one 152064-logit row, with
    and without top_k, and the oracle's C restatement of the host Sampler on
    the same logits (one core) beside it; prints one JSON line."""
    import numpy as np
    import torch
    from engine_amd import lib as L, ops
    n = 152064
    logits = (np.random.default_rng(0).standard_normal(n) * 2.5).astype(np.float32)
    x = torch.from_numpy(logits).reshape(1, -1).cuda()
    ws = torch.empty(L.kernels().lyk_hip_sample_workspace_bytes(1, n), dtype=torch.uint8, device="cuda")
    out = {}
    for name, (t, k, p) in {"top_k40_p0.95_T1": (1.0, 40, 0.95), "p0.9_T0.7": (0.7, 0, 0.9)}.items():
        for _ in range(3):
            ops.sample(x, t, k, p, [0.5], ws)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            ops.sample(x, t, k, p, [0.5], ws)
        e1.record()
        torch.cuda.synchronize()
        gpu_us = e0.elapsed_time(e1) * 1e3 / 10
        from oracle import oracle as O   # the CPU baseline leg
        sm = O.Sampler(t, p, k, 1)
        t0 = time.time()
        for _ in range(3):
            sm.sample(logits)
        cpu_us = (time.time() - t0) / 3 * 1e6
        out[name] = {"gpu_us": round(gpu_us, 1), "cpu_baseline_us": round(cpu_us, 1)}
    print(json.dumps({"metric": "device sampling latency, V=152064 (model-like logits, N(0, 2.5))", "unit": "us",
                      "cases": out, "cpu_baseline": {"kind": "port", "cores": 1,
                                                     "sample": "oracle C restatement of Sampler::Sample"}}),
          flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--quant", choices=["int4", "int8"], default="int4")
    ap.add_argument("--prefill-chunk", type=int, default=0, help="prompt rows per prefill chunk pass (0: default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--prefill-gemm", action="store_true", help="time the prefill GEMM instead (one JSON line)")
    ap.add_argument("--sample", action="store_true", help="time device sampling instead (one JSON line)")
    ap.add_argument("--gemv", action="store_true", help="time the isolated GEMV at config 2 instead (one JSON line)")
    ap.add_argument("--rows", type=int, default=1, help="DecodeBatch rows (>1: the batch leg instead, one JSON line)")
    ap.add_argument("--model", choices=["7b", "14b"], default="7b", help="architecture of the --rows leg")
    ap.add_argument("--prompts", default="", help="comma-separated prompt lengths of the --rows leg")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (single-GPU tier); "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    if args.copy_calibration:
        copy_calibration()
        return
    if args.prefill_gemm:
        prefill_gemm(args.quant)
        return
    if args.sample:
        sample_bench()
        return
    if args.gemv:
        gemv_bench(args.quant)
        return
    if args.rows > 1:
        batch_bench(args)
        return
    dec = run_decode(args)
    achieved = dec["step_bytes"] / (dec["kernel_us"] * 1e-6) / 1e9
    log(f"[bench] decode {dec['tok_s']:.1f} tok/s ({dec['ms']:.3f} ms/token wall, {dec['kernel_us']:.1f} us/step "
        f"on the stream, context {dec['ctx_end']}); {achieved:.0f} GB/s = {achieved / PEAK_HBM_GBS * 100:.1f}% of HBM peak")
    kernel = f"decode_step_kernel<1, {args.quant}, 128> (fused decode step)"
    workload = f"qwen2.5-7b {args.quant} bs1 prompt {args.prompt} greedy"
    roof = dict(bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                frac=round(achieved / PEAK_HBM_GBS, 4), traffic=measured_traffic(kernel, workload))
    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(int(round(dec["ctx_mean"])))
        log(f"[bench] cpu baseline {cpu['value']} tok/s ({time.time() - t0:.1f}s)")
    line = {
        "metric": "decode tok/s Qwen2.5-7B INT4 bs=1 on 1 MI355X; GEMV HBM GB/s vs peak",
        "value": round(dec["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xfp16" if args.quant == "int4" else "int8xfp16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-7B-architecture decode, INT4 weight-only (groups of 32, fp16 scales), "
                        "fp16 activations and KV, batch 1, greedy (GreedyRun)",
            "prompt_tokens": args.prompt,
            "decode_tokens": args.steps,
            "context_at_end": dec["ctx_end"],
            "quant": args.quant,
        },
        "prefill": {"tokens": args.prompt, "ttft_ms": round(dec["ttft_ms"], 1),
                    "tok_s": round(args.prompt / dec["ttft_ms"] * 1e3, 1),
                    "path": "chunk passes of up to 2048 rows (MFMA GEMMs, causal chunk attention), last token through "
                            "the fused step"},
        "phases": dec["phases"],
        "roofline": roof,
        "roofline_kernel": {"kernel": kernel, "workload": workload,
                            "avg_us": round(dec["kernel_us"], 2),
                            "bytes_per_launch": int(dec["step_bytes"])},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
