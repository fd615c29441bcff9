"""Decode throughput of the hip backend: Qwen2.5-7B-architecture INT4
weight-only decode at batch 1 on one MI355X (BASELINE.json metric, config 4).

  python bench.py [--steps K] [--warmup W] [--prompt P] [--quant int4|int8]

A step is one decode token of one sequence: one launch of the fused decode
step kernel (every layer, the LM head and the on-device greedy argmax),
chained by GreedyRun. Weights are random-init N(0, 0.02) (synthetic, no
checkpoint) quantized at load; the prompt is P uniform random token ids.
One JSON line is printed:
  value        decode tokens/s (whole job; one GPU)
  roofline     the dominant (only) kernel of a step, decode_step_kernel:
               algorithmic HBM bytes of one launch (packed GEMV weights and
               scales + K/V of the context, fp16) / its average duration,
               from HIP events on the model's stream around the timed steps
  cpu_baseline the reference engine's own CPU QwenModel (oracle/_ref), single
               thread as the reference runs it, on a bounded sample (see
               cpu_baseline.sample); the C restatement (oracle) if _ref is absent
  roofline.traffic  HBM bytes per launch measured by rocprofv3 (FETCH_SIZE +
               WRITE_SIZE, calibrated on a plain copy), read from
               profiles/decode_step_traffic.json when that file was measured on
               the same kernel and workload (bench_profile.py writes it); else null
Only N=1 is supported: this build targets one GPU.

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
    opts = M.Options(quant=args.quant, kv_pool_tokens=args.prompt + args.warmup + args.steps + 512)
    hip = M.HipModel.synthetic(cfg, seed=0, sigma=0.02, options=opts)
    log(f"[bench] load (synthetic 7B, {args.quant}) {time.time() - t0:.1f}s, "
        f"GEMV bytes/token {hip.gemv_weight_bytes / 1e9:.3f} GB")
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, cfg.vocab_size, args.prompt).astype(np.uint32)
    seq = hip.new_seq(args.prompt + args.warmup + args.steps + 8)
    t0 = time.time()
    code, logits = hip.prefill(seq, prompt)
    assert code == 0, f"prefill failed with code {code}"
    log(f"[bench] prefill {args.prompt} tokens {time.time() - t0:.1f}s")
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
    hip.close()
    return dict(tok_s=args.steps / dt, ms=dt * 1e3 / args.steps, ctx_end=ctx, kernel_us=kernel_us,
                step_bytes=step_bytes, gemv_bytes=gemv_bytes, tokens=toks)


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
def cpu_baseline(tokens=3):
    """Reference QwenModel (oracle/_ref) on the 7B architecture, single thread,
    with 1 and then 2 decoder layers; per-token time extrapolated to 28
    layers as t(1) + 27 * (t(2) - t(1)). Weights are random fp16 in a
    safetensors file (values do not change CPU time); the head is tied to the
    embedding, the same [152064, 3584] matvec as the untied 7B head."""
    from oracle import oracle as O
    from engine_amd.model import QWEN25_7B
    import dataclasses

    use_ref = O.ref_available()
    base = O.QwenConfig(**{**dataclasses.asdict(QWEN25_7B), "max_context_tokens": 64,
                           "tie_word_embeddings": True})
    rng = np.random.default_rng(2)
    block = (rng.standard_normal(1 << 24).astype(np.float32) * 0.02)
    times = {}
    for layers in (1, 2):
        cfg = dataclasses.replace(base, num_layers=layers)
        if use_ref:
            tensors = {}
            names = [("model.embed_tokens.weight", cfg.shape(O.T_EMBED)),
                     ("model.norm.weight", cfg.shape(O.T_FINAL_NORM))]
            for l in range(layers):
                for kind, suffix in O.LAYER_NAMES.items():
                    names.append((f"model.layers.{l}.{suffix}", cfg.shape(kind)))
            for name, shape in names:
                cnt = int(np.prod(shape))
                if "norm" in name:
                    tensors[name] = np.ones(shape, np.float32)
                else:
                    reps = -(-cnt // block.size)
                    tensors[name] = np.tile(block, reps)[:cnt].reshape(shape)
            path = os.path.join(tempfile.gettempdir(), f"lyk_cpu_baseline_{layers}.safetensors")
            O.write_safetensors(path, tensors, dtype="F16")
            del tensors
            m = O.RefModel(cfg, path)
            os.remove(path)
        else:
            m = O.OracleModel(cfg, threads=1)
            for kind, layer, arr in m.tensors():
                arr[...] = 1.0 if kind in (O.T_INPUT_NORM, O.T_POST_NORM, O.T_FINAL_NORM) else \
                    np.resize(block, arr.size).reshape(arr.shape)
        s = m.new_seq(16)
        code, logits = m.prefill(s, [1])
        t0 = time.perf_counter()
        for i in range(tokens):
            code, logits = m.decode(s, 2 + i)
        times[layers] = (time.perf_counter() - t0) / tokens
        del m, s
    per_layer = times[2] - times[1]
    t_token = times[1] + 27 * per_layer
    return dict(value=round(1.0 / t_token, 4), unit="tok/s", cores=1,
                kind="reference" if use_ref else "port",
                sample=(f"Qwen2.5-7B-architecture decode on the {'reference QwenModel (oracle/_ref)' if use_ref else 'C restatement (oracle)'}, "
                        f"single thread, {tokens} tokens each with 1 and 2 layers "
                        f"({times[1]:.2f}s, {times[2]:.2f}s per token); 28 layers extrapolated: "
                        f"{t_token:.2f}s per token"))


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
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--prefill-gemm", action="store_true", help="time the prefill GEMM instead (one JSON line)")
    ap.add_argument("--sample", action="store_true", help="time device sampling instead (one JSON line)")
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
        cpu = cpu_baseline()
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
        "roofline": roof,
        "roofline_kernel": {"kernel": kernel, "workload": workload,
                            "avg_us": round(dec["kernel_us"], 2),
                            "bytes_per_launch": int(dec["step_bytes"])},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
