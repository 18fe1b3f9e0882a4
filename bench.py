"""Benchmark of the multi-pathway attention forward on one MI355X.

Workload (the headline metric): isolated forward at
the ESM-2 150M shape, bf16, B=16, H=20, D=32, L=1024. Each sample has two
chains split at s ~ U[256, 768] and a padding tail of 0-10 % of L; Q/K/V of
both pathways ~ N(0, 1)/sqrt(32); RoPE (global positions) on the self pathway
and the D^-1/2 scale are applied inside the op. A "step" is one forward call
over the whole batch with inputs resident in HBM.

Algorithmic work per call: 4*B*H*L^2*D flops (one D-dot per selected logit
plus one D-FMA row update), 42.95 GFLOP at this shape; bytes: 7 tensors of
B*H*L*D bf16 + B*L*5 (chain id + pad flag), 146.9 MB.

Prints one JSON line (see the repository's measurement notes):
metric/value/unit, ms_per_step, roofline (MFMA-bound kernel) and a CPU
baseline (the fp32 eager restatement timed on this host on a bounded sample).
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
B, H, L, D = 16, 20, 1024, 32
SEED = 150


def make_workload(device, seed=SEED, d=D, dtype=torch.bfloat16):
    """The headline batch; ``d`` / ``dtype`` give the same
    batch at another head dim or element type (per-head-dim modes)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    xs = [(torch.randn(B, H, L, d, generator=g) / d ** 0.5).to(dtype).to(device)
          for _ in range(6)]
    cid = torch.zeros(B, L, dtype=torch.int32)
    pad = torch.zeros(B, L, dtype=torch.bool)
    for b in range(B):
        s = int(torch.randint(256, 769, (1,), generator=g))
        cid[b, s:] = 1
        n = int(torch.randint(0, L // 10 + 1, (1,), generator=g))
        if n:
            pad[b, L - n:] = True
    return xs, cid.to(device), pad.to(device)


def flops_fwd(b=B):
    return 4.0 * b * H * L * L * D


def flops_bwd(b=B):
    """dV, dP, dQ, dK: four L x L x D contractions per (b, h); recompute excluded."""
    return 8.0 * b * H * L * L * D


def bytes_fwd(b=B):
    return 7.0 * b * H * L * D * 2 + b * L * 5


def bytes_bwd(b=B):
    """6 inputs + O + dO read, 6 gradients written (bf16), LSE read, chain ids."""
    return 14.0 * b * H * L * D * 2 + b * H * L * 4 + b * L * 5


def host_cores():
    """(threads, CPU model): every core this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS when the host sets it (the
    GPU box's CPU share), and the model name from /proc/cpuinfo."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return n, model


def cpu_baseline(budget_s=20.0):
    """fp32 eager restatement (oracle/torch_ref.py) on host cores, one batch
    element at a time, until ~budget_s of CPU work; reported as TFLOP/s."""
    from oracle import torch_ref
    threads, cpu = host_cores()
    torch.set_num_threads(threads)
    torch.set_float32_matmul_precision("highest")
    xs, cid, pad = make_workload("cpu")
    xs = [x.float() for x in xs]
    per_elem = flops_fwd() / B
    # warm-up on one element
    torch_ref.forward(*[x[:1] for x in xs], chain_ids=cid[:1], key_pad=pad[:1], rope=True,
                      scale=D ** -0.5, dtype=torch.float32)
    times = []
    t_start = time.perf_counter()
    b = 0
    while (time.perf_counter() - t_start) < budget_s and len(times) < B:
        t0 = time.perf_counter()
        torch_ref.forward(*[x[b:b + 1] for x in xs], chain_ids=cid[b:b + 1],
                          key_pad=pad[b:b + 1], rope=True, scale=D ** -0.5, dtype=torch.float32)
        times.append(time.perf_counter() - t0)
        b += 1
    med = statistics.median(times)
    return {"value": per_elem / med / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cpu,
            "sample": f"fp32 eager restatement (oracle/torch_ref.py), {len(times)} of {B} batch "
                      f"elements of the 150M shape timed one at a time, median "
                      f"{med * 1e3:.1f} ms/element (full batch ~{med * B:.2f} s), "
                      f"{threads} threads on {cpu}"}


def model_batch(device, seed, B, lo, hi, min_chain):
    """B two-chain complexes of total length ~ U[lo, hi] (each chain >=
    min_chain tokens) over the 20 standard amino acids (token ids 4..23),
    laid out [A][B][pad] and padded (id 1) to the batch max."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    lens = [int(torch.randint(lo, hi + 1, (1,), generator=g)) for _ in range(B)]
    Lm = max(lens)
    tok = torch.ones(B, Lm, dtype=torch.long)
    cid = torch.ones(B, Lm, dtype=torch.long)
    for b, n in enumerate(lens):
        tok[b, :n] = torch.randint(4, 24, (n,), generator=g)
        s = int(torch.randint(min_chain, n - min_chain + 1, (1,), generator=g))
        cid[b, :s] = 0
    return tok.to(device), cid.to(device)


def bench_model(dev, size="650M", dtype=torch.bfloat16, B=8, steps=5, warmup=2,
                paths=("fused", "combine", "eager", "eager_reference")):
    """Full MINT forward (embedding extraction) with random-init weights:
    seconds per forward and sequences/s for each multimer-attention path:
    fused HIP kernel, materialised logits + HIP combine kernel, eager torch
    with an fp32 softmax ("eager") and eager torch with the reference's bf16
    softmax arithmetic ("eager_reference", modules_plus.py:182-194)."""
    from mint_plus_amd import esm2, modules
    torch.manual_seed(65)
    with torch.device(dev):
        model = esm2.MINT.from_config(size)
    model = model.to(dtype).eval()
    tok, cid = model_batch(dev, 650, B, 512, 1024, 64)
    stream = torch.cuda.current_stream(dev)
    out = {"model": size, "B": B, "L_max": int(tok.shape[1]),
           "tokens": int((tok != 1).sum()), "dtype": str(dtype).replace("torch.", "")}
    for path in paths:
        modules.enable_fused_multi_pathway(model, path == "fused")
        modules.use_eager_multimer(model, "reference" if path == "eager_reference" else path == "eager")

        def step():
            with torch.inference_mode():
                model(tok, chain_ids=cid, repr_layers=[model.num_layers])

        _, per = timed(step, steps, warmup, stream)
        ms = statistics.median(per)
        out[f"ms_fwd_{path}"] = round(ms, 3)
        out[f"seqs_per_sec_{path}"] = round(B / (ms * 1e-3), 2)
    for e in ("eager", "eager_reference"):
        if "fused" in paths and e in paths:
            out[f"speedup_fused_vs_{e}"] = round(out[f"ms_fwd_{e}"] / out["ms_fwd_fused"], 3)
    del model
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", choices=("fwd", "fwdbwd", "model", "attn3b", "attn650m", "combine", "dense",
                                       "headdim", "attn8m"),
                    default="fwd",
                    help="fwd: the headline forward (B=16); fwdbwd: forward + backward at the "
                         "training shape (B=8, dO ~ N(0, 1)); model: 650M MINT forward "
                         "sequences/s per attention path; attn3b / attn650m: the op at the 3B / "
                         "650M model's attention shape; dense: the 150M forward through the "
                         "reference's (B, L, L) chain-mask contract; "
                         "combine: the materialised-logit combine fwd and bwd (HBM-bound); "
                         "headdim: the headline batch at D = 16, 24, 32, 64 (one line each, "
                         "forward and forward+backward; --dtype); attn8m: fp32 forward and "
                         "forward+backward at the 8M model's attention shape (configs[0])")
    ap.add_argument("--dtype", choices=("bf16", "fp32"), default="bf16",
                    help="element type of --mode headdim")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the 650M model forward summary of the default line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="time a plain device copy of MIB MiB instead (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(each (b, h) of the op is independent; see the sharding notes).", file=sys.stderr)
        sys.exit(2)

    import mint_plus_amd
    from mint_plus_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(args.warmup):
            dst.copy_(src)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        print(json.dumps({"copy_bytes": n, "ms": ms, "GB/s": 2 * n / ms / 1e6}), flush=True)
        return
    if args.mode == "fwdbwd":
        return bench_fwdbwd(args, dev)
    if args.mode == "model":
        print(json.dumps(bench_model(dev, steps=max(3, min(args.steps, 10)),
                                     warmup=min(args.warmup, 3))), flush=True)
        return
    if args.mode in ("attn3b", "attn650m"):
        return bench_attn_shape(args, dev, args.mode[4:])
    if args.mode == "combine":
        return bench_combine(args, dev)
    if args.mode == "dense":
        return bench_dense(args, dev)
    if args.mode == "headdim":
        return bench_headdim(args, dev)
    if args.mode == "attn8m":
        return bench_attn8m(args, dev)
    xs, cid, pad = make_workload(dev)
    out = torch.empty_like(xs[0])

    def step():
        _lib.mpattn_fwd(*xs, chain_ids=cid, key_padding_mask=pad, rope=True, scale=D ** -0.5,
                        out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    # per-launch events on the launch stream
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))  # ms
    med = statistics.median(per)
    p10, p90 = per[len(per) // 10], per[(9 * len(per)) // 10]
    mean_ms = sum(per) / len(per)
    ms_per_step = wall * 1e3 / args.steps
    tflops = flops_fwd() / (med * 1e-3) / 1e12
    achieved = flops_fwd() / (mean_ms * 1e-3) / 1e12

    res = {
        "metric": "multi-pathway attn TFLOP/s & % bf16 MFMA peak (150M shape); seqs/sec 650M fwd",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(32) projections, 2 chains, 0-10% pad tail)",
        "config": {"workload": "150M isolated multi-pathway attention forward",
                   "B": B, "H": H, "L": L, "D": D, "rope": "fused", "chains": 2},
        "kernel_ms": {"median": round(med, 5), "p10": round(p10, 5), "p90": round(p90, 5),
                      "mean": round(mean_ms, 5)},
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "hbm_gbs_algorithmic": round(bytes_fwd() / (med * 1e-3) / 1e9, 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("fwd_150m")},
        "cpu_baseline": None,
    }
    if not args.no_model:
        # 650M full-model forward, sequences/s: fused HIP path vs eager attention
        res["model_650m_fwd"] = bench_model(dev, paths=("fused", "eager", "eager_reference"))
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


def measured_traffic(key):
    """HBM bytes per call from the committed rocprofv3 --pmc summary
    (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE per dispatch, scaled by
    the factors a plain copy of known size gives), or None if absent."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)[key]
    except (OSError, KeyError, ValueError):
        return None
    return int(rec["bytes_per_call"])


def timed(step, steps, warmup, stream):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    return wall, per


def bench_fwdbwd(args, dev):
    """Forward (saving LSE) + backward at configs[3]: B=8, dO ~ N(0, 1)."""
    from mint_plus_amd import _lib
    b8 = 8
    xs, cid, pad = make_workload(dev)
    xs = [x[:b8].contiguous() for x in xs]
    cid, pad = cid[:b8].contiguous(), pad[:b8].contiguous()
    g = torch.Generator(device="cpu").manual_seed(SEED + 1)
    go = torch.randn(b8, H, L, D, generator=g).to(torch.bfloat16).to(dev)
    sel = dict(chain_ids=cid, key_padding_mask=pad, rope=True, scale=D ** -0.5)
    out = torch.empty_like(xs[0])

    def step():
        _, lse = _lib.mpattn_fwd(*xs, need_lse=True, out=out, **sel)
        _lib.mpattn_bwd(*xs, out, lse, go, **sel)

    stream = torch.cuda.current_stream(dev)
    wall, per = timed(step, args.steps, args.warmup, stream)
    med = statistics.median(per)
    mean_ms = sum(per) / len(per)
    fl = flops_fwd(b8) + flops_bwd(b8)
    tflops = fl / (med * 1e-3) / 1e12
    achieved = fl / (mean_ms * 1e-3) / 1e12
    res = {
        "metric": "multi-pathway attn fwd+bwd TFLOP/s (150M training shape, bf16)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(32) projections, 2 chains, 0-10% pad tail, "
                "dO ~ N(0,1))",
        "config": {"workload": "multi-pathway attention forward+backward, frozen-150M "
                               "training shape", "B": b8, "H": H, "L": L, "D": D,
                   "rope": "fused", "chains": 2},
        "kernel_ms": {"median": round(med, 5), "p10": round(per[len(per) // 10], 5),
                      "p90": round(per[(9 * len(per)) // 10], 5), "mean": round(mean_ms, 5)},
        "flops_per_step": fl,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("fwdbwd_150m_b8")},
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)


def attn_shape_inputs(dev, shape):
    """Inputs of the op at a model's attention shape (bf16, N(0, 1/D)).

    3b: B=4, H=40, D=64, three chains of ~U[200, 800] tokens with
    L_total <= 2048, padded to 2048.
    650m: B=8, H=20, D=64, the 650M model's batch (two chains, L_total
    ~U[512, 1024], each chain >= 64, padded to the batch max; configs[2])."""
    g = torch.Generator(device="cpu").manual_seed(3000)
    if shape == "3b":
        b, h, l, d = 4, 40, 2048, 64
        cid = torch.full((b, l), 2, dtype=torch.int32)
        pad = torch.zeros(b, l, dtype=torch.bool)
        for i in range(b):
            while True:
                n = [int(torch.randint(200, 801, (1,), generator=g)) for _ in range(3)]
                if sum(n) <= l:
                    break
            cid[i, :n[0]] = 0
            cid[i, n[0]:n[0] + n[1]] = 1
            pad[i, sum(n):] = True
        data = "synthetic (3 chains ~U[200,800], padded to 2048)"
    else:
        b, h, d = 8, 20, 64
        tok, cid = model_batch("cpu", 650, b, 512, 1024, 64)
        l = int(tok.shape[1])
        cid = cid.to(torch.int32)
        pad = tok == 1
        data = f"synthetic (2 chains, L_total ~U[512,1024], padded to {l})"
    xs = [(torch.randn(b, h, l, d, generator=g) / d ** 0.5).to(torch.bfloat16).to(dev)
          for _ in range(6)]
    return xs, cid.to(dev), pad.to(dev), (b, h, l, d), data


def bench_attn_shape(args, dev, shape):
    """The op (forward, fused RoPE) at the 3B or 650M model's attention
    shape: TFLOP/s on the algorithmic 4*B*H*L^2*D."""
    from mint_plus_amd import _lib
    xs, cid, pad, (b, h, l, d), data = attn_shape_inputs(dev, shape)
    out = torch.empty_like(xs[0])

    def step():
        _lib.mpattn_fwd(*xs, chain_ids=cid, key_padding_mask=pad, rope=True, scale=d ** -0.5,
                        out=out)

    stream = torch.cuda.current_stream(dev)
    wall, per = timed(step, args.steps, args.warmup, stream)
    med = statistics.median(per)
    fl = 4.0 * b * h * l * l * d
    name = {"3b": "3B", "650m": "650M"}[shape]
    print(json.dumps({
        "metric": f"multi-pathway attn fwd TFLOP/s ({name} shape, bf16)",
        "value": round(fl / (med * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5), "higher_is_better": True,
        "dtype": "bf16", "data": data,
        "config": {"workload": f"{name}-shape multi-pathway attention forward (one layer)",
                   "B": b, "H": h, "L": l, "D": d, "rope": "fused",
                   "chains": 3 if shape == "3b" else 2},
        "kernel_ms": {"median": round(med, 5), "p10": round(per[len(per) // 10], 5),
                      "p90": round(per[(9 * len(per)) // 10], 5)},
        "pct_bf16_peak": round(100.0 * fl / (med * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
    }), flush=True)


PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA


def _fwd_fwdbwd_lines(args, dev, xs, cid, pad, d, dtype_name, peak, metric, config, data):
    """Time the forward and the forward+backward of the op on these inputs
    (fused RoPE, scale d^-1/2, dO ~ N(0, 1)); print one JSON line."""
    from mint_plus_amd import _lib
    b, h, l = xs[0].shape[:3]
    sel = dict(chain_ids=cid, key_padding_mask=pad, rope=True, scale=d ** -0.5)
    out = torch.empty_like(xs[0])
    g = torch.Generator(device="cpu").manual_seed(SEED + 2)
    go = torch.randn(xs[0].shape, generator=g).to(xs[0].dtype).to(dev)
    stream = torch.cuda.current_stream(dev)

    def fwd():
        _lib.mpattn_fwd(*xs, out=out, **sel)

    def fwdbwd():
        _, lse = _lib.mpattn_fwd(*xs, need_lse=True, out=out, **sel)
        _lib.mpattn_bwd(*xs, out, lse, go, **sel)

    ffl = 4.0 * b * h * l * l * d
    res = {"metric": metric, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "higher_is_better": True, "dtype": dtype_name, "data": data,
           "config": dict(config, B=b, H=h, L=l, D=d, rope="fused")}
    for name, fn, fl in (("fwd", fwd, ffl), ("fwdbwd", fwdbwd, 3.0 * ffl)):
        wall, per = timed(fn, args.steps, args.warmup, stream)
        med = statistics.median(per)
        mean_ms = sum(per) / len(per)
        res[f"{name}_ms"] = {"median": round(med, 5), "p10": round(per[len(per) // 10], 5),
                             "p90": round(per[(9 * len(per)) // 10], 5), "mean": round(mean_ms, 5)}
        res[f"{name}_tflops"] = round(fl / (med * 1e-3) / 1e12, 2)
        res[f"{name}_frac_peak"] = round(fl / (mean_ms * 1e-3) / 1e12 / peak, 4)
        if name == "fwd":
            res["ms_per_step"] = round(wall * 1e3 / args.steps, 5)
    res["value"] = res["fwd_tflops"]
    res["peak_tflops"] = peak
    print(json.dumps(res), flush=True)


def bench_headdim(args, dev):
    """The headline batch (B=16, H=20, L=1024, two chains, pad tail) at each
    head dim of the ESM-2 family (8M: 16, 35M: 24, 150M: 32, 650M/3B: 64),
    in bf16 or fp32. Algorithmic flops: forward 4*B*H*L^2*D, backward twice
    that (fwd+bwd 12*B*H*L^2*D; the backward's recompute is not counted)."""
    bf = args.dtype == "bf16"
    dt = torch.bfloat16 if bf else torch.float32
    peak = PEAK_BF16_TFLOPS if bf else PEAK_FP32_TFLOPS
    for d in (16, 24, 32, 64):
        xs, cid, pad = make_workload(dev, d=d, dtype=dt)
        _fwd_fwdbwd_lines(args, dev, xs, cid, pad, d, args.dtype, peak,
                          f"multi-pathway attn TFLOP/s (150M batch, D={d}, {args.dtype})",
                          {"workload": f"headline batch at head dim {d}", "chains": 2},
                          f"synthetic (seeded N(0,1)/sqrt({d}) projections, 2 chains, 0-10% pad tail)")
        del xs
        torch.cuda.empty_cache()


def bench_attn8m(args, dev):
    """The op in fp32 at the ESM-2 8M MINT model's attention shape
    (configs[0]): B=4, H=20, D=16, two chains of U[60,200] + U[40,160]
    residues plus <cls>/<eos> each, padded to the batch max."""
    g = torch.Generator(device="cpu").manual_seed(8)
    b, h, d = 4, 20, 16
    la = [int(torch.randint(60, 201, (1,), generator=g)) + 2 for _ in range(b)]
    lb = [int(torch.randint(40, 161, (1,), generator=g)) + 2 for _ in range(b)]
    l = max(x + y for x, y in zip(la, lb))
    cid = torch.zeros(b, l, dtype=torch.int32)
    pad = torch.zeros(b, l, dtype=torch.bool)
    for i in range(b):
        cid[i, la[i]:] = 1
        pad[i, la[i] + lb[i]:] = True
    xs = [(torch.randn(b, h, l, d, generator=g) / d ** 0.5).to(dev) for _ in range(6)]
    _fwd_fwdbwd_lines(args, dev, xs, cid.to(dev), pad.to(dev), d, "fp32", PEAK_FP32_TFLOPS,
                      "multi-pathway attn TFLOP/s (8M attention shape, fp32)",
                      {"workload": "8M MINT attention (configs[0]), one layer", "chains": 2},
                      "synthetic (seeded N(0,1)/4 projections, chains U[60,200]+2 and U[40,160]+2)")


def bench_dense(args, dev):
    """The 150M forward (the headline workload) with the chain information
    given as the reference kernel's (B, L, L) bool mask (True = different
    chains) instead of chain ids, fused RoPE; also forward + backward at the
    training shape (B=8) through the same mask."""
    from mint_plus_amd import _lib
    xs, cid, pad = make_workload(dev)
    cm = (cid[:, :, None] != cid[:, None, :]).contiguous()
    out = torch.empty_like(xs[0])

    def step():
        _lib.mpattn_fwd(*xs, chain_mask=cm, key_padding_mask=pad, rope=True, scale=D ** -0.5, out=out)

    wall, per = timed(step, args.steps, args.warmup, torch.cuda.current_stream(dev))
    med = statistics.median(per)
    fl = flops_fwd()
    # forward (saving LSE) + backward at the training shape (B=8) through the
    # same mask contract
    b8 = 8
    x8 = [x[:b8].contiguous() for x in xs]
    cm8, pad8 = cm[:b8].contiguous(), pad[:b8].contiguous()
    g = torch.Generator(device="cpu").manual_seed(SEED + 1)
    go = torch.randn(b8, H, L, D, generator=g).to(torch.bfloat16).to(dev)
    out8 = torch.empty_like(x8[0])
    sel = dict(chain_mask=cm8, key_padding_mask=pad8, rope=True, scale=D ** -0.5)

    def step_fb():
        _, lse = _lib.mpattn_fwd(*x8, need_lse=True, out=out8, **sel)
        _lib.mpattn_bwd(*x8, out8, lse, go, **sel)

    _, per_fb = timed(step_fb, max(10, args.steps // 2), args.warmup, torch.cuda.current_stream(dev))
    med_fb = statistics.median(per_fb)
    print(json.dumps({
        "fwdbwd_b8_ms": round(med_fb, 5),
        "fwdbwd_b8_tflops": round((flops_fwd(b8) + flops_bwd(b8)) / (med_fb * 1e-3) / 1e12, 2),
        "metric": "multi-pathway attn fwd TFLOP/s (150M shape, dense chain mask, bf16)",
        "value": round(fl / (med * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5), "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic (the headline workload, mask from its chain ids)",
        "config": {"workload": "150M isolated multi-pathway attention forward, (B, L, L) chain mask",
                   "B": B, "H": H, "L": L, "D": D, "rope": "fused", "chains": 2},
        "kernel_ms": {"median": round(med, 5), "p10": round(per[len(per) // 10], 5),
                      "p90": round(per[(9 * len(per)) // 10], 5)},
        "pct_bf16_peak": round(100.0 * fl / (med * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
    }), flush=True)


def bench_combine(args, dev, b=8):
    """fused_multimer_combine (fwd) and fused_multimer_combine_bwd at the
    150M shape with B=8: two (B, H, L, L) bf16 logit tensors, the (B, L, L)
    bool mask and two value tensors. Algorithmic bytes: fwd reads 2 logits +
    mask + 2 values and writes O; bwd reads the same plus dO and writes both
    d_logits and both d_values. ``bwd`` is the reference's signature (no
    forward statistics: a statistics pass reads both logit tensors first);
    ``bwd_fwdstats`` is the autograd path, given the forward's LSE and O
    (Delta = dO . O from them, no statistics pass); its bytes add O and LSE."""
    from mint_plus_amd import _lib
    g = torch.Generator(device=dev).manual_seed(77)
    il = (torch.randn(b, H, L, L, device=dev, generator=g) * 2).to(torch.bfloat16)
    el = (torch.randn(b, H, L, L, device=dev, generator=g) * 2).to(torch.bfloat16)
    vs = torch.randn(b, H, L, D, device=dev, generator=g).to(torch.bfloat16)
    vm = torch.randn(b, H, L, D, device=dev, generator=g).to(torch.bfloat16)
    go = torch.randn(b, H, L, D, device=dev, generator=g).to(torch.bfloat16)
    _, cid, _ = make_workload(dev)
    cid = cid[:b]
    cm = cid[:, :, None] != cid[:, None, :]
    stream = torch.cuda.current_stream(dev)
    lg = 2.0 * b * H * L * L * 2
    vb = b * H * L * D * 2
    fwd_bytes = lg + b * L * L + 3 * vb
    bwd_bytes = 2 * lg + b * L * L + 5 * vb  # each input read once, each gradient written once
    res = {"metric": "materialised combine HBM GB/s (150M shape, B=8, bf16)", "unit": "GB/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "bf16",
           "data": "synthetic logits N(0,4), 2 chains",
           "config": {"workload": "fused_multimer_combine fwd / bwd", "B": b, "H": H, "L": L,
                      "D": D}}
    out, lse = _lib.mpattn_combine_fwd(il, el, cm, vs, vm, need_lse=True)
    for name, fn, nbytes in (
            ("fwd", lambda: _lib.mpattn_combine_fwd(il, el, cm, vs, vm), fwd_bytes),
            ("bwd", lambda: _lib.mpattn_combine_bwd(il, el, cm, vs, vm, go), bwd_bytes),
            ("bwd_fwdstats", lambda: _lib.mpattn_combine_bwd(il, el, cm, vs, vm, go, lse=lse, out=out),
             bwd_bytes + vb + b * H * L * 4)):
        _, per = timed(fn, max(10, args.steps // 4), args.warmup, stream)
        med = statistics.median(per)
        res[f"{name}_ms"] = round(med, 4)
        res[f"{name}_GBs"] = round(nbytes / (med * 1e-3) / 1e9, 1)
        res[f"{name}_frac_hbm_peak"] = round(nbytes / (med * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
    res["value"] = res["fwd_GBs"]
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
