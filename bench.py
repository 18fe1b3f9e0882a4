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


def make_workload(device, seed=SEED):
    g = torch.Generator(device="cpu").manual_seed(seed)
    xs = [(torch.randn(B, H, L, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(device)
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


def cpu_baseline(budget_s=20.0):
    """fp32 eager restatement (oracle/torch_ref.py) on host cores, one batch
    element at a time, until ~budget_s of CPU work; reported as TFLOP/s."""
    from oracle import torch_ref
    threads = min(os.cpu_count() or 1, 16)
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
            "sample": f"fp32 eager restatement (oracle/torch_ref.py), {len(times)} of {B} batch "
                      f"elements of the 150M shape timed one at a time, median "
                      f"{med * 1e3:.1f} ms/element (full batch ~{med * B:.2f} s)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", choices=("fwd", "fwdbwd"), default="fwd",
                    help="fwd: the headline forward (B=16); fwdbwd: forward + backward at the "
                         "training shape (B=8, dO ~ N(0, 1))")
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
        "metric": "multi-pathway attn fwd TFLOP/s (150M shape, bf16)",
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


if __name__ == "__main__":
    main()
