"""Benchmark: ModernBERT-base encoder forward on one MI355X.

One step = one dn_forward_device over one batch of the workload (default
cfg3: 64 requests x 512 tokens, 384-token premise + 8 options x 16, the
premise/option block mask, all 22 layers, scorer head), with weights and
token arrays already resident in HBM. Prints one JSON line (see the keys
below). Synthetic data: weights N(0, 0.02) with InitRandom semantics and
seeded token ids; see decide_amd/synth.py.

  python bench.py [--steps K] [--warmup W] [--config cfg3] [--precision bf16]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "encoder tokens/sec + GEMM TFLOP/s (% bf16 MFMA peak), ModernBERT-base, 1 MI355X"
PEAK = {"bf16": 2.5e15, "fp32": 157.3e12}  # dense MFMA peaks, FLOP/s
H, I = 768, 1152
PROJ_FLOP_PER_TOKEN_LAYER = 2 * H * (3 * H + H + 2 * I + I)  # 10,027,008
WORKLOADS = {
    "cfg2": "cfg2: 1 Choice request x 112 tokens (64-token premise + 3 options x 16)",
    "cfg3": "cfg3: batch 64 x seq 512 (384-token premise + 8 options x 16), block-masked, 22 layers",
    "cfg4": "cfg4: batch 8 x seq 2816 (2048-token premise + 24 question segments, 84 options)",
    "cfg5": "cfg5: batch 1 x seq 64 (40-token premise + 2 options x 12)",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(cfg, weights, name: str, budget_s: float = 12.0):
    """The oracle (C++ restatement of the reference's Go AVX2 forward) on a
    bounded sample of the same workload: whole sequences of the workload until
    about budget_s seconds of CPU work."""
    import oracle
    from decide_amd.synth import config_batch

    threads = cpu_threads()
    oracle.set_workers(threads)
    model = oracle.OracleModel(cfg, weights)
    full = config_batch(name, vocab=cfg.vocab)
    toks, secs, nseq = 0, 0.0, 0
    while secs < budget_s and nseq < len(full) * 4:
        s = full[nseq % len(full)]
        t0 = time.perf_counter()
        model.forward([s])
        secs += time.perf_counter() - t0
        toks += len(s.ids)
        nseq += 1
    return {"value": toks / secs, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{nseq} sequence(s) of {name} ({toks} tokens) one forward per sequence, "
                      f"{secs:.1f} s; C++ restatement of the reference Go AVX2 path (oracle/)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--precision", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--probe-layer", type=int, default=1)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run one device copy of MIB MiB first (reference kernel for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the forward shards by sequence with no collective; see DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    from decide_amd import Engine, modernbert_base
    from decide_amd.nn import flatten, row_tokens
    from decide_amd.synth import config_batch, random_weights

    cfg = modernbert_base()
    log("generating weights")
    weights = random_weights(cfg, seed=0)
    batch = config_batch(args.config, vocab=cfg.vocab)
    seq_len, ids, pos, opt, nmask, _ = flatten(batch)
    T, R = int(seq_len.sum()), int(nmask.sum())
    log(f"workload {args.config}: {len(batch)} sequences, T={T}, R={R}")

    torch.cuda.init()
    dev = torch.device("cuda:0")
    eng = Engine(cfg, weights, precision=args.precision)
    stream = torch.cuda.current_stream()
    eng.set_stream(stream.cuda_stream)
    d_ids = torch.from_numpy(ids).to(dev)
    d_pos = torch.from_numpy(pos).to(dev)
    d_opt = torch.from_numpy(opt).to(dev)
    d_rt = torch.from_numpy(row_tokens(batch)).to(dev)
    d_out = torch.zeros(R, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def step():
        eng.forward_device(seq_len, d_ids.data_ptr(), d_pos.data_ptr(), d_opt.data_ptr(), R, d_rt.data_ptr(),
                           d_out.data_ptr())

    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {nbytes} bytes read + {nbytes} bytes written")
        del src, dst

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    eng.check_device_errors()

    eng.set_probe(args.probe_layer)
    per_step = []
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for k in range(args.steps):
        step()
        ev[k + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    probe, nprobe = eng.read_probe()
    eng.set_probe(-1)
    eng.check_device_errors()
    per_step = [ev[k].elapsed_time(ev[k + 1]) for k in range(args.steps)]
    gpu_ms = sum(per_step)
    ms_per_step = wall * 1e3 / args.steps
    value = T * args.steps / wall
    avg = {k: v / max(nprobe, 1) for k, v in probe.items()}
    log("per-launch ms (layer %d): %s" % (args.probe_layer, {k: round(v, 4) for k, v in avg.items()}))

    prec = args.precision
    # Roofline kernel: the Wi projection with the fused GeGLU epilogue, the
    # largest projection GEMM (N = 2I = 2304, K = H = 768); every launch of its
    # kernel symbol has this shape, so rocprof's per-symbol average is the
    # per-launch duration measured here. With few tokens (cfg2, cfg5: the
    # small-M kernel) the launch streams the weights and is bounded by HBM:
    # achieved = algorithmic bytes (weights + activations in + out) / time.
    wi_flop = 2.0 * T * (2 * I) * H
    esz = 2 if prec == "bf16" else 4
    wi_bytes = esz * (T * H + 2 * I * H + T * I)
    wi_s = avg["gemm_wi"] * 1e-3
    hbm_bound = T <= 128
    traffic = None
    tpath = os.path.join(HERE, "profiles", "gemm_wi_geglu_cfg3_traffic.json")
    if args.config == "cfg3" and prec == "bf16" and os.path.exists(tpath):
        with open(tpath) as fh:
            traffic = json.load(fh).get("hbm_bytes_per_launch")
    if hbm_bound:
        roof = {"bound": "hbm", "achieved": round(wi_bytes / wi_s / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(wi_bytes / wi_s / 8e12, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(wi_flop / wi_s / 1e12, 2), "peak": PEAK[prec] / 1e12,
                "unit": "TFLOP/s", "frac": round(wi_flop / wi_s / PEAK[prec], 4)}
    gemm_ms = avg["gemm_qkv"] + avg["gemm_wo"] + avg["gemm_wi"] + avg["gemm_mlpwo"]
    gemm_tflops = PROJ_FLOP_PER_TOKEN_LAYER * T / (gemm_ms * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": prec,
        "data": "synthetic: random-init weights N(0,0.02) (InitRandom semantics, numpy PCG64 seed 0), "
                "token ids uniform in [5,50368) minus specials, packed [CLS] premise [SEP] ([MASK] option)xK",
        "config": {"workload": WORKLOADS[args.config], "batch": len(batch), "seq_len": int(seq_len.max()),
                   "tokens_per_step": T, "rows_per_step": R, "layers": cfg.layers, "precision": prec},
        "gpu_ms_per_step_events": round(gpu_ms / args.steps, 4),
        "step_ms_p50": round(float(np.percentile(per_step, 50)), 4),
        "step_ms_p99": round(float(np.percentile(per_step, 99)), 4),
        "projection_gemm_tflops": round(gemm_tflops, 2),
        "projection_gemm_frac_peak": round(gemm_tflops * 1e12 / PEAK[prec], 4),
        "per_launch_ms": {k: round(v, 5) for k, v in avg.items()},
        "roofline": dict({"kernel": "%s, EPI_GEGLU (Wi projection + fused GeGLU), layer %d"
                                    % ("gemm_skinny_kernel" if hbm_bound else "gemm_nt_kernel", args.probe_layer)},
                         **roof, traffic=traffic, flop_per_launch=wi_flop, algorithmic_bytes_per_launch=wi_bytes),
    }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(cfg, weights, args.config, args.cpu_budget)
    eng.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
