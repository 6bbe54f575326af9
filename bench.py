"""Prefill benchmark of SAF's mixed-head attention path on one MI355X.

Default workload ("C2"): the 124M nanoGPT
(12 layers, 12 heads, d_model 768, head_dim 64, vocab 50304, RoPE, bias-free)
in bf16 with random-init weights (seed 1337), B=1, T=16384, uniform random
tokens; a random 25% of the (layer, head) pairs (36 of 144) frozen, each to the
causal mean, an exponential decay (rate ~U(0.001, 0.1)) or a sliding window
(w ~U{64..1024}), installed as decomposed heads and run by the closed-form
scan.  One step = model(x) to last-position logits under inference_mode
(nanogpt/bench_inference_triton.py:193-196 of the reference).

Prints ONE JSON line: whole-job prefill tokens/s, the roofline of the
dominant kernel (live-head flash, bf16 MFMA) measured with HIP events over the
timed region, and a CPU baseline (the oracle's restatement of the reference's
CPU path, timed on a bounded sample on this host).
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "selective-attention-freezing_amd")
for _p in (PKG, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "prefill tokens/sec (1 GPU) + % bf16 MFMA / HBM roofline, 124M SAF-25 @16K ctx"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_c2_model(T, device, dtype, seed=1337, n_layer=12):
    import torch
    from nanogpt.model import GPT, GPTConfig

    torch.manual_seed(seed)
    cfg = GPTConfig(block_size=T, vocab_size=50304, n_layer=n_layer, n_head=12, n_embd=768,
                    bias=False, position_encoding="rope", rand_attn_prior_repr="decomposed",
                    rand_seed=seed)
    model = GPT(cfg)
    g = torch.Generator().manual_seed(seed)
    n_pairs = n_layer * cfg.n_head
    pairs = torch.randperm(n_pairs, generator=g)[: n_pairs // 4].tolist()
    plan = {}
    for idx in pairs:
        layer, head = divmod(idx, cfg.n_head)
        kind = int(torch.randint(0, 3, (1,), generator=g))
        if kind == 0:
            plan.setdefault(layer, []).append((head, "mean", 0.0))
        elif kind == 1:
            rate = 0.001 + 0.099 * float(torch.rand(1, generator=g))
            plan.setdefault(layer, []).append((head, "decay", rate))
        else:
            w = int(torch.randint(64, 1025, (1,), generator=g))
            plan.setdefault(layer, []).append((head, "window", float(w)))
    model = model.to(device=device, dtype=dtype).eval()
    d = torch.arange(T, device=device, dtype=torch.float32)
    for layer, heads in plan.items():
        alpha = torch.zeros(len(heads), T, device=device)
        rho = torch.zeros(len(heads), T, device=device)
        for n, (_, kind, prm) in enumerate(heads):
            if kind == "decay":
                rho[n] = -prm * d
            elif kind == "window":
                rho[n] = torch.where(d < prm, 0.0, float("-inf"))
        model.transformer.h[layer].attn.freeze_heads_decomposed([h for h, _, _ in heads], alpha, rho)
    gx = torch.Generator().manual_seed(seed + 1)
    x = torch.randint(0, 50257, (1, T), generator=gx).to(device)
    return model, x, plan


TRAFFIC_FILE = os.path.join(REPO, "profiles", "flash_fwd_c2_hbm_traffic.txt")


def pmc_traffic(kernel_label):
    """HBM bytes per dispatch of a kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith(kernel_label + ":"):
            for part in line.split(","):
                k, _, v = part.partition("=")
                if k.strip() == "traffic_bytes":
                    return int(float(v))
    return None


def live_flops(plan, n_layer, n_head, B, T, hd):
    n_frozen = sum(len(v) for v in plan.values())
    n_live = n_layer * n_head - n_frozen
    return n_live * B * 4 * hd * T * (T + 1) // 2, n_live, n_frozen


def cpu_baseline(model, x, plan, T, max_layers=2):
    """Oracle restatement of the reference's CPU split path (fp32) on a bounded
    sample: `max_layers` of the model's layers at the full C2 shape plus the
    embedding / final norm / head, extrapolated linearly to all layers."""
    import torch
    from oracle import model_oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = model.config
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    freeze = []
    for layer, blk in enumerate(model.transformer.h):
        a = blk.attn
        rec = {"frozen": a.dyn_frozen.cpu().tolist(), "patterns": {}, "decomp": {}}
        for h in range(cfg.n_head):
            if rec["frozen"][h]:
                rec["decomp"][h] = (a.dyn_alpha[h].cpu(), a.dyn_rho[h].cpu(), a.dyn_z[h].cpu())
        freeze.append(rec)
    ocfg = {"n_layer": cfg.n_layer, "n_head": cfg.n_head, "n_embd": cfg.n_embd,
            "position_encoding": "rope", "rope_base": cfg.rope_base}
    idx = x.cpu()
    layers = list(range(min(max_layers, cfg.n_layer)))
    times = []
    for it in range(2):
        t0 = time.perf_counter()
        model_oracle.gpt_forward(sd, ocfg, freeze, idx, path="split", layers=layers)
        times.append(time.perf_counter() - t0)
        log(f"cpu baseline sample {it}: {times[-1]:.2f} s on {threads} threads")
    t_sample = min(times)
    t_full = t_sample * cfg.n_layer / len(layers)
    tok_s = idx.numel() / t_full
    return {"value": round(tok_s, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle split-path forward (fp32, torch CPU) of {len(layers)} of "
                       f"{cfg.n_layer} C2 layers at B=1 T={T} plus embedding/head, best of 2, "
                       f"extrapolated linearly to {cfg.n_layer} layers "
                       f"({t_sample:.2f} s per sample)")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seq-len", type=int, default=16384)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=2)
    ap.add_argument("--no-timer", action="store_true", help="skip per-kernel HIP events")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run device-to-device copies of this many MiB (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the mixed-head prefill on a single "
              f"MI355X and has no multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import torch
    import kernel
    from nanogpt import model as model_mod

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)
        return

    dev = "cuda"
    T = args.seq_len
    log(f"building C2 model T={T} layers={args.layers}")
    model, x, plan = build_c2_model(T, dev, torch.bfloat16, n_layer=args.layers)
    log("model built; verifying dispatch")
    cfg = model.config
    hd = cfg.n_embd // cfg.n_head
    flops, n_live, n_frozen = live_flops(plan, cfg.n_layer, cfg.n_head, 1, T, hd)

    with torch.inference_mode():
        before = model_mod.fused_dispatch_count()
        model(x)
        torch.cuda.synchronize()
        calls = model_mod.fused_dispatch_count() - before
        if calls != cfg.n_layer:
            raise RuntimeError(f"dispatch verification failed: {calls} != {cfg.n_layer}")
        for _ in range(args.warmup):
            model(x)
        torch.cuda.synchronize()

        log(f"warmup done; timing {args.steps} steps")
        timer = None if args.no_timer else kernel.KernelTimer()
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
        kernel.set_kernel_timer(timer)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s, e in zip(starts, ends):
            s.record()
            model(x)
            e.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        kernel.set_kernel_timer(None)

    step_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    total_ms = sum(step_ms)
    tok_s = x.numel() * args.steps / (total_ms / 1000.0)

    roof = None
    extra = {}
    if timer is not None:
        summ = timer.summary()
        if "flash" in summ:
            n, ms, work = summ["flash"]
            per_launch_ms = ms / n
            achieved = (work / n) / (per_launch_ms / 1000.0) / 1e12
            label = "flash_fwd_kernel<bf16,64,2>"
            roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                    "traffic": pmc_traffic(label) if T == 16384 else None,
                    "traffic_source": "profiles/flash_fwd_c2_hbm_traffic.txt", "kernel": label,
                    "launches": n, "avg_launch_ms": round(per_launch_ms, 4),
                    "flop_per_launch": work // n}
        if "scan" in summ:
            n, ms, work = summ["scan"]
            gbs = (work / n) / (ms / n / 1000.0) / 1e9
            extra["frozen_scan"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                    "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                    "launches": n, "avg_launch_ms": round(ms / n, 4),
                                    "bytes_per_launch": work // n}
        extra["attention_ms_per_step"] = round(sum(v[1] for v in summ.values()) / args.steps, 3)

    log(f"GPU: {tok_s:.0f} tokens/s, {total_ms / args.steps:.2f} ms/step")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(model, x, plan, T, max_layers=args.cpu_layers)

    line = {
        "metric": METRIC, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights seed 1337, uniform random tokens)",
        "config": {"workload": f"C2: 124M SAF-25% prefill, B=1, T={T}, {cfg.n_layer} layers, "
                               f"{n_frozen}/{cfg.n_layer * cfg.n_head} heads frozen "
                               f"(mean/decay/window closed-form scan), {n_live} live",
                   "batch": 1, "seq_len": T, "frozen_heads": n_frozen, "live_heads": n_live,
                   "median_step_ms": round(statistics.median(step_ms), 3),
                   "wall_s": round(wall, 3)},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
