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

--workload c4 --rate r measures BASELINE.json configs[4] instead: the
Qwen-style GQA model (transformers Qwen3 modules, random init) with
round(14 r) query heads per layer frozen to the causal mean, B=4, T=4096,
one step = backbone prefill to the last hidden state.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "selective-attention-freezing_amd")
for _p in (PKG, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "prefill tokens/sec (1 GPU) + % bf16 MFMA / HBM roofline, 124M SAF-25 @16K ctx"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
# v_exp_f32 issue ceiling: 256 CUs x 4 SIMDs x 64 lanes per 4-cycle
# transcendental issue x 2.4 GHz
EXP_ISSUE_PEAK = 256 * 4 * 64 / 4 * 2.4e9
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


def build_c0_model(device, dtype, T=1024, seed=1337, n_layer=12):
    """the 124M nanoGPT (random-init fp32 weights, seed
    1337), 3 of 12 heads per layer frozen to the causal mean (heads
    randperm(12) of a generator seeded 1337 + layer), installed as decomposed
    heads with alpha = rho = 0 (the reference's own statement that zero
    logits are the causal-uniform prior, nanogpt/bench_inference_triton.py:92-97);
    tokens uniform in [0, 50257), B = 1."""
    import torch
    from nanogpt.model import GPT, GPTConfig

    torch.manual_seed(seed)
    cfg = GPTConfig(block_size=T, vocab_size=50304, n_layer=n_layer, n_head=12, n_embd=768,
                    bias=False, position_encoding="rope", rand_attn_prior_repr="decomposed",
                    rand_seed=seed)
    model = GPT(cfg).to(device=device, dtype=dtype).eval()
    plan = {}
    for layer, blk in enumerate(model.transformer.h):
        heads = torch.randperm(12, generator=torch.Generator().manual_seed(seed + layer))[:3].tolist()
        z = torch.zeros(3, T, device=device)
        blk.attn.freeze_heads_decomposed(heads, z, z)
        plan[layer] = [(h, "mean", 0.0) for h in heads]
    x = torch.randint(0, 50257, (1, T), generator=torch.Generator().manual_seed(seed + 1)).to(device)
    return model, x, plan


TRAFFIC_FILE = os.path.join(REPO, "profiles", "flash_fwd_c2_hbm_traffic.txt")
SCAN_TRAFFIC_FILE = os.path.join(REPO, "profiles", "frozen_scan_sizing_hbm_traffic.txt")


def pmc_traffic(kernel_label, path=TRAFFIC_FILE):
    """HBM bytes per dispatch of a kernel from a committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    if not os.path.exists(path):
        return None
    for line in open(path):
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


def _oracle_inputs(model):
    """State dict (fp32 copy of the model's own weights) and per-layer freeze
    records of a GPT, in the oracle's input format."""
    cfg = model.config
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    freeze = []
    for blk in model.transformer.h:
        a = blk.attn
        rec = {"frozen": a.dyn_frozen.cpu().tolist(), "patterns": {}, "decomp": {}}
        for h in range(cfg.n_head):
            if rec["frozen"][h]:
                rec["decomp"][h] = (a.dyn_alpha[h].cpu(), a.dyn_rho[h].cpu(), a.dyn_z[h].cpu())
        freeze.append(rec)
    ocfg = {"n_layer": cfg.n_layer, "n_head": cfg.n_head, "n_embd": cfg.n_embd,
            "position_encoding": "rope", "rope_base": cfg.rope_base}
    return sd, ocfg, freeze


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(c2_model, c2_x, T, c2_layers=1, iters=5):
    """The reference's CPU path (the oracle's restatement of its split
    fallback, fp32 torch on this host's cores) at BASELINE configs[0], C0:
    the full 12-layer 124M forward at B=1, T=1024 with 3 causal-mean heads
    per layer, 1 warmup and `iters` timed forwards, median.  The same C0
    model runs on the GPU in bf16 beside it (prefill tokens/s at the same
    shape, and its last-position logits against the CPU forward's).  A
    secondary figure extrapolates `c2_layers` layers of the C2 model at its
    full shape to all 12 layers."""
    import torch
    from oracle import model_oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    m0, x0, _ = build_c0_model("cuda", torch.bfloat16)
    with torch.inference_mode():
        for _ in range(3):
            m0(x0)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
        for a, b in ev:
            a.record()
            gpu_last = m0(x0)
            b.record()
        torch.cuda.synchronize()
    gpu_ms = statistics.median(a.elapsed_time(b) for a, b in ev)
    sd, ocfg, freeze = _oracle_inputs(m0)
    idx = x0.cpu()
    del m0
    times = []
    for it in range(iters + 1):
        t0 = time.perf_counter()
        ref = model_oracle.gpt_forward(sd, ocfg, freeze, idx, path="split")
        dt = time.perf_counter() - t0
        if it:
            times.append(dt)
        log(f"cpu baseline C0 forward {it}: {dt:.3f} s on {threads} threads" + ("" if it else " (warmup)"))
    t_med = statistics.median(times)
    a = gpu_last.float().cpu().double().flatten()
    b = ref.double().flatten()
    cos = float(a @ b / (a.norm() * b.norm()))
    tokens = idx.numel()
    out = {"value": round(tokens / t_med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
           "sample": (f"C0 (BASELINE configs[0]): the full 12-layer 124M forward to last-position logits, "
                      f"B=1, T={tokens}, 3 causal-mean heads per layer, oracle split path (the reference's "
                      f"CPU fallback) in fp32 torch; 1 warmup + {iters} timed, median {t_med:.3f} s"),
           "cpu_model": cpu_model_name(), "torch_threads": torch.get_num_threads(),
           "gpu_same_shape": {"value": round(tokens / (gpu_ms / 1000.0), 1), "unit": "tokens/s",
                              "ms_per_forward": round(gpu_ms, 3), "dtype": "bf16",
                              "logits_cosine_vs_cpu": round(cos, 7)}}
    if c2_layers:
        sd2, ocfg2, freeze2 = _oracle_inputs(c2_model)
        idx2 = c2_x.cpu()
        layers = list(range(min(c2_layers, ocfg2["n_layer"])))
        t0 = time.perf_counter()
        model_oracle.gpt_forward(sd2, ocfg2, freeze2, idx2, path="split", layers=layers)
        dt = time.perf_counter() - t0
        t_full = dt * ocfg2["n_layer"] / len(layers)
        out["c2_extrapolated"] = {
            "value": round(idx2.numel() / t_full, 2), "unit": "tokens/s",
            "sample": (f"{len(layers)} of {ocfg2['n_layer']} C2 layers at B=1 T={T} plus embedding/head "
                       f"({dt:.2f} s), scaled linearly to all layers")}
        log(f"cpu baseline C2 sample: {dt:.2f} s for {len(layers)} layer(s)")
    return out


def c4_cpu_baseline(model, sd, masks, B, T, max_layers=1):
    """The oracle's restatement of the hybrid Qwen3 split path (fp32, torch CPU)
    on a bounded sample: `max_layers` layers at B=1 and the full T, plus
    embedding and final norm, extrapolated linearly to all layers and B."""
    import torch
    from oracle import qwen_oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = model.config
    mean = torch.ones(T, T).tril_()
    fr = [{"mask": m.numpy(), "dense": mean.expand(cfg.num_attention_heads, T, T)} for m in masks]
    ocfg = dict(n_layers=cfg.num_hidden_layers, n_heads=cfg.num_attention_heads,
                n_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, eps=cfg.rms_norm_eps,
                rope_theta=1e6)
    idx = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(2))
    layers = list(range(min(max_layers, cfg.num_hidden_layers)))
    times = []
    for it in range(2):
        t0 = time.perf_counter()
        qwen_oracle.qwen_forward(sd, ocfg, fr, idx, layers=layers)
        times.append(time.perf_counter() - t0)
        log(f"cpu baseline sample {it}: {times[-1]:.2f} s on {threads} threads")
    t_sample = min(times)
    t_full = t_sample * cfg.num_hidden_layers / len(layers) * B
    return {"value": round(B * T / t_full, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle hybrid Qwen3 split-path forward (fp32, torch CPU) of {len(layers)} of "
                       f"{cfg.num_hidden_layers} layers at B=1 T={T}, best of 2, extrapolated "
                       f"linearly to all layers and B={B} ({t_sample:.2f} s per sample)")}


def _time_pass(step, steps, timer):
    import torch
    import kernel
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    kernel.set_kernel_timer(timer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s, e in zip(starts, ends):
        s.record()
        step()
        e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel.set_kernel_timer(None)
    return [s.elapsed_time(e) for s, e in zip(starts, ends)], wall


def timed_steps(step, steps, warmup, use_timer):
    """Warm up, then time exactly `steps` calls of step() with HIP events;
    these uninstrumented steps give the throughput.  With use_timer, `steps`
    further calls carry per-kernel HIP events around every attention kernel
    (each event is a marker packet that drains the stream, about 2-3% of a
    C2 step) and give the kernel figures; the throughput never includes
    them."""
    import torch
    import kernel
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log(f"warmup done; timing {steps} steps")
    step_ms, wall = _time_pass(step, steps, None)
    summ = None
    if use_timer:
        timer = kernel.KernelTimer()
        inst_ms, _ = _time_pass(step, steps, timer)
        summ = timer.summary()
        log(f"kernel-timer pass: {sum(inst_ms) / steps:.3f} ms/step with per-kernel events")
    return step_ms, wall, summ


def kernel_rooflines(summ, flash_label, traffic, steps):
    """Roofline of the live-head flash kernel (bf16 MFMA) plus the frozen-head
    kernels' HBM figures, from the per-launch HIP event times."""
    roof, extra = None, {}
    if summ is None:
        return roof, extra
    if "flash" in summ:
        n, ms, work = summ["flash"]
        per_launch_ms = ms / n
        achieved = (work / n) / (per_launch_ms / 1000.0) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic,
                "traffic_source": "profiles/flash_fwd_c2_hbm_traffic.txt" if traffic else None,
                "kernel": flash_label, "launches": n, "avg_launch_ms": round(per_launch_ms, 4),
                "flop_per_launch": work // n}
    if "scan" in summ:
        n, ms, work = summ["scan"]
        gbs = (work / n) / (ms / n / 1000.0) / 1e9
        extra["frozen_scan"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                "launches": n, "avg_launch_ms": round(ms / n, 4),
                                "bytes_per_launch": work // n}
    if "dense" in summ:
        n, ms, work = summ["dense"]
        extra["frozen_dense_pv"] = {"launches": n, "avg_launch_ms": round(ms / n, 4),
                                    "flop_per_launch": work // n}
    # kernels on the launch stream only: the scan runs on a side stream
    # beside them, so its span would count time twice
    extra["attention_kernels_ms_per_step"] = round(
        sum(v[1] for k, v in summ.items() if k != "scan") / steps, 3)
    return roof, extra


C2_FIXTURE = os.path.join(REPO, "tests", "golden", "c2_last_logits.npz")


def c2_check(model, x):
    """Cosine of the GPU prefill output (last-position logits) against the
    fp32 oracle's logits for the same C2 model and tokens, computed on the
    host and stored by tests/golden/make_c2_fixture.py; None if the fixture
    is absent or was made for another shape."""
    import hashlib
    import torch
    if not os.path.exists(C2_FIXTURE):
        return None
    z = np.load(C2_FIXTURE)
    tok = hashlib.sha256(x.cpu().numpy().astype(np.int64).tobytes()).hexdigest()
    if str(z["tokens_sha256"]) != tok:
        return None
    with torch.inference_mode():
        got = model(x)[0, -1].double().cpu()
    ref = torch.from_numpy(z["logits"]).double()
    cos = float(got @ ref / (got.norm() * ref.norm()))
    return {"logits_cosine_vs_fp32_oracle": round(cos, 7), "pass": cos >= 0.9999, "bound": 0.9999,
            "reference": os.path.relpath(C2_FIXTURE, REPO)}


C3_FIXTURE = os.path.join(REPO, "tests", "golden", "c3_check.npz")
C4_FIXTURE = os.path.join(REPO, "tests", "golden", "c4_check.npz")


def _cosine(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return float(a @ b / (a.norm() * b.norm()))


def _fixture_for(path, tokens, **shape):
    """The fixture at `path` if it was made for these tokens and shape."""
    import hashlib
    if not os.path.exists(path):
        return None
    z = np.load(path)
    if str(z["tokens_sha256"]) != hashlib.sha256(tokens.cpu().numpy().astype(np.int64).tobytes()).hexdigest():
        return None
    if any(int(z[k]) != v for k, v in shape.items()):
        return None
    return z


def c3_check(model, x):
    """Cosine of the GPU prefill (last-position logits of both sequences, and
    the final LayerNorm output at sampled positions) against the fp32 oracle's
    values stored by tests/golden/make_c3_fixture.py; None if the fixture is
    absent or was made for another workload."""
    import torch
    z = _fixture_for(C3_FIXTURE, x, T=x.size(1), L=model.config.n_layer)
    if z is None:
        return None
    with torch.inference_mode():
        last = model(x)[:, -1].float().cpu()
        hid = model.forward_hidden(x)[:, torch.as_tensor(z["positions"], device=x.device)].float().cpu()
    cl = _cosine(last, torch.from_numpy(z["logits_last"]))
    ch = _cosine(hid, torch.from_numpy(z["hidden"]))
    return {"logits_cosine_vs_fp32_oracle": round(cl, 7), "hidden_cosine_vs_fp32_oracle": round(ch, 7),
            "pass": min(cl, ch) >= 0.9999, "bound": 0.9999, "reference": os.path.relpath(C3_FIXTURE, REPO)}


def c4_check(backbone, ids, f, L, bound=None):
    """Cosine of the GPU backbone output (final-norm hidden states at sampled
    positions of every sequence) against the fp32 oracle's, stored per frozen
    count f by tests/golden/make_c4_fixture.py; None if absent.  The default
    bound (bf16 runs) allows 1.5x the error that the same model reaches in
    bf16 through torch alone on the host (stored beside the oracle values):
    this 24-layer random-init model amplifies bf16 rounding, and transformers'
    own bf16 forward of it stays near cosine 0.9997."""
    import torch
    import qwen
    z = _fixture_for(C4_FIXTURE, ids, T=ids.size(1), B=ids.size(0), L=L)
    if z is None or f"hidden_f{f}" not in z.files:
        return None
    with torch.inference_mode():
        got = qwen.backbone_forward(backbone, ids)[:, torch.as_tensor(z["positions"], device=ids.device)]
    c = _cosine(got.float().cpu(), torch.from_numpy(z[f"hidden_f{f}"]))
    level = float(z[f"bf16_cos_f{f}"])
    if bound is None:
        bound = 1.0 - 1.5 * (1.0 - level)
    return {"hidden_cosine_vs_fp32_oracle": round(c, 7), "torch_bf16_cosine": round(level, 7),
            "pass": c >= bound, "bound": round(bound, 7), "reference": os.path.relpath(C4_FIXTURE, REPO)}


def run_c2(args):
    import torch
    from nanogpt import model as model_mod

    dev = "cuda"
    T = args.seq_len or 16384
    log(f"building C2 model T={T} layers={args.layers}")
    model, x, plan = build_c2_model(T, dev, torch.bfloat16, n_layer=args.layers)
    log("model built; verifying dispatch and output")
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
    check = c2_check(model, x) if cfg.n_layer == 12 else None
    if check is not None:
        log(f"C2 logits cosine vs the fp32 oracle: {check['logits_cosine_vs_fp32_oracle']:.7f}")
        if not check["pass"]:
            log("WARNING: the C2 prefill output fails the logits bound")
    with torch.inference_mode():
        step_ms, wall, summ = timed_steps(lambda: model(x), args.steps, args.warmup, not args.no_timer)

    total_ms = sum(step_ms)
    tok_s = x.numel() * args.steps / (total_ms / 1000.0)
    label = "flash_fwd_kernel<bf16,64,1>"
    roof, extra = kernel_rooflines(summ, label, pmc_traffic(label) if T == 16384 else None, args.steps)
    log(f"GPU: {tok_s:.0f} tokens/s, {total_ms / args.steps:.2f} ms/step")
    if "frozen_scan" in extra:
        # in the model the scan shares the GPU with the flash kernel (side
        # stream): its event span is not an HBM fraction
        sc = extra.pop("frozen_scan")
        extra["frozen_scan_in_model"] = {
            "launches": sc["launches"], "avg_span_ms": sc["avg_launch_ms"],
            "bytes_per_launch": sc["bytes_per_launch"],
            "note": "runs on a side stream overlapped with the live-head kernel; span, not HBM time"}
    frozen_roof = None
    if not args.no_sizing_scan:
        _, frozen_roof, _, _ = sizing_scan(8, 16384, max(args.steps, 10), 3)
        frozen_roof["workload"] = ("frozen-only sizing run B=8, H=12 closed-form heads, T=16384, hd 64 "
                                   "(403 MB per launch), timed in this process")
        log(f"frozen sizing scan: {frozen_roof['achieved']:.0f} GB/s = {frozen_roof['frac']:.3f} of HBM")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(model, x, T, c2_layers=args.cpu_layers)

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
        "frozen_roofline": frozen_roof,
        "check": check,
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def run_c4(args):
    """Qwen-style GQA (24 layers, hidden 896, 14 query /
    2 KV heads, head_dim 64, RoPE theta 1e6), bf16 random init, B=4, T=4096;
    round(rate * 14) query heads per layer frozen to the causal mean.  One step
    = backbone prefill to the last hidden state (bench_qwen_prefill_triton.py
    of the reference)."""
    import torch
    import qwen

    dev = "cuda"
    T = args.seq_len or 4096
    B = args.batch or 4
    cfg = qwen.qwen_config(n_layers=args.layers or 24, max_positions=max(T, 4096))
    log(f"building C4 model B={B} T={T} rate={args.rate} prior={args.prior_repr}")
    model = qwen.build_model(cfg, device=dev, dtype=torch.bfloat16, seed=1337)
    use_sdpa = args.rate == 0 and args.sdpa_live
    masks = qwen.nested_head_masks(args.rate, cfg.num_hidden_layers, cfg.num_attention_heads)
    sd = None
    if not args.no_cpu_baseline:   # the oracle reads the unconverted parameter names
        sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()
              if not k.startswith("lm_head")}
    if not use_sdpa:
        _, masks = qwen.convert_with_rate(model, args.rate, T, repr=args.prior_repr,
                                          fuse_live_only=args.rate == 0)
    f = int(masks[0].sum())
    H, L, hd = cfg.num_attention_heads, cfg.num_hidden_layers, cfg.head_dim
    ids = torch.randint(0, 151643, (B, T), generator=torch.Generator().manual_seed(1337)).to(dev)
    backbone = model.model
    with torch.inference_mode():
        n0 = qwen.fused_dispatch_count()
        qwen.backbone_forward(backbone, ids)
        torch.cuda.synchronize()
        calls = qwen.fused_dispatch_count() - n0
        if calls != (0 if use_sdpa else L):
            raise RuntimeError(f"dispatch verification failed: {calls} fused calls for {L} layers")
    check = c4_check(backbone, ids, f, L)
    if check is not None:
        log(f"check against the fp32 oracle fixture: {check}")
        if not check["pass"]:
            raise RuntimeError(f"C4 output check failed: {check}")
    with torch.inference_mode():
        step_ms, wall, summ = timed_steps(lambda: qwen.backbone_forward(backbone, ids), args.steps,
                                          args.warmup, not args.no_timer and not use_sdpa)
    total_ms = sum(step_ms)
    tok_s = B * T * args.steps / (total_ms / 1000.0)
    roof, extra = kernel_rooflines(summ, "flash_fwd_kernel<bf16,64,1>", None, args.steps)
    log(f"GPU: {tok_s:.0f} tokens/s, {total_ms / args.steps:.2f} ms/step")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = c4_cpu_baseline(model, sd, masks, B, T, max_layers=args.cpu_layers)
    attn = "torch SDPA for every head (unconverted model)" if use_sdpa else (
        f"fused HIP path, frozen heads as {args.prior_repr} priors"
        + (" (closed-form mean scan)" if args.prior_repr == "decomposed" else " (dense P.V)"))
    line = {
        "metric": "prefill tokens/sec (1 GPU), Qwen-style GQA with frozen query heads",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights seed 1337, uniform random tokens)",
        "config": {"workload": f"C4: Qwen3-style GQA {L}L hidden 896 14q/2kv hd 64, B={B}, T={T}, "
                               f"{f}/{H} query heads frozen per layer (rate {args.rate}); {attn}",
                   "batch": B, "seq_len": T, "frozen_per_layer": f, "live_per_layer": H - f,
                   "live_flops": (H - f) * L * B * 4 * hd * T * (T + 1) // 2,
                   "frozen_bytes": f * L * B * 2 * T * hd * 2,
                   "median_step_ms": round(statistics.median(step_ms), 3),
                   "wall_s": round(wall, 3)},
        "roofline": roof,
        "check": check,
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def run_c1(args):
    """the isolated mixed-head attention op at the 124M
    shape, B=8, H=12, T=4096, hd=64, bf16 Q/K/V ~ N(0, 1) from a CPU
    generator (seed 1337); heads randperm(12)[:3] frozen to exponential-decay
    patterns, rate ~U(0.001, 0.1), rows renormalised.  The same op runs with
    the decay heads as closed forms (the O(T) scan; the primary run), as
    generic decomposed heads (the decomposed P.V kernel) and
    materialised as dense bf16 patterns (the MFMA P.V kernel); frozen_pv (the
    split path) is timed on the same dense patterns.  The decomposed heads
    run beside the live-head kernel on a side stream ("decomp"), after it on
    one stream ("decomp_split") and alone ("decomp_alone": their kernels'
    own roofline)."""
    import torch
    import kernel

    B, H, hd = args.batch or 8, 12, 64
    T = args.seq_len or 4096
    g = torch.Generator().manual_seed(1337)
    fz = sorted(torch.randperm(H, generator=g)[:3].tolist())
    rates = [0.001 + 0.099 * float(x) for x in torch.rand(3, generator=g)]
    live = [h for h in range(H) if h not in fz]
    q = torch.randn(B, len(live), T, hd, generator=g).bfloat16().cuda()
    k = torch.randn(B, len(live), T, hd, generator=g).bfloat16().cuda()
    v = torch.randn(B, H, T, hd, generator=g).bfloat16().cuda()
    hidx = torch.zeros(H, dtype=torch.int32)
    for slot, h in enumerate(live):
        hidx[h] = slot
    d = torch.arange(T, dtype=torch.float32)
    alpha = torch.zeros(H, T)
    rho = torch.zeros(H, T)
    for f, c in zip(fz, rates):
        rho[f] = -c * d
    alpha, rho = alpha.cuda(), rho.cuda()
    z = kernel.decomposed_logz(alpha, rho)
    cf = kernel.classify_closed_form(alpha, rho, z)
    frozen2 = torch.zeros(H, dtype=torch.int32)
    frozen2[fz] = 2
    frozen1 = torch.zeros(H, dtype=torch.int32)
    frozen1[fz] = 1
    pidx = torch.zeros(H, dtype=torch.int32)
    for slot, f in enumerate(fz):
        pidx[f] = slot
    # the decay patterns materialised: P[i, j] = e^{-c (i - j)} / Z_i for j <= i
    ii = torch.arange(T, device="cuda", dtype=torch.float32)
    dist = (ii[:, None] - ii[None, :]).clamp_min(0)
    patt = torch.empty(len(fz), T, T, device="cuda", dtype=torch.bfloat16)
    for slot, c in enumerate(rates):
        pm = torch.exp(-c * dist).tril_()
        patt[slot] = (pm / pm.sum(-1, keepdim=True)).bfloat16()
        del pm
    del dist
    # the routing tables are resident inputs like q/k/v: created once, so the
    # op's host copy of them (cached on the tensor) is made at the first call
    # only, as in the model
    frozen2, frozen1, hidx, pidx = frozen2.cuda(), frozen1.cuda(), hidx.cuda(), pidx.cuda()
    vd = v[:, fz].contiguous()
    q0 = q[:, :0]
    frozen_d = torch.full((len(fz),), 2, dtype=torch.int32, device="cuda")
    alpha_d, rho_d, z_d = alpha[fz].contiguous(), rho[fz].contiguous(), z[fz].contiguous()
    runs = {
        "scan": lambda: kernel.fused_mixed_attn(q, k, v, None, frozen2, hidx, alpha=alpha, rho=rho, z=z,
                                                 closed_form=cf, validate=False),
        "decomp": lambda: kernel.fused_mixed_attn(q, k, v, None, frozen2, hidx, alpha=alpha, rho=rho, z=z,
                                                   validate=False),
        "dense": lambda: kernel.fused_mixed_attn(q, k, v, patt, frozen1, hidx, pidx, validate=False),
        # the decomposed heads after the live-head kernel on one stream, key
        # segments split (the schedule before the side-stream one)
        "decomp_split": lambda: kernel.fused_mixed_attn(q, k, v, None, frozen2, hidx, alpha=alpha, rho=rho, z=z,
                                                         validate=False, decomp_unsplit=False),
        # the decomposed heads alone (their kernels' own roofline)
        "decomp_alone": lambda: kernel.fused_mixed_attn(q0, q0, vd, None, frozen_d, None, alpha=alpha_d,
                                                         rho=rho_d, z=z_d, validate=False),
    }
    if args.c1_legs:
        keep = set(args.c1_legs.split(",")) | {"scan"}
        unknown = keep - set(runs)
        if unknown:
            raise SystemExit(f"--c1-legs: unknown legs {sorted(unknown)}")
        runs = {k2: fn for k2, fn in runs.items() if k2 in keep}
    n_live, nf = len(live), len(fz)
    flops_live = n_live * B * 4 * hd * T * (T + 1) // 2
    res = {}
    with torch.inference_mode():
        for name, fn in runs.items():
            step_ms, wall, summ = timed_steps(fn, args.steps, args.warmup, not args.no_timer)
            roof, extra = kernel_rooflines(summ, "flash_fwd_kernel<bf16,64,1>", None, args.steps)
            entry = {"ms_per_op": round(sum(step_ms) / args.steps, 4)}
            if roof:
                entry["flash"] = {k2: roof[k2] for k2 in ("achieved", "frac", "avg_launch_ms")}
            if summ and "dense" in summ:
                n, ms, fl = summ["dense"]
                nbytes = nf * T * (T + 1) // 2 * 2 + nf * B * 2 * T * hd * 2
                entry["frozen_dense_pv"] = {"avg_launch_ms": round(ms / n, 4), "bytes_per_launch": nbytes,
                                            "achieved_gbs": round(nbytes / (ms / n / 1000) / 1e9, 1),
                                            "frac_hbm": round(nbytes / (ms / n / 1000) / 1e9 / PEAK_HBM_GBS, 4)}
            if summ and "decomp" in summ and name == "decomp_alone":
                n, ms, fl = summ["decomp"]
                entry["frozen_decomp_pv"] = {"avg_launch_ms": round(ms / n, 4), "flop_per_launch": fl // n,
                                             "achieved_tflops": round(fl / n / (ms / n / 1000) / 1e12, 1),
                                             "frac_mfma": round(fl / n / (ms / n / 1000) / 1e12 / PEAK_BF16_TFLOPS, 4)}
            if "frozen_scan" in extra:
                entry["frozen_scan"] = {k2: extra["frozen_scan"][k2] for k2 in ("achieved", "frac", "avg_launch_ms")}
            res[name] = entry
        if not args.c1_legs:
            vf = v[:, fz].contiguous()
            fz_idx = torch.arange(nf, dtype=torch.int32, device="cuda")
            step_ms, _, _ = timed_steps(lambda: kernel.frozen_pv(patt, vf, fz_idx, T), args.steps, args.warmup,
                                        False)
            res["frozen_pv_split"] = {"ms_per_op": round(sum(step_ms) / args.steps, 4)}
    prim = res["scan"]
    log("GPU: C1 op " + ", ".join(f"{k2} {e['ms_per_op']:.3f} ms" for k2, e in res.items()))
    roof, _ = None, None
    line = {
        "metric": "isolated mixed-head attention op (C1), tokens/s through the op",
        "value": round(B * T / (prim["ms_per_op"] / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": prim["ms_per_op"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (Q/K/V ~ N(0, 1), seed 1337)",
        "config": {"workload": f"C1: B={B}, H={H}, T={T}, hd={hd}; heads {fz} frozen to decay rates "
                               f"{[round(c, 4) for c in rates]}; primary run: closed-form scan",
                   "live_flops": flops_live},
        "roofline": dict(prim.get("flash", {}), bound="mfma", peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                         kernel="flash_fwd_kernel<bf16,64,1>"),
        "cpu_baseline": None,
        "runs": res,
    }
    print(json.dumps(line), flush=True)


def build_c3_model(T, L, device, seed=1337):
    """1B-class SAF model (24 layers, d_model 2048, 16
    heads, hd 128, vocab 50304, RoPE, no bias), bf16 random init; per layer
    the heads randperm(16, seed + layer)[:4] are frozen to dense
    lower-triangular row-stochastic patterns softmax(N(0,1) logits masked
    causally), stored compactly in bf16 as (4, T, T).  Weights and pattern
    logits are drawn on the CPU (seeded), so the host reproduces the device's
    model exactly (tests/golden/make_c3_fixture.py)."""
    import torch
    from nanogpt.model import GPT, GPTConfig

    torch.manual_seed(seed)
    cfg = GPTConfig(block_size=T, vocab_size=50304, n_layer=L, n_head=16, n_embd=2048, bias=False,
                    position_encoding="rope", rand_attn_prior_repr="dense", freeze_pattern_dtype="bfloat16",
                    rand_seed=seed)
    model = GPT(cfg).to(device=device, dtype=torch.bfloat16).eval()
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    plan = {}
    for layer in range(L):
        heads = torch.randperm(cfg.n_head, generator=torch.Generator().manual_seed(seed + layer))[:4].tolist()
        g = torch.Generator().manual_seed(seed + layer)
        logits = torch.randn(len(heads), T, T, generator=g)
        logits.masked_fill_(~causal, float("-inf"))
        model.transformer.h[layer].attn.freeze_heads(heads, torch.softmax(logits, dim=-1).to(device))
        del logits
        plan[layer] = [(h, "dense", 0.0) for h in heads]
    x = torch.randint(0, 50257, (2, T), generator=torch.Generator().manual_seed(seed + 1)).to(device)
    return model, x, plan


def run_c3(args):
    """C3 prefill: last-position logits of the 1B-class model at B=2,
    T=8192, with the live-head flash (hd 128) and the dense P.V rooflines."""
    import torch
    from nanogpt import model as model_mod

    dev = "cuda"
    T = args.seq_len or 8192
    L = args.layers or 24
    log(f"building C3 model T={T} layers={L}")
    model, x, plan = build_c3_model(T, L, dev)
    B = x.size(0)
    H, hd = 16, 128
    n_dense = sum(len(v) for v in plan.values())
    n_live = L * H - n_dense
    with torch.inference_mode():
        before = model_mod.fused_dispatch_count()
        model(x)
        torch.cuda.synchronize()
        if model_mod.fused_dispatch_count() - before != L:
            raise RuntimeError("dispatch verification failed")
    check = c3_check(model, x)
    if check is not None:
        log(f"check against the fp32 oracle fixture: {check}")
        if not check["pass"]:
            raise RuntimeError(f"C3 output check failed: {check}")
    with torch.inference_mode():
        step_ms, wall, summ = timed_steps(lambda: model(x), args.steps, args.warmup, not args.no_timer)
    total_ms = sum(step_ms)
    tok_s = x.numel() * args.steps / (total_ms / 1000.0)
    roof, extra = kernel_rooflines(summ, "flash_fwd_kernel<bf16,128,1>", None, args.steps)
    if summ is not None and "dense" in summ:
        n, ms, flops = summ["dense"]
        per_ms = ms / n
        # pattern causal half read once per head (batch innermost), V read and Y written per (b, h)
        nbytes = (n_dense // L) * (T * (T + 1) // 2 * 2 + B * 2 * T * hd * 2)
        gbs = nbytes / (per_ms / 1000.0) / 1e9
        tfs = (flops / n) / (per_ms / 1000.0) / 1e12
        t_hbm, t_mfma = nbytes / (PEAK_HBM_GBS * 1e9), (flops / n) / (PEAK_BF16_TFLOPS * 1e12)
        extra["frozen_dense_pv"] = {
            "bound": "hbm" if t_hbm >= t_mfma else "mfma", "kernel": f"frozen_dense_kernel<bf16,bf16,128,nb{2 if B % 2 == 0 else 1}>",
            "achieved_gbs": round(gbs, 1), "achieved_tflops": round(tfs, 1),
            "frac": round(max(t_hbm, t_mfma) / (per_ms / 1000.0), 4),
            "bytes_per_launch": nbytes, "flop_per_launch": flops // n,
            "launches": n, "avg_launch_ms": round(per_ms, 4)}
    log(f"GPU: {tok_s:.0f} tokens/s, {total_ms / args.steps:.2f} ms/step")
    line = {
        "metric": "prefill tokens/sec (1 GPU), 1B-class SAF model with dense frozen patterns",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights and patterns seed 1337, uniform random tokens)",
        "config": {"workload": f"C3: 1B-class SAF prefill, {L}L d2048 16H hd128, B={B}, T={T}, "
                               f"{n_dense}/{L * H} heads frozen to dense bf16 patterns, {n_live} live",
                   "batch": B, "seq_len": T,
                   "live_flops": n_live * B * 4 * hd * T * (T + 1) // 2,
                   "median_step_ms": round(statistics.median(step_ms), 3), "wall_s": round(wall, 3)},
        "roofline": roof,
        "check": check,
        "cpu_baseline": None,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def run_bwd(args):
    """Backward of the isolated op at the C1 shape (B=8, H=12, T=4096, hd 64,
    bf16; heads randperm(12)[:3] frozen to exponential decays, installed as
    decomposed buffers): one step = forward + backward of sum(out * w) with
    respect to q, k, v (saf_mixed_attn_bwd: delta, dQ, dK/dV of the live
    heads, dV of the frozen heads).  Reports the backward alone, with the live
    heads' work counted in the FlashAttention convention (2.5x the forward's
    4 hd T(T+1)/2 flops per (batch, live head))."""
    import torch
    import kernel

    B, H, hd = args.batch or 8, 12, 64
    T = args.seq_len or 4096
    g = torch.Generator().manual_seed(1337)
    fz = sorted(torch.randperm(H, generator=g)[:3].tolist())
    rates = [0.001 + 0.099 * float(x) for x in torch.rand(3, generator=g)]
    live = [h for h in range(H) if h not in fz]
    q = torch.randn(B, len(live), T, hd, generator=g).bfloat16().cuda().requires_grad_(True)
    k = torch.randn(B, len(live), T, hd, generator=g).bfloat16().cuda().requires_grad_(True)
    v = torch.randn(B, H, T, hd, generator=g).bfloat16().cuda().requires_grad_(True)
    hidx = torch.zeros(H, dtype=torch.int32)
    for slot, h in enumerate(live):
        hidx[h] = slot
    d = torch.arange(T, dtype=torch.float32)
    alpha = torch.zeros(H, T)
    rho = torch.zeros(H, T)
    for f, c in zip(fz, rates):
        rho[f] = -c * d
    alpha, rho = alpha.cuda(), rho.cuda()
    z = kernel.decomposed_logz(alpha, rho)
    cf = kernel.classify_closed_form(alpha, rho, z)
    frozen = torch.zeros(H, dtype=torch.int32)
    frozen[fz] = 2
    frozen, hidx = frozen.cuda(), hidx.cuda()
    w = torch.randn(B, H, T, hd, generator=g).bfloat16().cuda()

    def fwd():
        return kernel.fused_mixed_attn(q, k, v, None, frozen, hidx, alpha=alpha, rho=rho, z=z, closed_form=cf,
                                       validate=False)

    for _ in range(args.warmup):
        fwd().backward(w)
    torch.cuda.synchronize()
    e = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
          torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for e0, e1, e2 in e:
        q.grad = k.grad = v.grad = None
        e0.record()
        y = fwd()
        e1.record()
        y.backward(w)
        e2.record()
    torch.cuda.synchronize()
    fwd_ms = statistics.median(a.elapsed_time(b) for a, b, _ in e)
    bwd_ms = statistics.median(b.elapsed_time(c) for _, b, c in e)
    flops_bwd = 2.5 * len(live) * B * 4 * hd * T * (T + 1) / 2
    tfs = flops_bwd / (bwd_ms / 1000.0) / 1e12
    line = {
        "metric": "backward of the mixed-head op (live-head FLOP/s, FlashAttention convention)",
        "value": round(tfs, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(fwd_ms + bwd_ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (N(0,1) q/k/v seed 1337)",
        "config": {"workload": f"C1 op backward: B={B}, H={H}, T={T}, hd={hd}, 3 decay heads (decomposed in the "
                               f"backward, closed-form scan in the forward), {len(live)} live",
                   "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4)},
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tfs / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": "bwd_dq_kernel + bwd_dkdv_kernel + bwd_frozen_dv_kernel (whole backward)"},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def sizing_scan(B, T, steps, warmup):
    """The frozen-only sizing run of the closed-form scan (the HBM-bound
    frozen-head kernel): every head of (B, H=12, T, hd=64) bf16 frozen to a
    seeded mix of causal mean, exponential decay (rate ~U(0.001, 0.1)) and
    sliding window (w ~U{64..1024}); at B=8, T=16384 that is 96 sequences of
    V read once and Y written once (403 MB).  One step = one
    fused_mixed_attn call (the scan and its workspace clear).  Returns the
    step times, the scan kernel's roofline (HIP events right around the
    kernel) and the head kinds / parameters."""
    import torch
    import kernel

    H, hd = 12, 64
    g = torch.Generator().manual_seed(1337)
    v = torch.randn(B, H, T, hd, generator=g).bfloat16().cuda()
    kind = np.zeros(H, dtype=np.int32)
    param = np.zeros(H, dtype=np.float32)
    for h in range(H):
        k = int(torch.randint(0, 3, (1,), generator=g))
        if k == 0:
            kind[h] = kernel.CLOSED_MEAN
        elif k == 1:
            kind[h], param[h] = kernel.CLOSED_DECAY, 0.001 + 0.099 * float(torch.rand(1, generator=g))
        else:
            kind[h], param[h] = kernel.CLOSED_WINDOW, float(int(torch.randint(64, 1025, (1,), generator=g)))
    frozen = torch.full((H,), 2, dtype=torch.int32, device="cuda")
    step = lambda: kernel.fused_mixed_attn(None, None, v, None, frozen, closed_form=(kind, param),
                                           validate=False)
    with torch.inference_mode():
        step_ms, wall, summ = timed_steps(step, steps, warmup, True)
    _, extra = kernel_rooflines(summ, None, None, steps)
    scan = extra["frozen_scan"]
    if (B, T) == (8, 16384):
        scan["traffic"] = pmc_traffic("scan_kernel<bf16,64>", SCAN_TRAFFIC_FILE)
        scan["traffic_source"] = os.path.relpath(SCAN_TRAFFIC_FILE, REPO)
    scan["kernel"] = "scan_kernel<bf16,64>"
    del v
    return step_ms, scan, kind, param


def run_scan(args):
    """The frozen-only sizing run alone (see sizing_scan)."""
    B = args.batch or 8
    T = args.seq_len or 16384
    step_ms, scan, kind, param = sizing_scan(B, T, args.steps, args.warmup)
    nbytes = scan["bytes_per_launch"]
    total_ms = sum(step_ms)
    line = {
        "metric": "closed-form frozen-head scan throughput (1 GPU), HBM GB/s",
        "value": round(nbytes * args.steps / (total_ms / 1000.0) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (V ~ N(0, 1), seed 1337)",
        "config": {"workload": f"frozen-only sizing run: B={B}, H=12 all frozen (mean/decay/window), T={T}, "
                               f"hd=64; V read once + Y written once = {nbytes} bytes per step",
                   "kinds": [int(k) for k in kind], "params": [float(x) for x in param]},
        "roofline": scan,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def run_logz(args):
    """Freeze-time precompute: row normalisers z = logsumexp_{j<=i}(alpha_j +
    rho_{i-j}) of a C2 layer's decomposed buffers (H = 12, S = 16384, fp32),
    one step = one kernel.decomposed_logz call (saf_decomposed_logz).  Beside
    it, the reference's row-chunked torch definition on the same GPU and the
    float64 oracle on the host cores (H = 1, S = 4096 sample)."""
    import torch
    import kernel
    from kernel.fused_attn import decomp_logits

    H = 12
    S = args.seq_len or 16384
    g = torch.Generator().manual_seed(1337)
    alpha = (torch.randn(H, S, generator=g) * 0.5).cuda()
    rho = (-torch.rand(H, S, generator=g) * 0.01 * torch.arange(S)).cuda()
    step = lambda: kernel.decomposed_logz(alpha, rho)
    step_ms, wall, _ = timed_steps(step, args.steps, args.warmup, False)
    total_ms = sum(step_ms)
    logits = H * S * (S + 1) // 2
    rate = logits * args.steps / (total_ms / 1000.0)

    def torch_chunked():  # kernel/fused_attn.py:101-116 on device tensors
        chunk = max(1, (1 << 27) // (H * S))
        z = torch.empty_like(alpha)
        for r0 in range(0, S, chunk):
            r1 = min(r0 + chunk, S)
            z[:, r0:r1] = decomp_logits(alpha, rho, rows=(r0, r1)).logsumexp(-1)
        return z

    ref = torch_chunked()
    err = float((step() - ref).abs().max())
    t_ms, _, _ = timed_steps(torch_chunked, 2, 0, False)
    torch_ms = sum(t_ms) / len(t_ms)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import saf_oracle as orc
        Sc = min(S, 4096)
        a64 = alpha[:1, :Sc].double().cpu().numpy()
        r64 = rho[:1, :Sc].double().cpu().numpy()
        t0 = time.perf_counter()
        orc.decomposed_logz(a64, r64)
        dt = time.perf_counter() - t0
        cpu = {"value": round(Sc * (Sc + 1) / 2 / dt / 1e9, 4), "unit": "G logits/s", "cores": 1, "kind": "port",
               "sample": f"oracle decomposed_logz (numpy float64), H=1, S={Sc}, {dt:.2f} s"}
    peak = EXP_ISSUE_PEAK
    line = {
        "metric": "decomposed-pattern row normalisers (freeze-time precompute, 1 GPU), G logits/s",
        "value": round(rate / 1e9, 1), "unit": "G logits/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (alpha ~ N(0, 0.25), rho_d = -U(0, 0.01) d, seed 1337)",
        "config": {"workload": f"decomposed_logz of one C2 layer: H={H}, S={S} fp32, {logits} logits per step"},
        "roofline": {"bound": "exp", "achieved": round(rate / 1e9, 1), "peak": round(peak / 1e9, 1),
                     "unit": "G exp/s", "frac": round(rate / peak, 4), "traffic": None,
                     "kernel": "decomp_logz_kernel", "avg_launch_ms": round(total_ms / args.steps, 4)},
        "torch_chunked_gpu_ms": round(torch_ms, 3),
        "speedup_vs_torch_chunked": round(torch_ms / (total_ms / args.steps), 1),
        "max_abs_diff_vs_torch_chunked": err,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def build_ckpt_pair(dirpath, T, seed=1337):
    """A synthetic checkpoint pair in the reference's export layout at the
    124M shape (block_size T): the same random-init weights saved as a full
    model (no frozen head) and as a frozen model with a random 25% of the
    (layer, head) pairs frozen to learned-looking decomposed priors (alpha ~
    N(0, 0.5^2), rho_d = -c d + N(0, 0.1^2) with c ~U(0.001, 0.05)), which are
    no closed form and run the decomposed P.V kernel (beside the live heads).
    Written on the CPU; returns (baseline path, frozen path)."""
    import torch
    from nanogpt.model import GPT, GPTConfig
    from nanogpt.checkpoint import save_reference_checkpoint

    torch.manual_seed(seed)
    cfg = GPTConfig(block_size=T, vocab_size=50304, n_layer=12, n_head=12, n_embd=768, bias=False,
                    position_encoding="rope", rand_attn_prior_repr="decomposed", rand_seed=seed)
    model = GPT(cfg).eval()
    base = os.path.join(dirpath, "saf124m_full.pt")
    save_reference_checkpoint(model, base, iter_num=0)
    g = torch.Generator().manual_seed(seed)
    pairs = torch.randperm(144, generator=g)[:36].tolist()
    d = torch.arange(T, dtype=torch.float32)
    per_layer = {}
    for idx in pairs:
        per_layer.setdefault(idx // 12, []).append(idx % 12)
    for layer, heads in per_layer.items():
        n = len(heads)
        alpha = torch.randn(n, T, generator=g) * 0.5
        c = 0.001 + 0.049 * torch.rand(n, 1, generator=g)
        rho = -c * d + torch.randn(n, T, generator=g) * 0.1
        model.transformer.h[layer].attn.freeze_heads_decomposed(heads, alpha, rho)
    frozen = os.path.join(dirpath, "saf124m_saf25.pt")
    save_reference_checkpoint(model, frozen, iter_num=0)
    return base, frozen


def ckpt_leg(spec):
    """One timing leg of a loaded export (nanogpt/bench_checkpoint_prefill.py:35-153):
    load, verify one fused dispatch per layer, warm up, optionally capture
    one prefill in a HIP graph, time `iters` prefills (HIP events), median."""
    import torch
    from nanogpt import model as model_mod
    from nanogpt.checkpoint import load_model

    model, cfg, ck = load_model(spec["ckpt"], "cuda", torch.bfloat16)
    del ck
    if spec["T"] > cfg.block_size:
        raise ValueError(f"T={spec['T']} exceeds the checkpoint's block_size {cfg.block_size}")
    frozen = sum(int(b.attn.dyn_frozen.sum()) for b in model.transformer.h)
    x = torch.randint(0, cfg.vocab_size, (spec["B"], spec["T"]),
                      generator=torch.Generator().manual_seed(spec["seed"] + 1)).cuda()
    with torch.inference_mode():
        n0 = model_mod.fused_dispatch_count()
        model(x)
        torch.cuda.synchronize()
        calls = model_mod.fused_dispatch_count() - n0
        if calls != cfg.n_layer:
            raise RuntimeError(f"expected {cfg.n_layer} fused dispatches, observed {calls}")
        for _ in range(spec["warmup"]):
            model(x)
        torch.cuda.synchronize()
        step = lambda: model(x)
        capture_ms = None
        if spec["graph"]:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    model(x)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            with torch.cuda.graph(graph):
                out = model(x)
            e1.record()
            torch.cuda.synchronize()
            capture_ms = e0.elapsed_time(e1)
            eager = model(x)
            graph.replay()
            torch.cuda.synchronize()
            a, b = out.double().flatten(), eager.double().flatten()
            cos = float(a @ b / (a.norm() * b.norm()))
            if cos < 0.9999:
                raise RuntimeError(f"graph replay differs from the eager prefill (cosine {cos:.6f})")
            step = graph.replay
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(spec["iters"])]
        for a, b in ev:
            a.record()
            step()
            b.record()
        torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in ev]
    med = statistics.median(ms)
    return {"variant": spec["variant"], "ckpt": os.path.basename(spec["ckpt"]), "frozen_heads": frozen,
            "median_ms": round(med, 4), "p10_ms": round(sorted(ms)[len(ms) // 10], 4),
            "p90_ms": round(sorted(ms)[(9 * len(ms)) // 10], 4),
            "tokens_per_s": round(spec["B"] * spec["T"] / (med / 1000.0), 1),
            "execution": "hip_graph" if spec["graph"] else "eager",
            "graph_capture_ms": None if capture_ms is None else round(capture_ms, 2)}


def _ckpt_leg_child(spec, conn):
    try:
        conn.send(ckpt_leg(spec))
    except Exception as e:  # reported by the parent
        conn.send({"error": f"{type(e).__name__}: {e}"})
    conn.close()


def run_ckpt(args):
    """Prefill of a loaded checkpoint pair (nanogpt/bench_checkpoint_prefill.py):
    the frozen export through the fused path against its full (all-live)
    export, B x T square causal prefill, optional HIP graph replay
    (--graph), and with --isolate every leg in a fresh spawned process in
    ABBA order per repeat.  Without --ckpt a synthetic pair is written
    (build_ckpt_pair)."""
    import multiprocessing as mp
    import tempfile

    T = args.seq_len or 4096
    B = args.batch or 8
    tmp = None
    if args.ckpt:
        base, frozen = args.ckpt_baseline, args.ckpt
    else:
        tmp = tempfile.mkdtemp(prefix="saf_ckpt_")
        log(f"writing a synthetic checkpoint pair (T={T}) to {tmp}")
        base, frozen = build_ckpt_pair(tmp, T)
    legs = []
    for r in range(args.repeats):
        order = [("baseline", base), ("frozen", frozen)]
        order = order + order[::-1] if args.isolate else order
        for variant, path in order:
            if path is None:
                continue
            legs.append({"variant": variant, "ckpt": path, "T": T, "B": B, "seed": 1337 + r,
                         "warmup": args.warmup, "iters": args.steps, "graph": args.graph, "repeat": r})
    results = []
    for spec in legs:
        if args.isolate:
            ctx = mp.get_context("spawn")
            parent, child = ctx.Pipe()
            proc = ctx.Process(target=_ckpt_leg_child, args=(spec, child))
            proc.start()
            res = parent.recv()
            proc.join()
            if "error" in res:
                raise RuntimeError(f"leg {spec['variant']} failed: {res['error']}")
        else:
            res = ckpt_leg(spec)
        res["repeat"] = spec["repeat"]
        log(f"{res['variant']}: {res['median_ms']:.3f} ms ({res['tokens_per_s']:.0f} tokens/s)")
        results.append(res)
    if tmp is not None:
        for f in os.listdir(tmp):
            os.remove(os.path.join(tmp, f))
        os.rmdir(tmp)
    med = lambda v: statistics.median(x["median_ms"] for x in results if x["variant"] == v)
    f_ms = med("frozen")
    line = {
        "metric": "prefill tokens/sec of a loaded SAF checkpoint (1 GPU)",
        "value": round(B * T / (f_ms / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(f_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic tokens; " + ("checkpoint files given" if args.ckpt else
                                        "synthetic export pair in the reference layout (seed 1337)"),
        "config": {"workload": f"checkpoint prefill: B={B}, T={T}, "
                               + ("isolated ABBA legs" if args.isolate else "in-process legs")
                               + (", HIP graph replay" if args.graph else ", eager"),
                   "frozen_ckpt": os.path.basename(frozen),
                   "baseline_ckpt": None if base is None else os.path.basename(base)},
        "roofline": None,
        "cpu_baseline": None,
        "legs": results,
    }
    if base is not None:
        b_ms = med("baseline")
        line["baseline_tokens_per_s"] = round(B * T / (b_ms / 1000.0), 1)
        line["speedup_vs_full"] = round(b_ms / f_ms, 4)
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["c1", "c2", "c3", "c4", "scan", "bwd", "logz", "ckpt"], default="c2",
                    help="c1: the isolated op (decay heads as scan / rebuild / dense); "
                         "c2: 124M nanoGPT SAF-25%% at 16K (the headline); c3: 1B-class with dense "
                         "frozen patterns; c4: Qwen-style GQA; "
                         "scan: frozen-only sizing run of the closed-form scan (HBM roofline); "
                         "bwd: the C1 op forward + backward; logz: freeze-time row normalisers; "
                         "ckpt: prefill of a loaded checkpoint pair")
    ap.add_argument("--ckpt", default=None, help="ckpt: frozen export (default: a synthetic pair)")
    ap.add_argument("--ckpt-baseline", default=None, help="ckpt: the matching full export")
    ap.add_argument("--graph", action="store_true", help="ckpt: time HIP graph replays of the prefill")
    ap.add_argument("--isolate", action="store_true",
                    help="ckpt: every leg in a fresh spawned process, ABBA order per repeat")
    ap.add_argument("--repeats", type=int, default=1, help="ckpt: repeats of the leg order")
    ap.add_argument("--seq-len", type=int, default=None)
    ap.add_argument("--batch", type=int, default=None, help="c1 / c4 / scan / ckpt batch (defaults 8 / 4 / 8 / 8)")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--rate", type=float, default=0.25, help="c4: frozen fraction of query heads")
    ap.add_argument("--c1-legs", default=None,
                    help="c1: comma list of legs to run (scan, decomp, dense, decomp_split, decomp_alone); "
                         "default all, the scan leg always")
    ap.add_argument("--prior-repr", choices=["decomposed", "dense"], default="decomposed",
                    help="c4: causal-mean prior as alpha = rho = 0 (scan) or a dense (T, T) pattern")
    ap.add_argument("--sdpa-live", action="store_true",
                    help="c4 at rate 0: leave the model unconverted (torch SDPA) instead of the HIP flash path")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sizing-scan", action="store_true",
                    help="c2: skip the in-process frozen-only sizing scan (frozen_roofline)")
    ap.add_argument("--cpu-layers", type=int, default=None)
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

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)
        return
    if args.workload == "scan":
        run_scan(args)
        return
    if args.workload == "ckpt":
        run_ckpt(args)
        return
    if args.workload == "bwd":
        run_bwd(args)
        return
    if args.workload == "logz":
        run_logz(args)
        return
    if args.workload == "c3":
        run_c3(args)
        return
    if args.workload == "c1":
        run_c1(args)
        return
    if args.workload == "c4":
        if args.cpu_layers is None:
            args.cpu_layers = 1
        run_c4(args)
    else:
        if args.layers is None:
            args.layers = 12
        if args.cpu_layers is None:
            args.cpu_layers = 1
        run_c2(args)


if __name__ == "__main__":
    main()
