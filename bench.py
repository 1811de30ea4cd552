"""Benchmark: one transformer-layer forward on one MI355X.

Prints ONE JSON line on stdout. A "step" is one layer forward
(OptimizedTransformer with num_layers=1, the reference's layer + final norm)
over one synthetic batch already resident in HBM.

Workload: BASELINE config 1 (the padded batch: B=8, S=512, d_model=512,
8 heads, d_ff=2048, key-padding mask), Xavier weights from the fixed seed.
`--config C1..C5` selects another config; `--all` adds a per-config table on
stderr.

Reported beside the layer time:
  roofline      the dominant kernel of the layer, timed alone with HIP events
                on the stream it launches on (torch's current stream), its
                algorithmic flops (or bytes) per launch over its average
                duration, against MI355X's published peak (dense fp16 MFMA
                2.5 PFLOP/s; HBM 8 TB/s);
  kernels       the same figures for every kernel of the layer;
  cpu_baseline  the reference layer (the repository's CPU oracle, fp32) timed
                on this machine's host cores on the same inputs.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(REPO, "distraction-optimizedtransformerlayer_amd")
for _p in (REPO, PKG_ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_MFMA_TFLOPS = 2500.0   # dense fp16/bf16
PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5"])
    p.add_argument("--all", action="store_true", help="also time every config (stderr table)")
    p.add_argument("--cpu-budget", type=float, default=20.0,
                   help="seconds of CPU-oracle timing for the baseline")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--graph", default="auto", choices=["auto", "off", "always"])
    return p.parse_args()


def sync():
    import torch

    torch.cuda.synchronize()


def time_layer(model, x, mask, steps, warmup):
    """Average ms per forward over `steps`, bracketed by synchronize."""
    import torch

    with torch.inference_mode():
        for _ in range(warmup):
            model(x, mask)
        sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            model(x, mask)
        sync()
        t1 = time.perf_counter()
    return (t1 - t0) * 1000.0 / steps


def device_us(fn, reps, replays=5):
    """Device time of one call of `fn`, in microseconds.

    `reps` back-to-back calls are captured into one hipGraph and the graph is
    replayed between two HIP events on the capture stream, so host launch
    overhead (Python, ctypes) does not pad short kernels.
    """
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    start.record(stream)
    for _ in range(replays):
        g.replay()
    end.record(stream)
    end.synchronize()
    us = start.elapsed_time(end) * 1000.0 / (reps * replays)
    g.reset()
    return us


def kernel_table(cfg, model, x, mask, reps):
    """Time each kernel of the layer alone (HIP events on the launch stream).

    Returns name -> dict(us, flops or bytes, achieved, unit, frac, bound).
    """
    import torch

    import kernel_ext
    from oracle.inputs import attention_useful_flops, lengths_of

    kx = kernel_ext.get_kernels()
    B, S, D, F, H = cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.ffn_dim, cfg.num_heads
    hd = D // H
    T = B * S
    layer = model.layers[0]
    attn = layer.attention
    dev = x.device
    mask_np = None if mask is None else mask.cpu().numpy()
    L = lengths_of(mask_np, cfg, B)

    with torch.inference_mode():
        x2 = x.reshape(T, D)
        planes = kx.fused_layernorm_split(x2, layer.norm1.weight, layer.norm1.bias)
        qkv_w, qkv_b = attn._get_qkv_weight()
        qkv = kx.linear_bias_split(planes, qkv_w, qkv_b, -1, True)
        q, k, v = qkv.view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4).unbind(0)
        amask = None if mask is None else mask[:, None, None, :]
        ctx = kx.fused_attention_forward(q, k, v, amask, cfg.causal, hd ** -0.5, 0, 1, 0)
        ctx2 = ctx.reshape(T, D)
        attn_out = kx.linear_bias(ctx2, attn.out_proj.weight, attn.out_proj.bias)
        _, n2 = kx.fused_add_layernorm(x2, attn_out, layer.norm2.weight, layer.norm2.bias,
                                       1e-5, True)
        hidden = kx.linear_gelu(n2, layer.ffn_in.weight, layer.ffn_in.bias, -1, -1, True)
        ffn = kx.linear_bias(hidden, layer.ffn_out.weight, layer.ffn_out.bias)

        ops = {
            "layernorm (norm1, split-fp16 out)": (
                lambda: kx.fused_layernorm_split(x2, layer.norm1.weight, layer.norm1.bias),
                "hbm", T * D * 8.0),
            "linear qkv (fp16x3, fp16 out)": (
                lambda: kx.linear_bias_split(planes, qkv_w, qkv_b, -1, True),
                "mfma", 2.0 * T * D * 3 * D),
            "attention": (
                lambda: kx.fused_attention_forward(q, k, v, amask, cfg.causal, hd ** -0.5, 0, 1, 0),
                "mfma", attention_useful_flops(cfg, L)),
            "linear out_proj": (
                lambda: kx.linear_bias(ctx2, attn.out_proj.weight, attn.out_proj.bias),
                "mfma", 2.0 * T * D * D),
            "add+layernorm (norm2, fp16 out)": (
                lambda: kx.fused_add_layernorm(x2, attn_out, layer.norm2.weight,
                                               layer.norm2.bias, 1e-5, True),
                "hbm", T * D * 14.0),
            "linear_gelu ffn_in (fp16 out)": (
                lambda: kx.linear_gelu(n2, layer.ffn_in.weight, layer.ffn_in.bias, -1, -1, True),
                "mfma", 2.0 * T * D * F),
            "linear ffn_out": (
                lambda: kx.linear_bias(hidden, layer.ffn_out.weight, layer.ffn_out.bias),
                "mfma", 2.0 * T * F * D),
            "add+layernorm (final, fp32 out)": (
                lambda: kx.fused_add_layernorm(x2, ffn, model.final_norm.weight,
                                               model.final_norm.bias, 1e-5, False),
                "hbm", T * D * 16.0),
        }
        out = {}
        for name, (fn, bound, work) in ops.items():
            us = device_us(fn, reps)
            if bound == "mfma":
                achieved = work / (us * 1e-6) / 1e12
                out[name] = dict(us=us, flops=work, bound="mfma", achieved=achieved,
                                 unit="TFLOP/s", peak=PEAK_MFMA_TFLOPS,
                                 frac=achieved / PEAK_MFMA_TFLOPS)
            else:
                achieved = work / (us * 1e-6) / 1e9
                out[name] = dict(us=us, bytes=work, bound="hbm", achieved=achieved,
                                 unit="GB/s", peak=PEAK_HBM_GBS, frac=achieved / PEAK_HBM_GBS)
    return out


def cpu_baseline(cfg, x_np, mask_np, params, budget_s):
    """The reference layer (the CPU oracle) timed on this host's cores."""
    import torch

    from oracle.layer import reference_layer

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    reference_layer(x_np, mask_np, params, cfg)  # warmup
    first = time.perf_counter() - t0
    n = max(1, min(10, int(budget_s / max(first, 1e-3))))
    samples = []
    for _ in range(n):
        t = time.perf_counter()
        reference_layer(x_np, mask_np, params, cfg)
        samples.append(time.perf_counter() - t)
    med = statistics.median(samples)
    model_name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": med * 1e6, "unit": "us/layer-fwd", "cores": threads, "kind": "port",
            "sample": f"full {cfg.name} layer forward (fp32 torch CPU oracle), median of {n} "
                      f"after 1 warmup; cpu={model_name}; torch={torch.__version__}"}


def run_config(name, steps, warmup, graph, with_kernels=True):
    import torch

    from layer_runner import TransformerConfig, build_model, to_device
    from optimized import config as ocfg
    from oracle.inputs import CONFIGS, gemm_flops, attention_useful_flops, lengths_of, make_case

    cfg = CONFIGS[name]
    x_np, mask_np, params = make_case(cfg)
    tcfg = TransformerConfig(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads,
                             cfg.ffn_dim, 1, cfg.causal)
    ocfg.CUDA_GRAPH = graph
    model = build_model(tcfg, params)
    x, mask = to_device(x_np, mask_np)
    ms = time_layer(model, x, mask, steps, warmup)
    ocfg.CUDA_GRAPH = "off"
    ms_eager = time_layer(model, x, mask, max(5, steps // 2), 2)
    ocfg.CUDA_GRAPH = graph
    L = lengths_of(mask_np, cfg, cfg.batch_size)
    flops = gemm_flops(cfg) + attention_useful_flops(cfg, L)
    res = dict(config=cfg, model=model, x=x, mask=mask, x_np=x_np, mask_np=mask_np,
               params=params, ms=ms, ms_eager=ms_eager, flops=flops,
               graphs=len(model._graphs))
    if with_kernels:
        res["kernels"] = kernel_table(cfg, model, x, mask, 20)
    return res


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (--gpus {args.gpus} "
              f"was asked for). The layer shards by batch with no exchange; see DESIGN.md.",
              file=sys.stderr)
        return 2
    import torch

    import kernel_ext

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    if kernel_ext.get_kernels() is None:
        raise RuntimeError(f"libdotl_hip.so did not load: {kernel_ext.load_error()}")

    log(f"[bench] device={torch.cuda.get_device_name(0)} config={args.config} "
        f"steps={args.steps} warmup={args.warmup} graph={args.graph}")
    r = run_config(args.config, args.steps, args.warmup, args.graph)
    cfg = r["config"]
    us = r["ms"] * 1000.0
    kt = r["kernels"]
    for kname, k in kt.items():
        log(f"[bench]   {kname:34s} {k['us']:9.2f} us  {k['achieved']:9.1f} {k['unit']:8s} "
            f"({100 * k['frac']:.1f}% of {k['peak']:.0f})")
    dom_name = max(kt, key=lambda n: kt[n]["us"])
    dom = kt[dom_name]
    attn = kt["attention"]
    ln = kt["add+layernorm (final, fp32 out)"]

    cpu = None
    if not args.no_cpu:
        log("[bench] timing the CPU oracle baseline ...")
        cpu = cpu_baseline(cfg, r["x_np"], r["mask_np"], r["params"], args.cpu_budget)
        log(f"[bench] cpu baseline {cpu['value']:.0f} us on {cpu['cores']} threads")

    line = {
        "metric": "layer fwd µs/geomean speedup vs CPU ref; attn MFMA util %, LN HBM GB/s",
        "value": round(us, 2),
        "unit": "us/layer-fwd",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 I/O; fp16 MFMA operands, fp32 accumulate (QKV: split fp16x3)",
        "data": "synthetic (seeded Xavier weights, N(0,1) x, key-padding lengths)",
        "config": {"workload": f"{cfg.name}: single-layer forward B={cfg.batch_size} "
                               f"S={cfg.seq_len} d_model={cfg.d_model} heads={cfg.num_heads} "
                               f"d_ff={cfg.ffn_dim} mask={cfg.mask} causal={cfg.causal}",
                   "graph": args.graph, "graph_captured": r["graphs"] > 0},
        "eager_us": round(r["ms_eager"] * 1000.0, 2),
        "tokens_per_s": round(cfg.tokens / (r["ms"] * 1e-3), 1),
        "layer_tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 2),
        "roofline": {"bound": dom["bound"], "kernel": dom_name,
                     "achieved": round(dom["achieved"], 2), "peak": dom["peak"],
                     "unit": dom["unit"], "frac": round(dom["frac"], 4), "traffic": None},
        "attn_mfma_util_pct": round(100 * attn["frac"], 2),
        "ln_hbm_gbs": round(ln["achieved"], 1),
        "kernels": {k: {"us": round(v["us"], 2), "achieved": round(v["achieved"], 2),
                        "unit": v["unit"], "frac": round(v["frac"], 4)} for k, v in kt.items()},
        "cpu_baseline": cpu,
        "speedup_vs_cpu": (round(cpu["value"] / us, 1) if cpu else None),
    }
    print(json.dumps(line), flush=True)

    if args.all:
        log("[bench] per-config table (graph replay / eager us, layer TFLOP/s)")
        for name in ["C1", "C2", "C3", "C4", "C5"]:
            rr = run_config(name, max(5, args.steps // 2), 3, args.graph, with_kernels=True)
            k = rr["kernels"]
            log(f"[bench] {name}: {rr['ms'] * 1000:.1f} us (eager {rr['ms_eager'] * 1000:.1f}) "
                f"layer {rr['flops'] / (rr['ms'] * 1e-3) / 1e12:.1f} TFLOP/s, attention "
                f"{100 * k['attention']['frac']:.1f}% MFMA, final add+LN "
                f"{k['add+layernorm (final, fp32 out)']['achieved']:.0f} GB/s")
            del rr
            torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
