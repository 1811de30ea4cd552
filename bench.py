"""Benchmark: one transformer-layer forward on one MI355X.

Prints ONE JSON line on stdout. A "step" is one layer forward
(OptimizedTransformer with num_layers=1, the reference's layer + final norm)
over one synthetic batch already resident in HBM.

Workload: BASELINE config 3 (C4, the largest: B=4, S=2048, d_model=2048,
16 heads of 128, d_ff=8192, no mask), Xavier weights from the fixed seed.
`--config C1..C5` selects another config. Unless --quick, the line also carries
a per-config table (C1..C5: layer µs, CPU-oracle µs, speedup, attention MFMA
utilisation, final add+LN GB/s) and the geomean speedup over the five
configs, the metric's second figure.

Reported beside the layer time:
  roofline      the dominant kernel of the layer, timed alone with HIP events
                on the stream it launches on (torch's current stream), its
                algorithmic flops (or bytes) per launch over its average
                duration, against MI355X's published peak (dense fp16 MFMA
                2.5 PFLOP/s; HBM 8 TB/s);
                The MFMA-bound entry also carries the rate measured live on
                this device by the library's register-only MFMA probe on
                random operands (mfma_ceiling): the matrix cores' power draw
                drops the clock under real data, so that rate (~60% of the
                datasheet figure on MI355X) is the practical roof;
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
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="C4", choices=["C1", "C2", "C3", "C4", "C5"])
    p.add_argument("--quick", action="store_true",
                   help="skip the per-config table (C1..C5 layer µs and CPU speedups)")
    p.add_argument("--cpu-budget", type=float, default=20.0,
                   help="seconds of CPU-oracle timing for the baseline")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--graph", default="auto", choices=["auto", "off", "always"])
    p.add_argument("--traffic", default="pmc", choices=["pmc", "off"],
                   help="HBM bytes of the dominant kernel from two rocprofv3 --pmc child runs")
    p.add_argument("--profile-ops", default=None, metavar="OP",
                   help="(child mode for --pmc) run one op of the layer and the copy, then exit")
    return p.parse_args()


def sync():
    import torch

    torch.cuda.synchronize()


SAMPLE_STEPS = 20   # forwards per HIP-event sample
MAX_SAMPLES = 5


def time_layer(model, x, mask, steps, warmup):
    """Time exactly `steps` forwards after `warmup` untimed ones.

    The timed region is bracketed by synchronize on both sides (its wall
    time gives `wall_ms`). Inside it, HIP events on the launch stream split
    the steps into up to MAX_SAMPLES samples of at least SAMPLE_STEPS
    forwards each (fewer when `steps` is short), as the reference times a
    forward with one event pair (torch_transformer_benchmark.py:859-872);
    the figure reported is the median sample's device time per forward.
    Returns dict(median_ms, samples_ms, wall_ms, steps_per_sample).
    """
    import torch

    n_samples = max(1, min(MAX_SAMPLES, steps // SAMPLE_STEPS))
    per = steps // n_samples
    bounds = [per * i for i in range(n_samples)] + [steps]
    with torch.inference_mode():
        for _ in range(warmup):
            model(x, mask)
        sync()
        stream = torch.cuda.current_stream()
        events = [torch.cuda.Event(enable_timing=True) for _ in bounds]
        t0 = time.perf_counter()
        events[0].record(stream)
        for i in range(n_samples):
            for _ in range(bounds[i + 1] - bounds[i]):
                model(x, mask)
            events[i + 1].record(stream)
        sync()
        t1 = time.perf_counter()
    samples = [events[i].elapsed_time(events[i + 1]) / (bounds[i + 1] - bounds[i])
               for i in range(n_samples)]
    return dict(median_ms=statistics.median(samples), samples_ms=samples,
                wall_ms=(t1 - t0) * 1000.0 / steps, steps_per_sample=per)


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


def layer_ops(cfg, model, x, mask):
    """Every kernel launch of one layer forward, as separately callable ops.

    Follows the path the model takes: on a padded batch with row packing on
    (the default), the first LayerNorm gathers the T_valid valid rows, the
    GEMMs and attention run on them, and the final add+LayerNorm scatters
    back to B*S rows. Returns name -> (fn, bound, algorithmic work per call,
    compulsory HBM bytes per call): work is flops for the MFMA kernels, HBM
    bytes for the LayerNorms. The intermediate tensors the ops read are
    produced once here, by the same kernels.
    """
    import torch

    import kernel_ext
    from optimized import config as ocfg
    from oracle.inputs import attention_useful_flops, lengths_of

    kx = kernel_ext.get_kernels()
    B, S, D, F, H = cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.ffn_dim, cfg.num_heads
    hd = D // H
    T = B * S
    layer = model.layers[0]
    attn = layer.attention
    mask_np = None if mask is None else mask.cpu().numpy()
    L = lengths_of(mask_np, cfg, B)
    packing = model._mask_packing(mask) if mask is not None else None
    if packing is not None and (packing.trivial or ocfg.ROW_PACKING == "off"):
        packing = None
    R = packing.t_valid if packing is not None else T   # rows the GEMMs see
    scale = hd ** -0.5
    fw, fb = model.final_norm.weight, model.final_norm.bias

    from optimized import kernels as okernels

    # The QKV arithmetic the model resolves for this input (config.QKV_PRECISION
    # "auto": split planes where some row attends to few keys, else one pass).
    okernels._qkv_few_keys = model._few_key_rows(x, model._mask_packing(mask))
    qkv_prec = okernels._qkv_precision()
    split = qkv_prec in ("fp16x2", "fp16x3")
    split_w = qkv_prec == "fp16x3"
    kind = "split" if split else "half"
    with torch.inference_mode():
        if packing is not None:
            ln1 = lambda: kx.fused_layernorm_rows(x, layer.norm1.weight, layer.norm1.bias,  # noqa: E731
                                                  packing.idx, 1e-5, kind, True)
            x2, planes = ln1()
            # read x, write the gathered x and the planes (or fp16 normed)
            ln1_bytes = R * D * (12.0 if split else 10.0)
        else:
            x2 = x.reshape(T, D)
            if split:
                ln1 = lambda: kx.fused_layernorm_split(x2, layer.norm1.weight, layer.norm1.bias)  # noqa: E731
            else:
                ln1 = lambda: kx.fused_layernorm(x2, layer.norm1.weight, layer.norm1.bias, 1e-5,  # noqa: E731
                                                 True)
            planes = ln1()
            ln1_bytes = T * D * (8.0 if split else 6.0)
        qkv_w, qkv_b = attn._get_qkv_weight()
        # an unpadded causal batch keeps the split planes for each sequence's
        # first rows only (model._split_prefix); the op is then the one-pass
        # GEMM, the prefix's split GEMM and their two copies
        prefix = model._split_prefix(x, model._mask_packing(mask)) if split else 0
        if prefix:
            planes4 = planes.view(2, B, S, D)
            qkv_fn = lambda: okernels._linear_bias_split_prefix(  # noqa: E731
                planes4, qkv_w, qkv_b, True, prefix).view(T, 3 * D)
            qkv_prec = f"fp16; {qkv_prec} on each sequence's first {prefix} rows"
        elif split:
            qkv_fn = lambda: kx.linear_bias_split(planes, qkv_w, qkv_b, -1, True,  # noqa: E731
                                                  split_weight=split_w)
        else:
            qkv_fn = lambda: kx.linear_bias(planes, qkv_w, qkv_b, -1, -1, True)  # noqa: E731
        qkv = qkv_fn()
        if packing is not None:
            q, k, v = qkv.view(R, 3, H, hd).unbind(1)
            attn_fn = lambda: kx.fused_attention_forward(q, k, v, None, cfg.causal, scale, 0, 1, 0,  # noqa: E731
                                                         cu_seqlens=packing.cu, max_seqlen=S)
            amask = None
        else:
            q, k, v = qkv.view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4).unbind(0)
            amask = None if mask is None else mask[:, None, None, :]
            attn_fn = lambda: kx.fused_attention_forward(q, k, v, amask, cfg.causal, scale,  # noqa: E731
                                                         0, 1, 0)
        ctx = attn_fn()
        ctx2 = ctx.reshape(R, D)
        # The model's choice: residual adds in out_proj's and ffn_out's
        # epilogues and plain LayerNorms after them, or add+LayerNorm kernels.
        resid = layer._residual_fused(x2)
        # rows narrow enough (and many enough) for the LayerNorms in the
        # out_proj / ffn_out epilogues (optimized.kernels._linear_norm)
        ln_epi = resid and okernels._ln_epilogue_wanted(R, D)
        if resid:
            attn_out = kx.linear_bias(ctx2, attn.out_proj.weight, attn.out_proj.bias, residual=x2)
            h1 = attn_out
            n2 = kx.fused_layernorm(h1, layer.norm2.weight, layer.norm2.bias, 1e-5, True)
        else:
            attn_out = kx.linear_bias(ctx2, attn.out_proj.weight, attn.out_proj.bias)
            h1, n2 = kx.fused_add_layernorm(x2, attn_out, layer.norm2.weight, layer.norm2.bias,
                                            1e-5, True)
        hidden = kx.linear_gelu(n2, layer.ffn_in.weight, layer.ffn_in.bias, -1, -1, True)
        ffn = kx.linear_bias(hidden, layer.ffn_out.weight, layer.ffn_out.bias,
                             residual=h1 if resid else None)
        if packing is not None and resid:
            final = lambda: kx.fused_layernorm_rows(ffn, fw, fb, packing.inv, 1e-5, "float", False)  # noqa: E731
            final_bytes = R * D * 4.0 + T * D * 4.0   # read the packed rows, write B*S rows
        elif packing is not None:
            final = lambda: kx.fused_add_layernorm_rows(h1, ffn, fw, fb, packing.inv, 1e-5)  # noqa: E731
            final_bytes = R * D * 8.0 + T * D * 4.0   # read two packed inputs, write B*S rows
        elif resid:
            final = lambda: kx.fused_layernorm(ffn, fw, fb, 1e-5, False)  # noqa: E731
            final_bytes = T * D * 8.0
        else:
            final = lambda: kx.fused_add_layernorm(x2, ffn, fw, fb, 1e-5, False)  # noqa: E731
            final_bytes = T * D * 16.0

    def nb(*ts):
        return float(sum(t.numel() * t.element_size() for t in ts if t is not None))

    # Compulsory HBM bytes per call: every operand read once, every output
    # written once (the fp16 weight copies the GEMMs read; the split QKV
    # weight is two fp16 planes).
    wq16 = 2.0 * (2 if split_w else 1) * qkv_w.numel()   # fp16 hi (+ lo) planes of W
    w16 = lambda lin: 2.0 * lin.weight.numel() + nb(lin.bias)  # noqa: E731
    cu_bytes = nb(packing.cu) if packing is not None else nb(mask)
    ops = {
        f"layernorm (norm1, {'split-fp16' if split else 'fp16'} out)": (
            ln1, "hbm", ln1_bytes, ln1_bytes),
        f"linear qkv ({qkv_prec}, fp16 out)": (
            qkv_fn, "mfma", 2.0 * R * D * 3 * D, nb(planes, qkv_b, qkv) + wq16),
        "attention": (attn_fn, "mfma", attention_useful_flops(cfg, L), nb(qkv, ctx) + cu_bytes),
    }
    if ln_epi:
        # out_proj + residual + norm2, ffn_out + residual + the final norm,
        # each one GEMM (the final one scattering to the padded rows, whose
        # zeros a second kernel writes)
        def final_fused():
            if packing is not None:
                _, out = kx.linear_layernorm(hidden, layer.ffn_out.weight, layer.ffn_out.bias, h1,
                                             fw, fb, 1e-5, "float", store_out=False,
                                             out_row=packing.idx, normed_rows=T)
                kx.zero_rows(out, packing.inv)
                return out
            return kx.linear_layernorm(hidden, layer.ffn_out.weight, layer.ffn_out.bias, h1, fw,
                                       fb, 1e-5, "float", store_out=False)[1]
        ops["linear out_proj (+ residual, + norm2 fp16 out)"] = (
            lambda: kx.linear_layernorm(ctx2, attn.out_proj.weight, attn.out_proj.bias, x2,
                                        layer.norm2.weight, layer.norm2.bias, 1e-5, "half"),
            "mfma", 2.0 * R * D * D, nb(ctx2, x2, h1, n2) + w16(attn.out_proj))
        if okernels._ffn_ln_wanted(n2, layer.ffn_in, layer.ffn_out):
            # the whole FFN with the residual add and the final norm, one
            # kernel (optimized.kernels._ffn_norm)
            def ffn_fused():
                if packing is not None:
                    return kx.ffn_layernorm(n2, layer.ffn_in.weight, layer.ffn_in.bias,
                                            layer.ffn_out.weight, layer.ffn_out.bias, h1, fw, fb,
                                            1e-5, "float", out_row=packing.idx, normed_rows=T,
                                            zero_padded=True)[1]
                return kx.ffn_layernorm(n2, layer.ffn_in.weight, layer.ffn_in.bias,
                                        layer.ffn_out.weight, layer.ffn_out.bias, h1, fw, fb,
                                        1e-5, "float")[1]
            ops["ffn (ffn_in, GELU, ffn_out, + residual, + final norm fp32 out)"] = (
                ffn_fused, "mfma", 4.0 * R * D * F,
                nb(n2, h1) + T * D * 4.0 + w16(layer.ffn_in) + w16(layer.ffn_out))
            return ops
        ops.update({
            "linear_gelu ffn_in (fp16 out)": (
                lambda: kx.linear_gelu(n2, layer.ffn_in.weight, layer.ffn_in.bias, -1, -1, True),
                "mfma", 2.0 * R * D * F, nb(n2, hidden) + w16(layer.ffn_in)),
            "linear ffn_out (+ residual, + final norm fp32 out)": (
                final_fused, "mfma", 2.0 * R * F * D,
                nb(hidden, h1) + T * D * 4.0 + w16(layer.ffn_out)),
        })
        return ops
    ops.update({
        "linear out_proj" + (" (+ residual)" if resid else ""): (
            lambda: kx.linear_bias(ctx2, attn.out_proj.weight, attn.out_proj.bias,
                                   residual=x2 if resid else None),
            "mfma", 2.0 * R * D * D,
            nb(ctx2, attn_out, x2 if resid else None) + w16(attn.out_proj)),
        ("layernorm (norm2, fp16 out)" if resid else "add+layernorm (norm2, fp16 out)"): (
            (lambda: kx.fused_layernorm(h1, layer.norm2.weight, layer.norm2.bias, 1e-5, True))
            if resid else
            (lambda: kx.fused_add_layernorm(x2, attn_out, layer.norm2.weight,
                                            layer.norm2.bias, 1e-5, True)),
            "hbm", R * D * (6.0 if resid else 14.0), R * D * (6.0 if resid else 14.0)),
        "linear_gelu ffn_in (fp16 out)": (
            lambda: kx.linear_gelu(n2, layer.ffn_in.weight, layer.ffn_in.bias, -1, -1, True),
            "mfma", 2.0 * R * D * F, nb(n2, hidden) + w16(layer.ffn_in)),
        "linear ffn_out" + (" (+ residual)" if resid else ""): (
            lambda: kx.linear_bias(hidden, layer.ffn_out.weight, layer.ffn_out.bias,
                                   residual=h1 if resid else None),
            "mfma", 2.0 * R * F * D, nb(hidden, ffn, h1 if resid else None) + w16(layer.ffn_out)),
        ("layernorm (final, fp32 out)" if resid else "add+layernorm (final, fp32 out)"): (
            final, "hbm", final_bytes, final_bytes),
    })
    return ops


def final_ln(kt):
    """The per-kernel table's entry for the layer's last (add+)LayerNorm
    kernel: the final norm, or norm1 where the final one runs in ffn_out's
    epilogue."""
    for tag in ("layernorm (final,", "layernorm (norm1,"):
        for k, v in kt.items():
            if k.startswith(tag) or k.startswith("add+" + tag):
                return v
    raise KeyError("no LayerNorm kernel in the table")


def kernel_table(cfg, model, x, mask, reps):
    """Time each kernel of the layer alone (HIP events on the launch stream).

    Returns name -> dict(us, flops or bytes, achieved, unit, frac, bound).
    """
    import torch

    out = {}
    with torch.inference_mode():
        for name, (fn, bound, work, io_bytes) in layer_ops(cfg, model, x, mask).items():
            us = device_us(fn, reps)
            if bound == "mfma":
                achieved = work / (us * 1e-6) / 1e12
                out[name] = dict(us=us, flops=work, io_bytes=io_bytes, bound="mfma",
                                 achieved=achieved,
                                 unit="TFLOP/s", peak=PEAK_MFMA_TFLOPS,
                                 frac=achieved / PEAK_MFMA_TFLOPS)
            else:
                achieved = work / (us * 1e-6) / 1e9
                out[name] = dict(us=us, bytes=work, io_bytes=io_bytes, bound="hbm",
                                 achieved=achieved,
                                 unit="GB/s", peak=PEAK_HBM_GBS, frac=achieved / PEAK_HBM_GBS)
    return out


# Kernel-symbol substring of each op family (the --pmc CSV names dispatches
# by symbol), and the calibration copy: dotl_smoke_test_identity over
# COPY_FLOATS floats reads and writes exactly 4 * COPY_FLOATS bytes.
KERNEL_FAMILY = (("ffn (", "ffn_ln_kernel"), ("attention", "attn_"), ("linear", "gemm"),
                 ("layernorm", "layernorm"))
COPY_SYMBOL = "identity_kernel"
COPY_FLOATS = 64 << 20
PROFILE_REPS = 5


def kernel_family(op_name):
    for prefix, symbol in KERNEL_FAMILY:
        if op_name.startswith(prefix) or prefix in op_name:
            return symbol
    raise KeyError(op_name)


def profile_ops(args):
    """Child mode for the --pmc passes: one op PROFILE_REPS times, then the copy.

    The op's inputs come from the layer's own kernels; the last PROFILE_REPS
    dispatches of the op's kernel family are the op alone.
    """
    import torch

    import kernel_ext
    from layer_runner import TransformerConfig, build_model, to_device
    from oracle.inputs import CONFIGS, make_case

    cfg = CONFIGS[args.config]
    x_np, mask_np, params = make_case(cfg)
    tcfg = TransformerConfig(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads,
                             cfg.ffn_dim, 1, cfg.causal)
    model = build_model(tcfg, params)
    x, mask = to_device(x_np, mask_np)
    fn = layer_ops(cfg, model, x, mask)[args.profile_ops][0]
    with torch.inference_mode():
        for _ in range(PROFILE_REPS):
            fn()
        torch.cuda.synchronize()
        src = torch.ones(COPY_FLOATS, device=x.device)
        for _ in range(PROFILE_REPS):
            kernel_ext.get_kernels().smoke_test_identity(src)
        torch.cuda.synchronize()
    return 0


def _pmc_pass(counter, op_name, config, outdir):
    """Mean per-dispatch `counter` (KiB) of the op and of the copy, from a child run."""
    import csv
    import glob
    import subprocess

    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", outdir,
           "-o", counter, "--", sys.executable, os.path.abspath(__file__),
           "--config", config, "--profile-ops", op_name]
    subprocess.run(cmd, check=True, timeout=180, stdout=subprocess.DEVNULL,
                   stderr=subprocess.DEVNULL, cwd=REPO)
    files = glob.glob(os.path.join(outdir, "**", f"{counter}_counter_collection.csv"),
                      recursive=True)
    if not files:
        raise RuntimeError(f"no {counter} counter file under {outdir}")
    rows = list(csv.DictReader(open(files[0])))
    fam = kernel_family(op_name)

    def mean_last(symbol):
        vals = [(int(r["Dispatch_Id"]), float(r["Counter_Value"])) for r in rows
                if symbol in r["Kernel_Name"] and r["Counter_Name"] == counter]
        vals = sorted(vals)[-PROFILE_REPS:]
        if len(vals) < PROFILE_REPS:
            raise RuntimeError(f"{counter}: {len(vals)} dispatches of {symbol}")
        return sum(v for _, v in vals) / len(vals)

    return mean_last(fam), mean_last(COPY_SYMBOL)


def measure_traffic(op_name, config):
    """HBM bytes per launch of `op_name` from two rocprofv3 --pmc passes.

    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are each scaled by what the
    same counter reads for the calibration copy, whose true traffic is
    4 * COPY_FLOATS bytes each way. Returns (bytes, detail) or (None, reason).
    """
    import shutil
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not on PATH"
    outdir = tempfile.mkdtemp(prefix="dotl_pmc_")
    try:
        op_rd, copy_rd = _pmc_pass("FETCH_SIZE", op_name, config, outdir)
        op_wr, copy_wr = _pmc_pass("WRITE_SIZE", op_name, config, outdir)
    except Exception as e:  # the figure is optional; the bench line is not
        return None, f"pmc pass failed: {e}"
    finally:
        shutil.rmtree(outdir, ignore_errors=True)
    true_bytes = 4.0 * COPY_FLOATS
    f_rd = true_bytes / (copy_rd * 1024.0)
    f_wr = true_bytes / (copy_wr * 1024.0)
    traffic = op_rd * 1024.0 * f_rd + op_wr * 1024.0 * f_wr
    return traffic, {"fetch_kib": round(op_rd, 1), "write_kib": round(op_wr, 1),
                     "fetch_scale": round(f_rd, 4), "write_scale": round(f_wr, 4)}


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
    model = build_model(tcfg, params)
    x, mask = to_device(x_np, mask_np)
    # Eager first: a model replays a graph it has captured whatever the knob
    # says later (as the reference's does), so the eager figure is taken
    # before any capture.
    ocfg.CUDA_GRAPH = "off"
    eager = time_layer(model, x, mask, steps, warmup)
    ocfg.CUDA_GRAPH = graph
    timed = time_layer(model, x, mask, steps, warmup)
    L = lengths_of(mask_np, cfg, cfg.batch_size)
    # Work on the rows that carry it: a padded batch's GEMMs are counted on
    # its valid rows (the packed path computes only those), attention on
    # valid query x valid key pairs.
    flops = gemm_flops(cfg, rows=int(L.sum())) + attention_useful_flops(cfg, L)
    res = dict(config=cfg, model=model, x=x, mask=mask, x_np=x_np, mask_np=mask_np,
               params=params, ms=timed["median_ms"], ms_eager=eager["median_ms"],
               timed=timed, eager=eager, flops=flops, t_valid=int(L.sum()),
               graphs=len(model._graphs))
    if with_kernels:
        res["kernels"] = kernel_table(cfg, model, x, mask, 20)
    return res


def mfma_ceiling(kx, workgroups=768, iters=128):
    """The matrix cores' sustained fp16 rate on this device, measured: the
    library's register-only MFMA probe at the C4 QKV product's MFMA count
    (768 workgroups x 4 waves x 2048 v_mfma_f32_32x32x16_f16). With random
    operands the clock drops under the matrix cores' power draw; that rate,
    not the 2.5 PFLOP/s datasheet figure, is what a GEMM on real data can
    reach."""
    flops = workgroups * 4 * iters * 16 * 32768
    res = {"probe": f"dotl_mfma_ceiling_probe: {workgroups} workgroups x 4 waves x "
                    f"{iters * 16} MFMAs, {flops / 1e9:.1f} GFLOP a launch"}
    for key, rnd in (("constant_tflops", False), ("random_tflops", True)):
        us = min(kx.mfma_ceiling_us(workgroups, iters, random_operands=rnd) for _ in range(3))
        res[key] = round(flops / (us * 1e-6) / 1e12, 1)
    res["random_frac_of_datasheet"] = round(res["random_tflops"] / PEAK_MFMA_TFLOPS, 4)
    return res


def main():
    # The package's [info] lines (graph capture notes) go to stderr: stdout
    # carries exactly one line, the JSON result.
    real_stdout = sys.stdout
    sys.stdout = sys.stderr
    try:
        return _main(real_stdout)
    finally:
        sys.stdout = real_stdout


def _main(out):
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (--gpus {args.gpus} "
              f"was asked for). The layer shards by batch: replicated weights, each rank a slice "
              f"of the batch, nothing exchanged, so one GPU's share at its real shape is what "
              f"this measures.",
              file=sys.stderr)
        return 2
    if args.profile_ops:
        return profile_ops(args)
    import torch

    import kernel_ext

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    if kernel_ext.get_kernels() is None:
        raise RuntimeError(f"libdotl_hip.so did not load: {kernel_ext.load_error()}")
    from optimized import config as ocfg

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
    ceiling = mfma_ceiling(kernel_ext.get_kernels())
    log(f"[bench] MFMA ceiling (fp16 32x32x16 from registers): {ceiling['random_tflops']:.0f} "
        f"TFLOP/s on random operands, {ceiling['constant_tflops']:.0f} on constant ones")
    attn = kt["attention"]
    ln = final_ln(kt)

    traffic, traffic_detail = None, "not measured (--traffic off)"
    if args.traffic == "pmc":
        log(f"[bench] HBM traffic of '{dom_name}' from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE ...")
        traffic, traffic_detail = measure_traffic(dom_name, args.config)
        log(f"[bench] traffic {traffic} bytes/launch ({traffic_detail})")

    cpu = None
    if not args.no_cpu:
        log("[bench] timing the CPU oracle baseline ...")
        cpu = cpu_baseline(cfg, r["x_np"], r["mask_np"], r["params"], args.cpu_budget)
        log(f"[bench] cpu baseline {cpu['value']:.0f} us on {cpu['cores']} threads")

    per_config, geomean = {}, None
    if not args.quick:
        log("[bench] per-config table: layer µs (graph replay), CPU oracle µs, attention MFMA %, "
            "final add+LN GB/s")
        speedups = []
        for name in ["C1", "C2", "C3", "C4", "C5"]:
            rr = r if name == args.config else run_config(
                name, max(SAMPLE_STEPS * MAX_SAMPLES, args.steps), 5, args.graph)
            k = rr["kernels"]
            entry = {"us": round(rr["ms"] * 1000.0, 2), "eager_us": round(rr["ms_eager"] * 1000.0, 2),
                     "samples_us": [round(v * 1000.0, 2) for v in rr["timed"]["samples_ms"]],
                     "steps_per_sample": rr["timed"]["steps_per_sample"],
                     "graph_captured": rr["graphs"] > 0,
                     "layer_tflops": round(rr["flops"] / (rr["ms"] * 1e-3) / 1e12, 2),
                     "layer_mfma_pct": round(100 * rr["flops"] / (rr["ms"] * 1e-3) / 1e12
                                             / PEAK_MFMA_TFLOPS, 2),
                     "attn_mfma_util_pct": round(100 * k["attention"]["frac"], 2),
                     "ln_hbm_gbs": round(final_ln(k)["achieved"], 1)}
            if not args.no_cpu:
                c = cpu if (name == args.config and cpu) else cpu_baseline(
                    rr["config"], rr["x_np"], rr["mask_np"], rr["params"], args.cpu_budget / 3)
                entry["cpu_us"] = round(c["value"], 1)
                entry["speedup_vs_cpu"] = round(c["value"] / (rr["ms"] * 1000.0), 2)
                speedups.append(entry["speedup_vs_cpu"])
            per_config[name] = entry
            log(f"[bench] {name}: {entry}")
            if rr is not r:
                del rr
                torch.cuda.empty_cache()
        if speedups and len(speedups) == 5:
            geomean = round(math.exp(sum(math.log(v) for v in speedups) / len(speedups)), 2)
            log(f"[bench] geomean speedup vs CPU oracle over C1..C5: {geomean}x")

    line = {
        "metric": "layer fwd µs/geomean speedup vs CPU ref; attn MFMA util %, LN HBM GB/s",
        "value": round(us, 2),
        "unit": "us/layer-fwd",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["timed"]["wall_ms"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp32 I/O; fp16 MFMA operands, fp32 accumulate (QKV "
                  + ocfg.QKV_PRECISION + ": LayerNorm output as split fp16 hi+lo, two "
                  "passes, where some query row attends to < "
                  + str(ocfg._QKV_SPLIT_MIN_KEYS) + " keys; else one fp16 pass)"),
        "data": "synthetic (seeded Xavier weights, N(0,1) x, key-padding lengths)",
        "config": {"workload": f"{cfg.name}: single-layer forward B={cfg.batch_size} "
                               f"S={cfg.seq_len} d_model={cfg.d_model} heads={cfg.num_heads} "
                               f"d_ff={cfg.ffn_dim} mask={cfg.mask} causal={cfg.causal}",
                   "graph": args.graph, "graph_captured": r["graphs"] > 0},
        "timing": (f"value = median of {len(r['timed']['samples_ms'])} HIP-event samples of "
                   f"{r['timed']['steps_per_sample']} forwards each inside the {args.steps} timed "
                   f"steps; ms_per_step = their wall time / steps"),
        "samples_us": [round(v * 1000.0, 2) for v in r["timed"]["samples_ms"]],
        "eager_us": round(r["ms_eager"] * 1000.0, 2),
        "tokens_per_s": round(cfg.tokens / (r["ms"] * 1e-3), 1),
        "layer_tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 2),
        "layer_mfma_pct": round(100 * r["flops"] / (r["ms"] * 1e-3) / 1e12 / PEAK_MFMA_TFLOPS, 2),
        "layer_work": (f"GEMM 8TD^2+4TDF on T={r['t_valid']} valid rows + attention "
                       f"4*hd*H*pairs = {r['flops'] / 1e9:.2f} GFLOP"),
        "roofline": {"bound": dom["bound"], "kernel": dom_name,
                     "achieved": round(dom["achieved"], 2), "peak": dom["peak"],
                     "unit": dom["unit"], "frac": round(dom["frac"], 4),
                     "traffic": None if traffic is None else round(traffic),
                     "traffic_detail": traffic_detail,
                     "compulsory_bytes": round(dom["io_bytes"]),
                     "sustained_peak": (ceiling["random_tflops"] if dom["bound"] == "mfma"
                                        else None),
                     "frac_of_sustained": (round(dom["achieved"] / ceiling["random_tflops"], 4)
                                           if dom["bound"] == "mfma" else None)},
        "mfma_ceiling": ceiling,
        "attn_mfma_util_pct": round(100 * attn["frac"], 2),
        "ln_hbm_gbs": round(ln["achieved"], 1),
        "kernels": {k: {"us": round(v["us"], 2), "achieved": round(v["achieved"], 2),
                        "unit": v["unit"], "frac": round(v["frac"], 4)} for k, v in kt.items()},
        "cpu_baseline": cpu,
        "speedup_vs_cpu": (round(cpu["value"] / us, 1) if cpu else None),
    }
    if per_config:
        line["per_config"] = per_config
        line["geomean_speedup_vs_cpu"] = geomean
    print(json.dumps(line), file=out, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
