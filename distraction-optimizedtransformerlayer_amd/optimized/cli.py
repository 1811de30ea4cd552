"""Command-line overrides for optimized/config.py.

The same three hooks and flags as the reference (reference optimized/cli.py:21-171):
parse_args() -> add_arguments(parser); validate_args() -> validate_args(args,
device, dtype); main() -> apply_overrides(args). Two flags are added for this
build's precision edges: --qkv-precision and --gelu-fp16.
"""

from __future__ import annotations

import argparse

from . import config


def add_arguments(parser: argparse.ArgumentParser) -> None:
    """Add the optimization flags to a harness's own parser."""
    parser.add_argument("--attn-backend", choices=("custom",), default=None,
                        help="override ATTENTION_BACKEND for this run (one legal value)")
    parser.add_argument("--attn-impl", choices=("auto", "scalar", "wmma", "tile"), default=None,
                        help="override ATTENTION_IMPL: which attention kernel runs")
    parser.add_argument("--attn-precision", choices=("auto", "fp32", "tf32", "fp16", "bf16"),
                        default=None,
                        help="override ATTENTION_PRECISION: the arithmetic attention "
                             "contracts in (the MFMA kernel has fp16)")
    parser.add_argument("--linear-gelu", choices=("auto", "tf32", "off"), default=None,
                        help="override LINEAR_GELU: 'auto' fp16 operands, 'tf32' the split "
                             "fp16x3 arithmetic, 'off' F.linear + F.gelu")
    parser.add_argument("--linear-bias", choices=("auto", "tf32", "off"), default=None,
                        help="override LINEAR_BIAS for QKV/out_proj/ffn_out: 'auto' fp16, "
                             "'tf32' split fp16x3, 'off' F.linear")
    parser.add_argument("--layernorm", choices=("auto", "off"), default=None,
                        help="override LAYERNORM for the entry LayerNorm")
    parser.add_argument("--qkv-fp16", choices=("auto", "off"), default=None,
                        help="override QKV_FP16: write q/k/v in fp16 for attention")
    parser.add_argument("--normed-fp16", choices=("auto", "off"), default=None,
                        help="override NORMED_FP16: fp16 LayerNorm outputs where the "
                             "consuming GEMM narrows anyway")
    parser.add_argument("--cp-async", choices=("auto", "sync", "off"), default=None,
                        help="override CP_ASYNC (accepted; no effect on gfx950)")
    parser.add_argument("--cuda-graph", choices=("off", "auto", "always"), default=None,
                        help="override CUDA_GRAPH: capture the forward pass into a hipGraph")
    parser.add_argument("--qkv-precision", choices=("auto", "fp16x2", "fp16x3", "fp16"),
                        default=None,
                        help="override QKV_PRECISION: arithmetic of the QKV projection")
    parser.add_argument("--gelu-fp16", choices=("auto", "off"), default=None,
                        help="override GELU_FP16: store the GELU output in fp16 for ffn_out")


def apply_overrides(args: argparse.Namespace) -> None:
    """Write the requested overrides into config, before any model is built."""
    pairs = (("attn_backend", "ATTENTION_BACKEND"), ("attn_impl", "ATTENTION_IMPL"),
             ("attn_precision", "ATTENTION_PRECISION"), ("linear_gelu", "LINEAR_GELU"),
             ("linear_bias", "LINEAR_BIAS"), ("layernorm", "LAYERNORM"),
             ("qkv_fp16", "QKV_FP16"), ("normed_fp16", "NORMED_FP16"),
             ("cp_async", "CP_ASYNC"), ("cuda_graph", "CUDA_GRAPH"),
             ("qkv_precision", "QKV_PRECISION"), ("gelu_fp16", "GELU_FP16"))
    for arg, knob in pairs:
        value = getattr(args, arg, None)
        if value is not None:
            setattr(config, knob, value)

    # torch.compile's reduce-overhead mode captures graphs itself; stand down
    # when graphs were only the default, refuse when both were asked for.
    if getattr(args, "compile_user", False) and config.CUDA_GRAPH != "off":
        if getattr(args, "cuda_graph", None) is None:
            config.CUDA_GRAPH = "off"
            print("[info] --compile-user: CUDA_GRAPH forced off, since "
                  "--compile-mode reduce-overhead already captures graphs")
        else:
            raise ValueError("--compile-user and --cuda-graph are two implementations of "
                             "the same optimization; pick one.")


def validate_args(args: argparse.Namespace, device, dtype) -> None:
    """Warn about combinations that do nothing. Never raises."""
    cuda_graph = getattr(args, "cuda_graph", None)
    if cuda_graph in ("auto", "always") and getattr(device, "type", "cuda") != "cuda":
        print("[warning] --cuda-graph has no effect on a non-GPU device")
    try:
        activation = args.batch_size * args.seq_len * args.d_model
    except AttributeError:
        return
    if cuda_graph == "always" and activation > config._GRAPH_MAX_ACTIVATION:
        print(f"[warning] --cuda-graph always at {activation} activation elements is past "
              f"the capture gate ({config._GRAPH_MAX_ACTIVATION}); it pins the whole "
              f"working set in the graph's private pool")
