"""Dispatch into the gfx950 kernels (reference optimized/kernels.py:1-339).

The boundary between torch ops and libdotl_hip.so, reached through
kernel_ext.get_kernels(). Same function names, arguments and fallback rules
as the reference:

  * attention has no fallback: a missing extension or an uncovered shape
    raises (reference optimized/kernels.py:297-338);
  * the elementwise helpers and the GEMMs answer in torch when the extension
    is missing or declines a shape (the reference's undefined-tensor / None
    convention). Every such answer is counted in `fallback_counts`, so a test
    can assert that the configured shapes never take one.

Precision edges are decided here (which tensors cross HBM as fp16, and the
QKV projection's arithmetic); see the notes on config.QKV_PRECISION.
"""

from __future__ import annotations

from collections import Counter
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import config

# op name -> times a torch fallback answered instead of a kernel
fallback_counts: Counter = Counter()

# Last values pushed into the extension's process-wide knobs (pushed on change).
_fp16_pushed = None
_cp_async_pushed = None

# Set (to a graphs._GraphIO) only while a forward is being captured into a
# hipGraph: the entry LayerNorm then reads the input, and the output
# LayerNorm writes the output, through the graph's I/O slot.
_graph_io = None


# Set by OptimizedTransformer.forward for the duration of a forward of a
# model with more than one block (config.STACK_PRECISION): rounding error
# compounds through the residual stream from block to block, so a stack
# spends more of its arithmetic on precision than one block needs.
_stack_precision = False


# Set by OptimizedTransformer.forward: whether some query row of this forward
# attends to fewer than config._QKV_SPLIT_MIN_KEYS keys (what
# QKV_PRECISION = "auto" resolves on).
_qkv_few_keys = True
# Rows of each sequence whose QKV keeps the split arithmetic when only a
# causal prefix attends to few keys (0: every row, as _qkv_precision says).
_qkv_split_prefix = 0


def _qkv_precision() -> str:
    """The QKV arithmetic this forward applies (config.QKV_PRECISION, "auto" resolved)."""
    v = config.QKV_PRECISION
    if v == "auto":
        return "fp16x2" if _qkv_few_keys else "fp16"
    return v


def _lb() -> str:
    """config.LINEAR_BIAS as this forward applies it: "auto" becomes the split
    fp16x3 arithmetic ("tf32") inside a multi-block forward."""
    v = config.LINEAR_BIAS
    return "tf32" if (v == "auto" and _stack_precision) else v


def _lg() -> str:
    """config.LINEAR_GELU as this forward applies it (see _lb)."""
    v = config.LINEAR_GELU
    return "tf32" if (v == "auto" and _stack_precision) else v


def _input_io(x: torch.Tensor):
    """io argument for a LayerNorm reading `x`: the slot when x is the input
    of the forward being captured, else None."""
    io = _graph_io
    if io is not None and x is io.x_stand_in:
        io.in_bound = True
        return (io.slot, 1)
    return None


def _output_io():
    """io argument for the forward's output LayerNorm while capturing."""
    io = _graph_io
    return (io.slot, 2) if io is not None else None


def _note_output(out: torch.Tensor, io) -> torch.Tensor:
    """Record which tensor stands for the slot-bound output."""
    if io is not None and _graph_io is not None:
        _graph_io.out_ptr = out.data_ptr()
    return out


def _sync_attention_precision(kernels) -> None:
    """Keep the extension's fp16 knob (what "auto" precision resolves to) in step."""
    global _fp16_pushed
    want = config.ATTENTION_PRECISION in ("auto", "fp16")
    if _fp16_pushed != want:
        kernels.wmma_set_fp16(want)
        _fp16_pushed = want


def _sync_cp_async(kernels) -> None:
    global _cp_async_pushed
    want = config._CP_ASYNC_CODE[config.CP_ASYNC]
    if _cp_async_pushed != want and hasattr(kernels, "wmma_set_cp_async"):
        kernels.wmma_set_cp_async(want)
        _cp_async_pushed = want


def _custom_kernels():
    """The extension object, or None when the library would not load."""
    import kernel_ext

    return kernel_ext.get_kernels()


def _add_layernorm(x: torch.Tensor, sub: torch.Tensor, norm,
                   normed_half: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """(x + sub, norm(x + sub)) in one kernel. A 16-bit x keeps its dtype
    throughout (normed_half narrows fp32 only)."""
    normed_half = normed_half and x.dtype == torch.float32
    kernels = _custom_kernels()
    if kernels is not None:
        return tuple(kernels.fused_add_layernorm(x, sub, norm.weight, norm.bias, norm.eps,
                                                 normed_half))
    fallback_counts["add_layernorm"] += 1
    total = x + sub
    out = F.layer_norm(total, (total.shape[-1],), norm.weight, norm.bias, norm.eps)
    return total, (out.half() if normed_half else out)


def _add_layernorm_output(x: torch.Tensor, sub: torch.Tensor, norm) -> torch.Tensor:
    """norm(x + sub) as the forward's output: the sum is not stored (nothing
    reads it), and under capture the result goes through the graph's slot."""
    kernels = _custom_kernels()
    if kernels is not None:
        io = _output_io()
        return _note_output(kernels.fused_add_layernorm_final(x, sub, norm.weight, norm.bias,
                                                              norm.eps, io=io), io)
    fallback_counts["add_layernorm"] += 1
    total = x + sub
    return F.layer_norm(total, (total.shape[-1],), norm.weight, norm.bias, norm.eps)


def _entry_norm(x: torch.Tensor, norm) -> Tuple[torch.Tensor, torch.Tensor]:
    """(residual stream, norm1(x)) for the model's first LayerNorm.

    Normally the residual stream is x itself. While a graph is captured with
    x bound to its I/O slot, the norm also writes a copy of x (from the same
    read), and that copy is the residual stream: every later read of x then
    happens inside the graph's own memory, so the bound input is read once.
    """
    io = _input_io(x) if config.LAYERNORM != "off" else None
    if io is None:
        return x, norm(x)
    rows, width = x.numel() // x.shape[-1], x.shape[-1]
    if x.dtype != torch.float32:
        kind = "float"     # the normed output in x's own dtype
    elif _normed_split_wanted():
        kind = "split"
    elif _normed_wants_fp16(rows, width):
        kind = "half"
    else:
        kind = "float"
    x_copy, normed = _custom_kernels().fused_layernorm_copy(x, norm.weight, norm.bias,
                                                           norm.eps, kind, io=io)
    return x_copy, normed


def _linear_gelu(x: torch.Tensor, lin, out_half: bool = False) -> torch.Tensor:
    """GELU_erf(lin(x)) with the GELU in the GEMM epilogue."""
    if _lg() != "off" and lin.bias is not None:
        kernels = _custom_kernels()
        if kernels is not None:
            out = kernels.linear_gelu(x, lin.weight, lin.bias, -1,
                                      config._GEMM_MATH_CODE[_lg()], out_half)
            if out is not None:
                return out
    fallback_counts["linear_gelu"] += 1
    out = F.gelu(F.linear(x.to(lin.weight.dtype), lin.weight, lin.bias), approximate="none")
    return out.half() if (out_half and out.dtype == torch.float32) else out


def _split_planes(t: torch.Tensor) -> torch.Tensor:
    """fp32 -> [2, ...] fp16 planes: hi = fp16(t), lo = fp16((t - hi) * 2^12)."""
    hi = t.half()
    lo = ((t - hi.float()) * 4096.0).half()
    return torch.stack([hi, lo])


def _normed_split_wanted() -> bool:
    """Should a LayerNorm feeding the QKV projection emit split fp16 planes?

    Yes exactly when that projection runs a split arithmetic (fp16x2 or
    fp16x3) on the pipelined GEMM: the planes carry ~22 bits of the LayerNorm
    output in the same bytes as fp32, already in the form the MFMA passes
    read.
    """
    return (_lb() == "auto" and _qkv_precision() in ("fp16x3", "fp16x2")
            and config.NORMED_FP16 != "off")


def _layernorm_split(x: torch.Tensor, norm) -> torch.Tensor:
    """LayerNorm(x) as split fp16 planes [2, *x.shape]; for a 16-bit x, the
    plain LayerNorm in x's dtype (planes carry fp32 values only)."""
    if x.dtype != torch.float32:
        return _layernorm(x, norm)
    kernels = _custom_kernels()
    if kernels is not None:
        return kernels.fused_layernorm_split(x, norm.weight, norm.bias, norm.eps)
    fallback_counts["layernorm"] += 1
    return _split_planes(F.layer_norm(x, (x.shape[-1],), norm.weight, norm.bias, norm.eps))


def _add_layernorm_split(x: torch.Tensor, sub: torch.Tensor, norm):
    """(x + sub, LayerNorm(x + sub) as split fp16 planes); a 16-bit x gets
    the plain add+LayerNorm in its dtype."""
    if x.dtype != torch.float32:
        return _add_layernorm(x, sub, norm)
    kernels = _custom_kernels()
    if kernels is not None:
        return tuple(kernels.fused_add_layernorm_split(x, sub, norm.weight, norm.bias, norm.eps))
    fallback_counts["add_layernorm"] += 1
    total = x + sub
    return total, _split_planes(F.layer_norm(total, (total.shape[-1],), norm.weight,
                                             norm.bias, norm.eps))


def _linear_bias_split(planes: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                       out_half: bool = False) -> torch.Tensor:
    """planes-as-x @ weight^T + bias in the split arithmetic _qkv_precision() names."""
    kernels = _custom_kernels()
    if kernels is not None:
        out = kernels.linear_bias_split(planes, weight, bias, -1, out_half,
                                        split_weight=_qkv_precision() == "fp16x3")
        if out is not None:
            return out
    fallback_counts["linear_bias"] += 1
    x = planes[0].float() + planes[1].float() / 4096.0
    out = F.linear(x, weight, bias)
    return out.half() if out_half else out


def _linear_bias_split_prefix(planes: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                              out_half: bool, prefix: int) -> torch.Tensor:
    """The QKV projection of split planes [2, B, S, D] when only each
    sequence's first `prefix` rows need the split arithmetic (a causal batch:
    those rows' queries see only keys of the same prefix): one fp16 pass over
    every row on the hi plane (the LayerNorm output rounded to fp16, the
    operand a one-pass projection reads), then the split passes over the
    prefix rows, written over theirs."""
    B, S, D = planes.shape[1], planes.shape[2], planes.shape[3]
    out = _linear_bias(planes[0], weight, bias, out_half=out_half,
                       math=config._QKV_MATH_CODE["fp16"])
    # (run on a second stream beside the one-pass GEMM, this small GEMM
    # measured no faster at C3: 262 us either way, and eager 313)
    kernels = _custom_kernels()
    if B == 1 and kernels is not None and planes.is_contiguous() and out.is_contiguous():
        # one sequence: its prefix rows are contiguous in both planes and in
        # the output, so the split GEMM reads and writes them in place
        done = kernels.linear_bias_planes(planes[0, 0, :prefix], planes[1, 0, :prefix], weight,
                                          bias, out[0, :prefix],
                                          split_weight=_qkv_precision() == "fp16x3")
        if done is not None:
            return out
    pre = planes[:, :, :prefix].reshape(2, B * prefix, D).contiguous()
    pre_out = _linear_bias_split(pre, weight, bias, out_half=out_half)
    out[:, :prefix] = pre_out.view(B, prefix, -1)
    return out


def _layernorm_pack(x: torch.Tensor, norm, packing) -> Tuple[torch.Tensor, torch.Tensor]:
    """(valid rows of x, LayerNorm of them): the gather into packed rows.

    The normed rows take the form the QKV projection consumes: split fp16
    planes for the fp16x3 projection, else fp16 or fp32 as _normed_wants_fp16
    decides.
    """
    width = x.shape[-1]
    if x.dtype != torch.float32:
        kind = "float"     # the normed rows in x's own dtype
    elif _normed_split_wanted():
        kind = "split"
    elif _normed_wants_fp16(packing.t_valid, width):
        kind = "half"
    else:
        kind = "float"
    kernels = _custom_kernels()
    if kernels is not None:
        x_rows, normed = kernels.fused_layernorm_rows(x, norm.weight, norm.bias, packing.idx,
                                                      norm.eps, kind, True, io=_input_io(x))
        return x_rows, normed
    fallback_counts["layernorm"] += 1
    x_rows = x.reshape(-1, width).index_select(0, packing.idx.long())
    out = F.layer_norm(x_rows, (width,), norm.weight, norm.bias, norm.eps)
    if kind == "split":
        return x_rows, _split_planes(out)
    return x_rows, (out.half() if kind == "half" else out)


def _add_layernorm_unpack(x: torch.Tensor, sub: torch.Tensor, norm, packing) -> torch.Tensor:
    """LayerNorm(x + sub) of packed rows, returned as [B, S, D] with zero padded rows.

    The model's last add+LN and the reference's final masked_fill in one
    kernel; the residual sum is not stored.
    """
    width = x.shape[-1]
    shape = (packing.batch, packing.seq_len, width)
    kernels = _custom_kernels()
    if kernels is not None:
        io = _output_io()
        out = kernels.fused_add_layernorm_rows(x, sub, norm.weight, norm.bias, packing.inv,
                                               norm.eps, io=io)
        return _note_output(out, io).view(shape)
    fallback_counts["add_layernorm"] += 1
    y = F.layer_norm(x + sub, (width,), norm.weight, norm.bias, norm.eps)
    out = torch.zeros(packing.batch * packing.seq_len, width, dtype=y.dtype, device=y.device)
    out.index_copy_(0, packing.idx.long(), y)
    return out.view(shape)


def _layernorm_unpack(x: torch.Tensor, norm, packing) -> torch.Tensor:
    """LayerNorm of packed rows, returned as [B, S, D] with zero padded rows:
    the model's output norm and the reference's final masked_fill in one
    kernel (the scatter back from packed rows)."""
    width = x.shape[-1]
    shape = (packing.batch, packing.seq_len, width)
    kernels = _custom_kernels()
    if kernels is not None:
        io = _output_io()
        _, out = kernels.fused_layernorm_rows(x, norm.weight, norm.bias, packing.inv, norm.eps,
                                              "float", False, io=io)
        return _note_output(out, io).view(shape)
    fallback_counts["layernorm"] += 1
    y = F.layer_norm(x, (width,), norm.weight, norm.bias, norm.eps)
    out = torch.zeros(packing.batch * packing.seq_len, width, dtype=y.dtype, device=y.device)
    out.index_copy_(0, packing.idx.long(), y)
    return out.view(shape)


def _layernorm(x: torch.Tensor, norm, out_half: bool = False,
               output: bool = False) -> torch.Tensor:
    """LayerNorm(x) * w + b: a norm with no residual add before it.

    `output`: this is the forward's output norm (bound to the graph's I/O
    slot while capturing)."""
    out_half = out_half and x.dtype == torch.float32
    if config.LAYERNORM != "off":
        kernels = _custom_kernels()
        if kernels is not None:
            io = _output_io() if output else None
            return _note_output(kernels.fused_layernorm(x, norm.weight, norm.bias, norm.eps,
                                                        out_half, io=io), io)
    fallback_counts["layernorm"] += 1
    out = F.layer_norm(x, (x.shape[-1],), norm.weight, norm.bias, norm.eps)
    return out.half() if out_half else out


def _attention_wants_fp16() -> bool:
    """Will attention really contract q/k/v in fp16 (so fp16 q/k/v are free)?"""
    if config.QKV_FP16 == "off":
        return False
    if config.ATTENTION_IMPL not in ("auto", "wmma"):
        return False
    return config.ATTENTION_PRECISION in ("auto", "fp16")


def _qkv_math_code() -> int:
    """linear_bias `math` for the QKV projection (_qkv_precision())."""
    if _lb() == "tf32":
        return config._GEMM_MATH_CODE["tf32"]
    return config._QKV_MATH_CODE[_qkv_precision()]


def _normed_wants_fp16(rows: int, width: int) -> bool:
    """Should a LayerNorm feeding the QKV projection emit fp16?

    Only when that projection narrows its A operand to fp16 anyway: one-pass
    fp16 math. The split fp16x3 projection needs the fp32 values.
    """
    if config.NORMED_FP16 == "off" or _lb() != "auto":
        return False
    if _qkv_math_code() != -1:
        return False
    if width > config._NORMED_FP16_MAX_K:
        return False
    return config._QKV_FP16_MIN_ROWS <= rows <= config._LINEAR_BIAS_MAX_ROWS


def _gelu_input_wants_fp16(rows: int, width: int) -> bool:
    """Should norm2 emit fp16 for linear_gelu (which narrows A with the same RNE)?"""
    if config.NORMED_FP16 == "off" or _lg() != "auto":
        return False
    if width > config._NORMED_FP16_MAX_K:
        return False
    return config._QKV_FP16_MIN_ROWS <= rows <= config._LINEAR_BIAS_MAX_ROWS


def _gelu_output_wants_fp16(rows: int) -> bool:
    """Should linear_gelu store fp16 for ffn_out (whose fp16 math narrows it anyway)?"""
    if config.GELU_FP16 == "off" or _lb() != "auto":
        return False
    return rows <= config._LINEAR_BIAS_MAX_ROWS


def _linear_bias(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                 out_half: bool = False, math: Optional[int] = None,
                 residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x @ weight^T + bias on the MFMA GEMM; `math` overrides the config's.

    With `residual` (fp32, the output's shape) the result is residual + that,
    the add done in the GEMM's epilogue where the kernel can (else added
    here, and counted as a fallback).
    """
    rows = x.numel() // x.shape[-1] if x.dim() >= 1 and x.shape[-1] else 0
    if (_lb() != "off" and bias is not None
            and rows <= config._LINEAR_BIAS_MAX_ROWS):
        kernels = _custom_kernels()
        if kernels is not None:
            code = config._GEMM_MATH_CODE[_lb()] if math is None else math
            out = kernels.linear_bias(x, weight, bias, -1, code, out_half, residual=residual)
            if out is not None:
                return out
            if residual is not None:
                out = kernels.linear_bias(x, weight, bias, -1, code, out_half)
                if out is not None:
                    fallback_counts["linear_bias_residual"] += 1
                    return residual + out
    fallback_counts["linear_bias"] += 1
    out = F.linear(x.to(weight.dtype), weight, bias)
    if residual is not None:
        out = residual + out
    if x.dtype in (torch.float16, torch.bfloat16):
        want = x.dtype
    else:
        want = torch.float16 if out_half else torch.float32
    return out if out.dtype == want else out.to(want)


def _residual_epilogue_wanted(width_in: int) -> bool:
    """Fold the residual adds into out_proj's and ffn_out's epilogues?

    Where the GEMM runs the pipelined kernel on fp16 operands (its K a
    multiple of 64), the add+LayerNorm after it then becomes a plain
    LayerNorm: one tensor read instead of two, none written back.
    """
    return (config.RESIDUAL_EPILOGUE != "off" and _lb() == "auto"
            and width_in % 64 == 0 and width_in >= config._RESIDUAL_EPILOGUE_MIN_D)


def _ln_epilogue_wanted(rows: int, width: int) -> bool:
    """Apply the LayerNorm after out_proj / ffn_out in that GEMM's epilogue
    (one workgroup's tile spans the whole row)?"""
    return (config.LN_EPILOGUE != "off" and config.LAYERNORM != "off" and _lb() == "auto"
            and width % 4 == 0 and width <= config._LN_EPILOGUE_MAX_D
            and rows >= config._LN_EPILOGUE_MIN_ROWS)


def _ln_epilogue_call(call, width: int, kind: str, store_out: bool, packing, output: bool,
                      zeroes_padded: bool = False):
    """Run a kernel with the LayerNorm epilogue (`call(**kw)`: linear_layernorm
    or ffn_layernorm with every other argument bound) in the layer's form:
    with `packing` its normed rows land in the padded [B, S, width] layout
    (fp32) and the padded rows are zeroed (by the kernel itself where
    `zeroes_padded`, else by zero_rows); `output` binds the normed tensor to
    a captured graph's output slot. None where the kernel declines."""
    io = _output_io() if output else None
    if packing is not None:
        extra = {"zero_padded": True} if zeroes_padded else {}
        res = call(normed="float", store_out=store_out, out_row=packing.idx,
                   normed_rows=packing.batch * packing.seq_len, io=io, **extra)
        if res is None:
            return None
        h, out = res
        if not zeroes_padded:
            _custom_kernels().zero_rows(out, packing.inv, io=io)
        out = _note_output(out, io)
        return h, out.view(packing.batch, packing.seq_len, width)
    res = call(normed=kind, store_out=store_out, io=io)
    if res is None:
        return None
    h, out = res
    return h, _note_output(out, io)


def _linear_norm(x: torch.Tensor, lin, residual: torch.Tensor, norm, kind: str,
                 store_out: bool = True, packing=None, output: bool = False):
    """(residual + lin(x), norm of that): `kind` is the normed form, "float",
    "half" (fp16) or "split" (fp16 hi/lo planes).

    One GEMM whose epilogue adds the residual and normalises each row where
    _ln_epilogue_wanted (bit-identical to the two kernels); else the GEMM
    with its residual epilogue, then the LayerNorm. With `packing` the normed
    rows land in the padded [B, S, D] layout with zero padded rows (the
    model's output norm, always fp32). `output`: the normed tensor is the
    forward's output (a captured graph's output slot). `store_out` False:
    the caller does not read the sum (None may come back for it).
    """
    width = lin.weight.shape[0]
    rows = x.numel() // x.shape[-1]
    if _ln_epilogue_wanted(rows, width) and x.dtype == torch.float16 and lin.bias is not None:
        kernels = _custom_kernels()
        if kernels is not None:
            res = _ln_epilogue_call(
                lambda **kw: kernels.linear_layernorm(x, lin.weight, lin.bias, residual,
                                                      norm.weight, norm.bias, norm.eps, **kw),
                width, kind, store_out, packing, output)
            if res is not None:
                return res
    h = _linear_bias(x, lin.weight, lin.bias, residual=residual)
    if packing is not None:
        return h, _layernorm_unpack(h, norm, packing)
    if kind == "split":
        return h, _layernorm_split(h, norm)
    return h, _layernorm(h, norm, out_half=kind == "half", output=output)


def _ffn_ln_wanted(x: torch.Tensor, ffn_in, ffn_out) -> bool:
    """Run the FFN, its residual add and the following LayerNorm as one
    kernel (config.FFN_LN)? Exactly where the two GEMMs it replaces would be
    the one-pass GELU GEMM with an fp16 output and the GEMM with the
    LayerNorm epilogue, and the kernel's shapes hold."""
    rows, d_model = x.numel() // x.shape[-1], x.shape[-1]
    d_ff = ffn_in.weight.shape[0]
    return (config.FFN_LN != "off" and x.dtype == torch.float16 and _lg() == "auto"
            and ffn_in.bias is not None and ffn_out.bias is not None
            and _gelu_output_wants_fp16(rows) and _ln_epilogue_wanted(rows, d_model)
            and d_model == 256 and d_ff % 64 == 0 and d_ff <= 2048)


def _ffn_norm(x: torch.Tensor, ffn_in, ffn_out, residual: torch.Tensor, norm, kind: str,
              store_out: bool = True, packing=None, output: bool = False):
    """(residual + ffn_out(GELU(ffn_in(x))), norm of that), the forms and
    arguments as _linear_norm's: one kernel where _ffn_ln_wanted (the hidden
    activations never reach memory; bit-identical to the two GEMMs), else
    _linear_gelu followed by _linear_norm."""
    rows = x.numel() // x.shape[-1]
    if _ffn_ln_wanted(x, ffn_in, ffn_out):
        kernels = _custom_kernels()
        if kernels is not None:
            res = _ln_epilogue_call(
                lambda **kw: kernels.ffn_layernorm(x, ffn_in.weight, ffn_in.bias, ffn_out.weight,
                                                   ffn_out.bias, residual, norm.weight,
                                                   norm.bias, norm.eps, **kw),
                x.shape[-1], kind, store_out, packing, output, zeroes_padded=True)
            if res is not None:
                return res
    hidden = _linear_gelu(x, ffn_in, out_half=_gelu_output_wants_fp16(rows))
    return _linear_norm(hidden, ffn_out, residual, norm, kind, store_out, packing, output)


def _ffn_block_eligible(x, ffn_in, ffn_out) -> bool:
    """Would _ffn_block run the fused kernel for this block (rather than decline)?"""
    if config.FFN_BLOCK == "off":
        return False
    if (_lg() != "auto" or _lb() != "auto"
            or config.NORMED_FP16 == "off" or config.GELU_FP16 == "off"):
        return False
    if ffn_in.bias is None or ffn_out.bias is None or x.dtype != torch.float32:
        return False
    d_model, d_ff = x.shape[-1], ffn_in.weight.shape[0]
    if config.FFN_BLOCK != "force" and d_model > config._FFN_BLOCK_MAX_D:
        return False
    return d_model <= 128 and d_ff <= 512 and d_model % 8 == 0 and d_ff % 8 == 0


def _ffn_block(x, attn_out, norm1, ffn_in, ffn_out, norm2):
    """The fused post-attention block, or None to run it unfused
    (reference optimized/kernels.py:269-294).

    The kernel's arithmetic is the default unfused chain's (fp16 LayerNorm
    output, fp16 GEMM operands, fp16 GELU output), so it is used only while
    the knobs select exactly that chain: a request for the split fp16x3
    GEMMs, or for fp32 edges, runs unfused.
    """
    if config.FFN_BLOCK == "off":
        return None
    if (_lg() != "auto" or _lb() != "auto"
            or config.NORMED_FP16 == "off" or config.GELU_FP16 == "off"):
        return None
    if ffn_in.bias is None or ffn_out.bias is None or x.dtype != torch.float32:
        return None
    if config.FFN_BLOCK != "force" and x.shape[-1] > config._FFN_BLOCK_MAX_D:
        return None
    kernels = _custom_kernels()
    if kernels is None or not hasattr(kernels, "fused_ffn_block"):
        return None
    out = kernels.fused_ffn_block(x, attn_out, norm1.weight, norm1.bias, ffn_in.weight,
                                  ffn_in.bias, ffn_out.weight, ffn_out.bias, norm2.weight,
                                  norm2.bias, norm1.eps)
    return (out[0], out[1]) if out else None



def _attention_kernels():
    """The loaded extension, synced with the attention knobs; raises without it.

    Attention runs only on this build's own MFMA kernels: with libdotl_hip.so
    absent there is nothing to run it on, and the call fails.
    """
    import kernel_ext

    kernels = kernel_ext.get_kernels()
    if kernels is None:
        raise RuntimeError(f"attention needs libdotl_hip.so, which is not loaded "
                           f"({kernel_ext.load_error()}); build it with "
                           f"`python __graft_entry__.py` (hipcc, gfx950)")
    _sync_attention_precision(kernels)
    _sync_cp_async(kernels)
    return kernels

def _attention_packed(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, packing,
                      is_causal: bool, scale: float) -> torch.Tensor:
    """Attention over packed sequences ([T_valid, H, hd] views) -> [T_valid, H*hd].

    No mask: each sequence's rows are exactly its valid tokens. The grid is
    sized by the padded length S (not the longest valid one), so a captured
    graph depends on the packing's sizes only.
    """
    kernels = _attention_kernels()
    return kernels.fused_attention_forward(
        q, k, v, None, is_causal, scale,
        config._IMPL_CODE[config.ATTENTION_IMPL], config._OUT_LAYOUT_BSHD,
        config._PRECISION_CODE[config.ATTENTION_PRECISION],
        cu_seqlens=packing.cu, max_seqlen=packing.seq_len)


def _attention_dispatch(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        attn_mask: Optional[torch.Tensor], is_causal: bool,
                        scale: float) -> torch.Tensor:
    """Attention on the MFMA kernel; there is no other route.

    Returns [B, S, H*head_dim]. `attn_mask` ([B,1,1,S] key mask, True = may
    attend) and `is_causal` may both be set: causal stays a flag so the kernel
    skips the tiles past the diagonal instead of masking them.
    """
    kernels = _attention_kernels()
    return kernels.fused_attention_forward(
        q, k, v, attn_mask, is_causal, scale,
        config._IMPL_CODE[config.ATTENTION_IMPL],
        config._OUT_LAYOUT_BSHD,
        config._PRECISION_CODE[config.ATTENTION_PRECISION],
    )
