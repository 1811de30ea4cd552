"""Drop-in replacements for the baseline's submodules (reference optimized/layers.py).

Parameter and submodule names match BaselineTransformer's
(torch_transformer_benchmark.py:70-245), so one state_dict loads into either
model with strict=True: the parameter names are the weight format.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import config
from . import kernels as okernels
from .kernels import (_add_layernorm, _add_layernorm_output, _add_layernorm_split,
                      _add_layernorm_unpack,
                      _attention_dispatch, _attention_packed, _attention_wants_fp16,
                      _ffn_block, _ffn_block_eligible, _gelu_input_wants_fp16,
                      _gelu_output_wants_fp16, _layernorm, _layernorm_split,
                      _linear_bias, _linear_bias_split, _linear_bias_split_prefix,
                      _ffn_norm, _linear_gelu, _linear_norm,
                      _normed_split_wanted, _normed_wants_fp16, _qkv_math_code,
                      _residual_epilogue_wanted)
from .util import _version_or_none


class MyLinear(nn.Module):
    """nn.Linear's parameter names and shapes (weight [out, in], bias [out])."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        self.bias = nn.Parameter(torch.empty(out_features)) if bias else None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # out_proj and ffn_out; the QKV weights are fused in MySelfAttention and
        # ffn_in goes through _linear_gelu.
        return _linear_bias(x, self.weight, self.bias)


class MyLayerNorm(nn.Module):
    """nn.LayerNorm's parameter names and shapes."""

    def __init__(self, d_model: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d_model))
        self.bias = nn.Parameter(torch.zeros(d_model))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # Reached by the model's first norm (every other one is fused into a
        # residual add) and by the padded path's trailing norm. Its consumer
        # is a QKV projection: split fp16 planes for the fp16x3 projection, or
        # fp16 where that projection narrows anyway.
        if _normed_split_wanted():
            return _layernorm_split(x, self)
        rows = x.numel() // x.shape[-1]
        return _layernorm(x, self, out_half=_normed_wants_fp16(rows, x.shape[-1]))


class MySelfAttention(nn.Module):
    """BaselineSelfAttention's submodule names (q_proj, k_proj, v_proj, out_proj)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = MyLinear(d_model, d_model)
        self.k_proj = MyLinear(d_model, d_model)
        self.v_proj = MyLinear(d_model, d_model)
        self.out_proj = MyLinear(d_model, d_model)
        # Fused [3D, D] QKV weight and [3D] bias, rebuilt when a source
        # parameter moves (device/dtype) or changes (version). Plain
        # attributes, so they stay out of state_dict().
        self._qkv_key: Optional[Tuple] = None
        self._qkv_weight: Optional[torch.Tensor] = None
        self._qkv_bias: Optional[torch.Tensor] = None
        self._qkv_generation = 0   # rebuild count (graph capture checks it)

    def _get_qkv_weight(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Q, K and V projections as one [3*d_model, d_model] GEMM operand.

        One GEMM with N = 3D instead of three with N = D: three times the
        output tiles per launch, one read of the normalised input instead of
        three (reference optimized/layers.py:88-110 does the same for its card).
        """
        wq, wk, wv = self.q_proj.weight, self.k_proj.weight, self.v_proj.weight
        key = (wq.device, wq.dtype, _version_or_none(wq), _version_or_none(wk),
               _version_or_none(wv), _version_or_none(self.q_proj.bias),
               _version_or_none(self.k_proj.bias), _version_or_none(self.v_proj.bias))
        if self._qkv_key != key:
            with torch.no_grad():
                self._qkv_weight = torch.cat([wq, wk, wv], dim=0)
                self._qkv_bias = torch.cat([self.q_proj.bias, self.k_proj.bias,
                                            self.v_proj.bias], dim=0)
            self._qkv_key = key
            self._qkv_generation += 1
        return self._qkv_weight, self._qkv_bias

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
                causal: bool = False, mask_is_trivial: bool = False,
                packing=None, residual: Optional[torch.Tensor] = None,
                norm: Optional["MyLayerNorm"] = None, norm_kind: str = "float"):
        """`x` is [B, S, D], or [2, B, S, D] split fp16 planes of it (the form
        a LayerNorm emits for the split QKV projection).

        With `packing` (an optimized.packing.RowPacking), `x` holds only the
        valid rows, [T_valid, D] or planes [2, T_valid, D]; attention runs over
        the packed sequences and the result is [T_valid, D], with no padded
        rows to zero.

        With `residual` (not on the masked padded path) the result is
        residual + out_proj(...), the add done in out_proj's epilogue; with
        `norm` as well, the pair (that sum, norm of it in form `norm_kind`),
        the LayerNorm in the same epilogue where the row is narrow enough.
        """
        if packing is not None:
            return self._forward_packed(x, causal, packing, residual, norm, norm_kind)
        split = x.dim() == 4
        batch, seq_len = (x.shape[1], x.shape[2]) if split else (x.shape[0], x.shape[1])
        qkv_w, qkv_b = self._get_qkv_weight()
        rows = batch * seq_len
        # fp16 q/k/v when attention contracts in fp16: the projection's
        # epilogue applies the RNE attention would apply while staging.
        want_half = (_attention_wants_fp16()
                     and config._QKV_FP16_MIN_ROWS <= rows <= config._LINEAR_BIAS_MAX_ROWS)
        if split and okernels._qkv_split_prefix:
            qkv = _linear_bias_split_prefix(x, qkv_w, qkv_b, want_half, okernels._qkv_split_prefix)
        elif split:
            qkv = _linear_bias_split(x, qkv_w, qkv_b, out_half=want_half)
        else:
            qkv = _linear_bias(x, qkv_w, qkv_b, out_half=want_half, math=_qkv_math_code())
        # [B, S, 3, H, hd] -> three strided [B, H, S, hd] views; no copies.
        q, k, v = (qkv.view(batch, seq_len, 3, self.num_heads, self.head_dim)
                   .permute(2, 0, 3, 1, 4).unbind(0))

        use_mask = valid_token_mask is not None and not mask_is_trivial
        # Key padding stays a [B, 1, 1, S] mask and causal stays a flag.
        attn_mask = valid_token_mask[:, None, None, :] if use_mask else None
        context = _attention_dispatch(q, k, v, attn_mask=attn_mask, is_causal=causal,
                                      scale=self.scale)
        if residual is not None and not use_mask:
            if norm is not None:
                return _linear_norm(context, self.out_proj, residual, norm, norm_kind)
            return _linear_bias(context, self.out_proj.weight, self.out_proj.bias,
                                residual=residual)
        output = self.out_proj(context)
        if use_mask:
            output = output.masked_fill(~valid_token_mask[..., None], 0)
        if residual is not None:
            output = residual + output
        return output

    def _forward_packed(self, x: torch.Tensor, causal: bool, packing,
                        residual: Optional[torch.Tensor] = None,
                        norm: Optional["MyLayerNorm"] = None, norm_kind: str = "float"):
        split = x.dim() == 3
        rows = packing.t_valid
        qkv_w, qkv_b = self._get_qkv_weight()
        want_half = (_attention_wants_fp16()
                     and config._QKV_FP16_MIN_ROWS <= rows <= config._LINEAR_BIAS_MAX_ROWS)
        if split:
            qkv = _linear_bias_split(x, qkv_w, qkv_b, out_half=want_half)
        else:
            qkv = _linear_bias(x, qkv_w, qkv_b, out_half=want_half, math=_qkv_math_code())
        # [T_valid, 3, H, hd] -> three strided [T_valid, H, hd] views.
        q, k, v = qkv.view(rows, 3, self.num_heads, self.head_dim).unbind(1)
        context = _attention_packed(q, k, v, packing, causal, self.scale)
        if residual is not None:
            if norm is not None:
                return _linear_norm(context, self.out_proj, residual, norm, norm_kind)
            return _linear_bias(context, self.out_proj.weight, self.out_proj.bias,
                                residual=residual)
        return self.out_proj(context)


class MyTransformerBlock(nn.Module):
    """BaselineTransformerBlock's submodule names (norm1, attention, norm2, ffn_in, ffn_out)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int, causal: bool) -> None:
        super().__init__()
        self.norm1 = MyLayerNorm(d_model)
        self.attention = MySelfAttention(d_model, num_heads)
        self.norm2 = MyLayerNorm(d_model)
        self.ffn_in = MyLinear(d_model, ffn_dim)
        self.ffn_out = MyLinear(ffn_dim, d_model)
        self.causal = causal

    def forward(self, x: torch.Tensor, normed: torch.Tensor, next_norm: "MyLayerNorm",
                valid_token_mask: Optional[torch.Tensor] = None, mask_is_trivial: bool = False,
                next_norm_is_output: bool = False,
                packing=None) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
        """Returns (residual stream, next_norm applied to it).

        `normed` is norm1(x), computed by whoever produced x; `next_norm` is
        the LayerNorm that consumes this block's output (the next block's
        norm1, or final_norm), so both residual adds fuse with a norm.

        With `packing`, x and normed hold the valid rows only ([T_valid, D];
        normed may be split planes) and so does the result, except when
        next_norm is the model's output norm: that one is returned in the
        padded [B, S, D] layout with zero padded rows, and the residual
        stream, which nothing reads after it, is not materialised (None).
        """
        if packing is not None:
            return self._forward_packed(x, normed, next_norm, next_norm_is_output, packing)
        use_mask = valid_token_mask is not None and not mask_is_trivial
        if not use_mask and self._residual_fused(x):
            return self._forward_residual_fused(x, normed, next_norm, next_norm_is_output)
        attn_out = self.attention(normed, valid_token_mask, self.causal, mask_is_trivial)

        if not use_mask:
            fused = _ffn_block(x, attn_out, self.norm2, self.ffn_in, self.ffn_out, next_norm)
            if fused is not None:
                return fused

        rows = x.numel() // x.shape[-1]
        x, normed = _add_layernorm(x, attn_out, self.norm2,
                                   normed_half=_gelu_input_wants_fp16(rows, x.shape[-1]))
        hidden = _linear_gelu(normed, self.ffn_in, out_half=_gelu_output_wants_fp16(rows))
        ffn_out = self.ffn_out(hidden)

        if use_mask:
            # The reference zeroes padded rows between the add and the norm.
            x = (x + ffn_out).masked_fill(~valid_token_mask[..., None], 0)
            if not next_norm_is_output:
                return x, next_norm(x)
            # the model zeroes the padded rows of this norm's output again,
            # so it is not the forward's output tensor
            return x, _final_norm(x, next_norm, output=False)

        if next_norm_is_output:
            # the model's output: the residual sum is not stored
            return None, _add_layernorm_output(x, ffn_out, next_norm)
        if _normed_split_wanted():
            return _add_layernorm_split(x, ffn_out, next_norm)
        trailing_half = _normed_wants_fp16(rows, x.shape[-1])
        return _add_layernorm(x, ffn_out, next_norm, normed_half=trailing_half)

    def _residual_fused(self, x: torch.Tensor) -> bool:
        """Run out_proj and ffn_out with the residual adds in their epilogues?
        Not where the fused FFN block will take the block's second half."""
        d_model, d_ff = x.shape[-1], self.ffn_in.weight.shape[0]
        rows = x.numel() // d_model
        # the epilogue is the pipelined kernel's: fp16 operands in (ctx from
        # attention, hidden from linear_gelu), K a multiple of 64
        return (x.dtype == torch.float32
                and _residual_epilogue_wanted(d_model) and _residual_epilogue_wanted(d_ff)
                and _attention_wants_fp16() and _gelu_output_wants_fp16(rows)
                and not _ffn_block_eligible(x, self.ffn_in, self.ffn_out))

    def _forward_residual_fused(self, x, normed, next_norm, next_norm_is_output, packing=None):
        """The block with h1 = x + out_proj(...) and h2 = h1 + ffn_out(...)
        formed in the GEMM epilogues (the same fp32 sums the add+LayerNorm
        kernels would form), each followed by its LayerNorm -- in the same
        epilogue where the rows are narrow enough (_linear_norm), else as a
        plain LayerNorm of h1 / h2; at d_model 256 the whole FFN with its add
        and LayerNorm is one kernel (_ffn_norm). Outputs are bit-identical to
        the add+LayerNorm chain."""
        rows = x.numel() // x.shape[-1]
        width = x.shape[-1]
        kind2 = "half" if _gelu_input_wants_fp16(rows, width) else "float"
        h1, normed2 = self.attention(normed, None, self.causal, True, packing=packing, residual=x,
                                     norm=self.norm2, norm_kind=kind2)
        if next_norm_is_output:
            # the model's output: never narrowed; the sum is not read after it
            h2, out = _ffn_norm(normed2, self.ffn_in, self.ffn_out, h1, next_norm, "float",
                                store_out=False, packing=packing, output=True)
            return (None if packing is not None else h2), out
        if _normed_split_wanted():
            kind = "split"
        else:
            kind = "half" if _normed_wants_fp16(rows, width) else "float"
        return _ffn_norm(normed2, self.ffn_in, self.ffn_out, h1, next_norm, kind)

    def _forward_packed(self, x, normed, next_norm, next_norm_is_output, packing):
        if self._residual_fused(x):
            return self._forward_residual_fused(x, normed, next_norm, next_norm_is_output,
                                                packing)
        attn_out = self.attention(normed, None, self.causal, True, packing=packing)
        if not next_norm_is_output:
            fused = _ffn_block(x, attn_out, self.norm2, self.ffn_in, self.ffn_out, next_norm)
            if fused is not None:
                return fused
        rows, width = packing.t_valid, x.shape[-1]
        x, normed = _add_layernorm(x, attn_out, self.norm2,
                                   normed_half=_gelu_input_wants_fp16(rows, width))
        hidden = _linear_gelu(normed, self.ffn_in, out_half=_gelu_output_wants_fp16(rows))
        ffn_out = self.ffn_out(hidden)
        if next_norm_is_output:
            return None, _add_layernorm_unpack(x, ffn_out, next_norm, packing)
        if _normed_split_wanted():
            return _add_layernorm_split(x, ffn_out, next_norm)
        return _add_layernorm(x, ffn_out, next_norm,
                              normed_half=_normed_wants_fp16(rows, width))


def _final_norm(x: torch.Tensor, norm: "MyLayerNorm", output: bool = True) -> torch.Tensor:
    """The model's output norm: never narrowed. `output`: its result is the
    forward's output tensor (bound to a captured graph's output slot)."""
    return _layernorm(x, norm, out_half=False, output=output)
