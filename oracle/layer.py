"""The reference layer, restated on the CPU in torch.

Follows BaselineTransformer op for op, for as many blocks as the weight dict
holds (torch_transformer_benchmark.py):

  attention   :96-133   q/k/v projections, split heads, scores * hd^-1/2,
                        causal triu(1) -> -inf, key mask -> -inf, fp32 softmax,
                        P @ V, merge heads, out_proj, masked_fill padded rows
  block       :234-245  x + attn(norm1(x)); x + ffn_out(gelu_erf(ffn_in(norm2(x))));
                        masked_fill padded rows
  model       :262-272  every block in order, final_norm, masked_fill padded rows

The reference arithmetic is PyTorch's own (nn.Linear, nn.LayerNorm,
torch.matmul, torch.softmax, F.gelu), so the restatement calls the same
functional forms. `dtype` is float32 for the parity oracle (exact fp32 on the
CPU; stricter than the harness's TF32-on GPU baseline, :1095-1104) or float64
for the pinning checks.

`norm_first=False` gives the post-LN reading of the same block
(x = LN1(x + attn(x)); x = LN2(x + ffn(x))), kept so the ambiguity in the
config text can be graded with the same kernels; the reference code is pre-LN.
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F

from .inputs import LayerConfig


def _t(a, dtype):
    if isinstance(a, torch.Tensor):
        return a.to(dtype)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype)


def layer_norm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor,
               eps: float = 1e-5) -> torch.Tensor:
    """nn.LayerNorm over the last dim: biased variance, eps inside the sqrt."""
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    """nn.Linear: x @ w^T + b, w in [out, in] layout."""
    return F.linear(x, w, b)


def gelu(x: torch.Tensor) -> torch.Tensor:
    """Exact erf GELU (approximate="none"), as the block uses (:241)."""
    return F.gelu(x, approximate="none")


def attention(x: torch.Tensor, p: Dict[str, torch.Tensor], prefix: str,
              num_heads: int, valid: Optional[torch.Tensor], causal: bool) -> torch.Tensor:
    """BaselineSelfAttention.forward (:96-133)."""
    B, S, D = x.shape
    hd = D // num_heads
    scale = hd ** -0.5

    def split(t):
        return t.view(B, S, num_heads, hd).transpose(1, 2).contiguous()

    q = split(linear(x, p[prefix + "q_proj.weight"], p[prefix + "q_proj.bias"]))
    k = split(linear(x, p[prefix + "k_proj.weight"], p[prefix + "k_proj.bias"]))
    v = split(linear(x, p[prefix + "v_proj.weight"], p[prefix + "v_proj.bias"]))

    scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
    if causal:
        tri = torch.ones((S, S), dtype=torch.bool).triu(diagonal=1)
        scores = scores.masked_fill(tri, float("-inf"))
    if valid is not None:
        scores = scores.masked_fill(~valid[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    del scores
    ctx = torch.matmul(probs, v)
    del probs
    ctx = ctx.transpose(1, 2).contiguous().view(B, S, D)
    out = linear(ctx, p[prefix + "out_proj.weight"], p[prefix + "out_proj.bias"])
    if valid is not None:
        out = out.masked_fill(~valid[..., None], 0)
    return out


def num_layers_of(params: Dict) -> int:
    """Blocks a state dict holds (layers.0. .. layers.{L-1}.)."""
    return 1 + max(int(k.split(".")[1]) for k in params if k.startswith("layers."))


def reference_layer(x, valid, params, cfg: LayerConfig, dtype=torch.float32,
                    norm_first: bool = True, threads: Optional[int] = None) -> torch.Tensor:
    """BaselineTransformer.forward(x, valid) on the CPU.

    x       [B, S, D] array or tensor; valid [B, S] bool or None
    params  name -> array, keyed as the reference's state_dict; every block
            it holds (layers.0. .. layers.{L-1}.) runs, in order, then the
            final norm (reference :262-272)
    returns [B, S, D] tensor of `dtype`
    """
    if threads is not None:
        torch.set_num_threads(threads)
    with torch.inference_mode():
        p = {k: _t(v, dtype) for k, v in params.items()}
        h = _t(x, dtype)
        m = None if valid is None else _t(valid, torch.bool)
        for i in range(num_layers_of(params)):
            pre = f"layers.{i}."
            if norm_first:
                h = h + attention(layer_norm(h, p[pre + "norm1.weight"], p[pre + "norm1.bias"]),
                                  p, pre + "attention.", cfg.num_heads, m, cfg.causal)
                n2 = layer_norm(h, p[pre + "norm2.weight"], p[pre + "norm2.bias"])
                h = h + linear(gelu(linear(n2, p[pre + "ffn_in.weight"],
                                           p[pre + "ffn_in.bias"])),
                               p[pre + "ffn_out.weight"], p[pre + "ffn_out.bias"])
            else:
                h = layer_norm(h + attention(h, p, pre + "attention.", cfg.num_heads, m,
                                             cfg.causal),
                               p[pre + "norm1.weight"], p[pre + "norm1.bias"])
                f = linear(gelu(linear(h, p[pre + "ffn_in.weight"], p[pre + "ffn_in.bias"])),
                           p[pre + "ffn_out.weight"], p[pre + "ffn_out.bias"])
                h = layer_norm(h + f, p[pre + "norm2.weight"], p[pre + "norm2.bias"])
            if m is not None:
                h = h.masked_fill(~m[..., None], 0)
        out = layer_norm(h, p["final_norm.weight"], p["final_norm.bias"])
        if m is not None:
            out = out.masked_fill(~m[..., None], 0)
        return out


def reference_attention(q, k, v, valid_keys=None, causal=False, scale=None,
                        dtype=torch.float32) -> torch.Tensor:
    """Attention op alone, [B, H, S, hd] in and out, the baseline's arithmetic.

    A fully masked query row gives NaN in the baseline's softmax; the kernels'
    convention (l == 0 -> 0 output, attention_wmma.cuh:1724-1733, and
    verify_kernel.py:84-85's nan_to_num) is applied here so the two compare.
    `valid_keys` is a [B, S] bool key mask (True = may be attended).
    """
    q, k, v = (_t(t, dtype) for t in (q, k, v))
    S = q.shape[2]
    if scale is None:
        scale = q.shape[-1] ** -0.5
    scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
    if causal:
        tri = torch.ones((S, S), dtype=torch.bool).triu(diagonal=1)
        scores = scores.masked_fill(tri, float("-inf"))
    if valid_keys is not None:
        vk = _t(valid_keys, torch.bool)
        scores = scores.masked_fill(~vk[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    out = torch.matmul(probs, v)
    return torch.nan_to_num(out, nan=0.0)
