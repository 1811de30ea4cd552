"""fp64 brute-force restatements used to pin oracle.layer on tiny shapes.

Each op is written from its definition with explicit loops (or the textbook
closed form), independent of torch, so a dropped term, a wrong sign or index
or a transposed operand in oracle.layer shows up as a mismatch:

  layer_norm  mean and biased variance per row, eps inside the sqrt
              (nn.LayerNorm semantics, torch_transformer_benchmark.py:225-226)
  linear      y[i, o] = sum_k x[i, k] * W[o, k] + b[o]   (nn.Linear, :83-86)
  gelu        0.5 x (1 + erf(x / sqrt 2))                (F.gelu exact, :241)
  attention   per (b, h, i): scores over keys j, -inf where j > i (causal) or
              the key is invalid, max-subtracted softmax, weighted sum of V;
              a row with no valid key gives 0 (the kernels' convention)
  layer       pre-LN block + final norm + padded-row zeroing (:234-245, :262-272)
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    D = x.shape[-1]
    flat = x.reshape(-1, D)
    of = out.reshape(-1, D)
    for r in range(flat.shape[0]):
        row = flat[r]
        mean = 0.0
        for v in row:
            mean += v
        mean /= D
        var = 0.0
        for v in row:
            var += (v - mean) * (v - mean)
        var /= D
        inv = 1.0 / math.sqrt(var + eps)
        for c in range(D):
            of[r, c] = (row[c] - mean) * inv * float(w[c]) + float(b[c])
    return out


def linear(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray]) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    K = x.shape[-1]
    O = w.shape[0]
    flat = x.reshape(-1, K)
    out = np.zeros((flat.shape[0], O), dtype=np.float64)
    for i in range(flat.shape[0]):
        for o in range(O):
            acc = 0.0
            for k in range(K):
                acc += flat[i, k] * w[o, k]
            out[i, o] = acc + (0.0 if b is None else float(b[o]))
    return out.reshape(*x.shape[:-1], O)


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    f = np.vectorize(lambda v: 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))))
    return f(x) if x.size else x.copy()


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, valid_keys=None,
              causal: bool = False, scale: Optional[float] = None) -> np.ndarray:
    """q, k, v [B, H, S, hd] -> [B, H, S, hd], fp64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, S, hd = q.shape
    if scale is None:
        scale = hd ** -0.5
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for i in range(S):
                s = []
                for j in range(S):
                    ok = True
                    if causal and j > i:
                        ok = False
                    if valid_keys is not None and not valid_keys[b, j]:
                        ok = False
                    if ok:
                        acc = 0.0
                        for d in range(hd):
                            acc += q[b, h, i, d] * k[b, h, j, d]
                        s.append((j, acc * scale))
                if not s:
                    continue
                m = max(val for _, val in s)
                e = [(j, math.exp(val - m)) for j, val in s]
                z = sum(val for _, val in e)
                for j, p in e:
                    out[b, h, i, :] += (p / z) * v[b, h, j, :]
    return out


def block(x: np.ndarray, valid: Optional[np.ndarray], params: Dict[str, np.ndarray],
          prefix: str, num_heads: int, causal: bool) -> np.ndarray:
    """One pre-LN block (BaselineTransformerBlock.forward, :234-245), fp64,
    from the ops above: x + attn(norm1 x), + ffn(norm2 .), padded rows zeroed."""
    p = {k: np.asarray(v, dtype=np.float64) for k, v in params.items()}
    x = np.asarray(x, dtype=np.float64)
    B, S, D = x.shape
    hd = D // num_heads
    pre = prefix

    def heads(t):
        return t.reshape(B, S, num_heads, hd).transpose(0, 2, 1, 3)

    n1 = layer_norm(x, p[pre + "norm1.weight"], p[pre + "norm1.bias"])
    a = pre + "attention."
    q = heads(linear(n1, p[a + "q_proj.weight"], p[a + "q_proj.bias"]))
    k = heads(linear(n1, p[a + "k_proj.weight"], p[a + "k_proj.bias"]))
    v = heads(linear(n1, p[a + "v_proj.weight"], p[a + "v_proj.bias"]))
    ctx = attention(q, k, v, valid, causal).transpose(0, 2, 1, 3).reshape(B, S, D)
    att = linear(ctx, p[a + "out_proj.weight"], p[a + "out_proj.bias"])
    if valid is not None:
        att = np.where(valid[..., None], att, 0.0)
    h = x + att
    n2 = layer_norm(h, p[pre + "norm2.weight"], p[pre + "norm2.bias"])
    f = linear(gelu(linear(n2, p[pre + "ffn_in.weight"], p[pre + "ffn_in.bias"])),
               p[pre + "ffn_out.weight"], p[pre + "ffn_out.bias"])
    h = h + f
    if valid is not None:
        h = np.where(valid[..., None], h, 0.0)
    return h


def model(x: np.ndarray, valid: Optional[np.ndarray], params: Dict[str, np.ndarray],
          num_heads: int, causal: bool, num_layers: int = 1) -> np.ndarray:
    """`num_layers` blocks (layers.0. .. layers.{L-1}.), then the final norm
    and the padded-row zeroing (BaselineTransformer.forward, :262-272)."""
    h = np.asarray(x, dtype=np.float64)
    for i in range(num_layers):
        h = block(h, valid, params, f"layers.{i}.", num_heads, causal)
    out = layer_norm(h, np.asarray(params["final_norm.weight"], dtype=np.float64),
                     np.asarray(params["final_norm.bias"], dtype=np.float64))
    if valid is not None:
        out = np.where(valid[..., None], out, 0.0)
    return out


def layer(x: np.ndarray, valid: Optional[np.ndarray], params: Dict[str, np.ndarray],
          num_heads: int, causal: bool) -> np.ndarray:
    """One pre-LN block plus final norm, fp64, from the ops above."""
    return model(x, valid, params, num_heads, causal, 1)
