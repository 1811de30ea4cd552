"""Seeded synthetic inputs for the five layer configs, bit-identical everywhere.

The reference harness draws its inputs with torch's device generator
(`generate_random_case`, torch_transformer_benchmark.py:500-540) and its
weights from nn.Linear's default init (:83-86, 231-232). The configs this
build is measured on ask instead for Xavier-uniform weights, zero biases and
LayerNorm gamma=1 / beta=0, drawn from a fixed seed, so the stream here is our
own: numpy's PCG64, which gives the same bits on any machine and any torch
version. What is kept from the harness is the *meaning* of each draw:

  * x ~ N(0, 1) * input_scale                       (:516-524)
  * lengths inclusive of S, valid[b, s] = s < len_b  (:530-538)
  * padded rows of x are zeroed                      (:539)

Generation order is fixed: x, then Wq, Wk, Wv, Wo, W1, W2, then the lengths.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

SEED_BASE = 1234  # the harness default --seed (torch_transformer_benchmark.py:1079)


@dataclass(frozen=True)
class LayerConfig:
    """One BASELINE config. Field names follow TransformerConfig (:42-49)."""

    name: str
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    causal: bool
    # "none" or "keypad": a [B, S] bool key-padding mask from drawn lengths
    mask: str
    # valid lengths are drawn uniformly from [len_lo, seq_len], inclusive
    len_lo: int
    input_scale: float
    seed_offset: int

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def tokens(self) -> int:
        return self.batch_size * self.seq_len


CONFIGS: Dict[str, LayerConfig] = {
    "C1": LayerConfig("C1", 2, 64, 128, 4, 512, False, "none", 64, 1.0, 0),
    "C2": LayerConfig("C2", 8, 512, 512, 8, 2048, False, "keypad", 256, 1.0, 1),
    "C3": LayerConfig("C3", 1, 4096, 1024, 16, 4096, True, "none", 4096, 1.0, 2),
    "C4": LayerConfig("C4", 4, 2048, 2048, 16, 8192, False, "none", 2048, 0.5, 3),
    "C5": LayerConfig("C5", 10000, 16, 256, 4, 1024, False, "keypad", 1, 1.0, 4),
}

# Parameter names, in state_dict order, of BaselineTransformer(num_layers=1)
# (torch_transformer_benchmark.py:222-272). They are the weight format: the
# optimized model loads the same dict with strict=True.
PARAM_NAMES = (
    "layers.0.norm1.weight", "layers.0.norm1.bias",
    "layers.0.attention.q_proj.weight", "layers.0.attention.q_proj.bias",
    "layers.0.attention.k_proj.weight", "layers.0.attention.k_proj.bias",
    "layers.0.attention.v_proj.weight", "layers.0.attention.v_proj.bias",
    "layers.0.attention.out_proj.weight", "layers.0.attention.out_proj.bias",
    "layers.0.norm2.weight", "layers.0.norm2.bias",
    "layers.0.ffn_in.weight", "layers.0.ffn_in.bias",
    "layers.0.ffn_out.weight", "layers.0.ffn_out.bias",
    "final_norm.weight", "final_norm.bias",
)


def xavier_uniform(rng: np.random.Generator, out_features: int,
                   in_features: int) -> np.ndarray:
    """U(-a, a) with a = sqrt(6 / (fan_in + fan_out)), shape [out, in]."""
    a = float(np.sqrt(6.0 / (in_features + out_features)))
    return rng.uniform(-a, a, size=(out_features, in_features)).astype(np.float32)


def make_case(cfg: LayerConfig, seed: Optional[int] = None,
              batch: Optional[int] = None, nonzero_affine: bool = False):
    """Draw (x, valid_mask, params) for one config.

    x          float32 [B, S, D]
    valid_mask bool [B, S] (True = valid token) or None when cfg.mask == "none"
    params     dict name -> float32 array, keyed by PARAM_NAMES

    `batch` overrides B (the first `batch` rows of the same stream are NOT the
    same as a smaller draw; it is a separate, smaller case). `nonzero_affine`
    replaces the zero biases and unit/zero LayerNorm affine with seeded
    non-trivial values, drawn after everything else, so the bias and affine
    paths are exercised.
    """
    s = SEED_BASE + cfg.seed_offset if seed is None else seed
    rng = np.random.Generator(np.random.PCG64(s))
    B = cfg.batch_size if batch is None else batch
    S, D, F = cfg.seq_len, cfg.d_model, cfg.ffn_dim

    x = rng.standard_normal((B, S, D), dtype=np.float32)
    if cfg.input_scale != 1.0:
        x = (x * np.float32(cfg.input_scale)).astype(np.float32)

    wq = xavier_uniform(rng, D, D)
    wk = xavier_uniform(rng, D, D)
    wv = xavier_uniform(rng, D, D)
    wo = xavier_uniform(rng, D, D)
    w1 = xavier_uniform(rng, F, D)
    w2 = xavier_uniform(rng, D, F)

    mask = None
    if cfg.mask == "keypad":
        lengths = rng.integers(cfg.len_lo, S + 1, size=B)
        mask = np.arange(S)[None, :] < lengths[:, None]
        x = np.where(mask[..., None], x, np.float32(0)).astype(np.float32)

    zeros = lambda n: np.zeros(n, dtype=np.float32)  # noqa: E731
    ones = lambda n: np.ones(n, dtype=np.float32)  # noqa: E731
    params = {
        "layers.0.norm1.weight": ones(D), "layers.0.norm1.bias": zeros(D),
        "layers.0.attention.q_proj.weight": wq, "layers.0.attention.q_proj.bias": zeros(D),
        "layers.0.attention.k_proj.weight": wk, "layers.0.attention.k_proj.bias": zeros(D),
        "layers.0.attention.v_proj.weight": wv, "layers.0.attention.v_proj.bias": zeros(D),
        "layers.0.attention.out_proj.weight": wo, "layers.0.attention.out_proj.bias": zeros(D),
        "layers.0.norm2.weight": ones(D), "layers.0.norm2.bias": zeros(D),
        "layers.0.ffn_in.weight": w1, "layers.0.ffn_in.bias": zeros(F),
        "layers.0.ffn_out.weight": w2, "layers.0.ffn_out.bias": zeros(D),
        "final_norm.weight": ones(D), "final_norm.bias": zeros(D),
    }
    if nonzero_affine:
        for name in PARAM_NAMES:
            if name.endswith(".bias"):
                n = params[name].shape[0]
                params[name] = (0.1 * rng.standard_normal(n)).astype(np.float32)
            elif "norm" in name:
                n = params[name].shape[0]
                params[name] = (1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    return x, mask, params


def lengths_of(mask: Optional[np.ndarray], cfg: LayerConfig, batch: int) -> np.ndarray:
    """Valid length per sequence (all S when there is no mask)."""
    if mask is None:
        return np.full(batch, cfg.seq_len, dtype=np.int64)
    return mask.sum(axis=1).astype(np.int64)


def attention_useful_flops(cfg: LayerConfig, lengths: np.ndarray) -> float:
    """4 * hd * H * sum_b pairs_b: valid query x valid key (key <= query if causal)."""
    L = lengths.astype(np.float64)
    if cfg.causal:
        pairs = L * (L + 1) / 2.0
    else:
        pairs = L * L
    return 4.0 * cfg.head_dim * cfg.num_heads * float(pairs.sum())


def gemm_flops(cfg: LayerConfig, rows: Optional[int] = None) -> float:
    """8 T D^2 + 4 T D F: QKV (6TD^2) + out_proj (2TD^2) + two FFN GEMMs.

    `rows` replaces T = B*S by the number of rows that carry work: a padded
    batch's valid rows (sum of the lengths), the rows whose outputs survive
    the reference's masked_fill of padded rows.
    """
    T = cfg.tokens if rows is None else int(rows)
    D, F = cfg.d_model, cfg.ffn_dim
    return 8.0 * T * D * D + 4.0 * T * D * F


def layernorm_bytes(cfg: LayerConfig, normed_bytes: int = 4) -> float:
    """One plain LN (read x, write normed) + two add+LN (read x, sub; write x_new, normed)."""
    T, D = cfg.tokens, cfg.d_model
    return float(T * D * ((4 + normed_bytes) + 2 * (12 + normed_bytes)))


def stack_layers(params: Dict[str, np.ndarray], num_layers: int,
                 seed: Optional[int] = None) -> Dict[str, np.ndarray]:
    """A `num_layers`-block weight dict whose block 0 and final norm are `params`'.

    Blocks 1 .. L-1 get their own Xavier-uniform weights (zero biases, unit /
    zero LayerNorm affine, as block 0 under the configs' spec), drawn from a
    PCG64 stream seeded by `seed` (default: derived from block 0's first
    weight, so a config always stacks the same way). Key names follow the
    reference's state_dict (layers.{i}.*).
    """
    if num_layers == 1:
        return dict(params)
    wq0 = params["layers.0.attention.q_proj.weight"]
    D = wq0.shape[0]
    F = params["layers.0.ffn_in.weight"].shape[0]
    if seed is None:
        seed = SEED_BASE + int(np.float64(wq0[0, 0]).view(np.uint64) % (1 << 31))
    rng = np.random.Generator(np.random.PCG64(seed))
    out = dict(params)
    for i in range(1, num_layers):
        pre = f"layers.{i}."
        out[pre + "norm1.weight"] = np.ones(D, dtype=np.float32)
        out[pre + "norm1.bias"] = np.zeros(D, dtype=np.float32)
        for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
            out[pre + f"attention.{name}.weight"] = xavier_uniform(rng, D, D)
            out[pre + f"attention.{name}.bias"] = np.zeros(D, dtype=np.float32)
        out[pre + "norm2.weight"] = np.ones(D, dtype=np.float32)
        out[pre + "norm2.bias"] = np.zeros(D, dtype=np.float32)
        out[pre + "ffn_in.weight"] = xavier_uniform(rng, F, D)
        out[pre + "ffn_in.bias"] = np.zeros(F, dtype=np.float32)
        out[pre + "ffn_out.weight"] = xavier_uniform(rng, D, F)
        out[pre + "ffn_out.bias"] = np.zeros(D, dtype=np.float32)
    return out
