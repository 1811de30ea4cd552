"""Build an OptimizedTransformer from a config and a weight dict.

The reference builds its models inside the harness
(torch_transformer_benchmark.py:42-66 for TransformerConfig, :292-302 for
copy_model_weights with strict=True, :1181-1194 for the device move). This is
the same sequence for callers that are not the harness: the tests, bench.py
and the build smoke check.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np
import torch

from optimized import OptimizedTransformer


@dataclass(frozen=True)
class TransformerConfig:
    """The reference harness's model config (torch_transformer_benchmark.py:42-66)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(f"d_model ({self.d_model}) must be divisible by "
                             f"num_heads ({self.num_heads})")


def build_model(cfg: TransformerConfig, params: Dict[str, np.ndarray],
                device: str = "cuda") -> OptimizedTransformer:
    """OptimizedTransformer with `params` loaded strictly, moved to `device`, eval()."""
    cfg.validate()
    model = OptimizedTransformer(cfg)
    state = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in params.items()}
    model.load_state_dict(state, strict=True)
    return model.to(device=device, dtype=torch.float32).eval()


def to_device(x: np.ndarray, mask: Optional[np.ndarray], device: str = "cuda"):
    """Host arrays -> (x fp32, mask bool or None) on the device."""
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(device)
    mt = None if mask is None else torch.from_numpy(np.ascontiguousarray(mask)).to(device)
    return xt, mt
