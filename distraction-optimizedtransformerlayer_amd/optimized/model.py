"""The optimized transformer (reference optimized/model.py:1-277)."""

from __future__ import annotations

import weakref
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import config
from .graphs import _GraphRunner, _capture_graph, _graph_eligible, _graph_key, _graph_note_decline
from .layers import MyLayerNorm, MyTransformerBlock
from .util import _version_or_none


class OptimizedTransformer(nn.Module):
    """BaselineTransformer's forward on the gfx950 kernels.

    Parameter and submodule names match BaselineTransformer
    (torch_transformer_benchmark.py:248-272), so copy_model_weights() loads one
    state_dict into either with strict=True. A harness mixes it in as
    `class UserOptimizedTransformer(OptimizedTransformer, BaselineTransformer)`;
    BaselineTransformer.__init__ is deliberately not called.
    """

    def __init__(self, config_) -> None:
        nn.Module.__init__(self)
        self.config = config_
        self.layers = nn.ModuleList([
            MyTransformerBlock(config_.d_model, config_.num_heads, config_.ffn_dim,
                               config_.causal)
            for _ in range(config_.num_layers)
        ])
        self.final_norm = MyLayerNorm(config_.d_model)
        # Trivial-mask memo, graph cache and chunk-size cache: plain
        # attributes, out of state_dict().
        self._triv_ref: Optional[weakref.ReferenceType] = None
        self._triv_version: Optional[int] = None
        self._triv: bool = False
        self._graphs: Dict[Tuple, _GraphRunner] = {}
        self._graph_denied: set = set()
        self._chunk_rows: Dict[Tuple, int] = {}
        self._device_budget: Optional[int] = None

    def _mask_is_trivial(self, mask: Optional[torch.Tensor]) -> bool:
        """True when every position is valid. One D2H sync per new mask object.

        Keyed on a weakref (a live weakref proves the object was never freed,
        unlike a recycled data_ptr) plus the version counter.
        """
        if mask is None:
            return False
        version = _version_or_none(mask)
        cached = self._triv_ref() if self._triv_ref is not None else None
        if cached is mask and self._triv_version == version:
            return self._triv
        self._triv = bool(mask.all().item())
        self._triv_ref = weakref.ref(mask)
        self._triv_version = version
        return self._triv

    def _forward_eager(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                       use_mask: bool) -> torch.Tensor:
        """The whole model with every host decision already made: capturable.

        No device->host reads and no lazily built state that outlives the call
        (graph capture's warmup builds those first).
        """
        normed = self.layers[0].norm1(x)
        last = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            next_norm = self.final_norm if index == last else self.layers[index + 1].norm1
            x, normed = layer(x, normed, next_norm, valid_token_mask, not use_mask,
                              index == last)
        if use_mask:
            normed = normed.masked_fill(~valid_token_mask[..., None], 0)
        return normed

    def forward(self, x: torch.Tensor,
                valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        mask_is_trivial = self._mask_is_trivial(valid_token_mask)
        use_mask = valid_token_mask is not None and not mask_is_trivial
        key = _graph_key(x, use_mask)
        runner = self._graphs.get(key)
        if runner is None:
            runner = self._maybe_capture(key, x, valid_token_mask, use_mask)
        if runner is not None:
            return runner.replay(x, valid_token_mask)
        if config.MICROBATCH_FALLBACK and x.is_cuda and x.shape[0] > 1:
            return self._forward_chunk_on_oom(x, valid_token_mask, use_mask)
        return self._forward_eager(x, valid_token_mask, use_mask)

    def _rows_within_budget(self, x: torch.Tensor) -> int:
        """Batch rows whose predicted peak fits the device budget."""
        rows = x.shape[0]
        per_row = x.shape[1] * x.shape[2] * x.element_size() * config._MICROBATCH_PEAK_FACTOR
        if per_row <= 0:
            return rows
        if self._device_budget is None:
            _, total = torch.cuda.mem_get_info(x.device)
            self._device_budget = int(total * config._MICROBATCH_BUDGET_FRACTION)
        if per_row * rows <= self._device_budget:
            return rows
        return max(config._MICROBATCH_MIN_ROWS, min(rows, self._device_budget // per_row))

    def _forward_chunk_on_oom(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                              use_mask: bool) -> torch.Tensor:
        """_forward_eager, retried over halving batch chunks on out-of-memory.

        The chunk size that worked is cached per shape, so results stay stable
        across calls (reference optimized/model.py:194-246).
        """
        rows = x.shape[0]
        key = (rows, x.shape[1], x.shape[2], x.dtype, use_mask)
        n = self._chunk_rows.get(key)
        if n is None:
            n = self._rows_within_budget(x)
        if n >= rows:
            try:
                return self._forward_eager(x, valid_token_mask, use_mask)
            except torch.OutOfMemoryError:
                torch.cuda.empty_cache()
                n = rows // 2
        while n >= config._MICROBATCH_MIN_ROWS:
            out = None
            try:
                out = torch.empty_like(x)
                for lo in range(0, rows, n):
                    hi = min(lo + n, rows)
                    chunk_mask = valid_token_mask[lo:hi] if valid_token_mask is not None else None
                    out[lo:hi] = self._forward_eager(x[lo:hi], chunk_mask, use_mask)
                self._chunk_rows[key] = n
                return out
            except torch.OutOfMemoryError:
                del out
                torch.cuda.empty_cache()
                if n <= config._MICROBATCH_MIN_ROWS:
                    raise
                n //= 2
        return self._forward_eager(x, valid_token_mask, use_mask)

    def _maybe_capture(self, key: Tuple, x: torch.Tensor,
                       valid_token_mask: Optional[torch.Tensor],
                       use_mask: bool) -> Optional[_GraphRunner]:
        """Capture a graph for this key, or decide not to (failures are remembered)."""
        if key in self._graph_denied:
            return None
        if not _graph_eligible(x, len(self._graphs)):
            _graph_note_decline(x)
            return None
        runner = _capture_graph(self, x, valid_token_mask, use_mask)
        if runner is None:
            self._graph_denied.add(key)
            return None
        self._graphs[key] = runner
        return runner
