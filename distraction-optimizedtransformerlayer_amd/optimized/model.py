"""The optimized transformer (reference optimized/model.py:1-277)."""

from __future__ import annotations

import weakref
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import config
from .graphs import _GraphRunner, _capture_graph, _graph_eligible, _graph_key, _graph_note_decline
from .kernels import _layernorm_pack
from .layers import MyLayerNorm, MyTransformerBlock
from .packing import RowPacking, build_packing
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
        self._packing: Optional[RowPacking] = None
        self._graphs: Dict[Tuple, _GraphRunner] = {}
        self._graph_denied: set = set()
        self._chunk_rows: Dict[Tuple, int] = {}
        self._device_budget: Optional[int] = None

    def _mask_packing(self, mask: Optional[torch.Tensor]) -> Optional[RowPacking]:
        """The mask's RowPacking, built once per mask object (one D2H sync).

        Keyed on a weakref (a live weakref proves the object was never freed,
        unlike a recycled data_ptr) plus the version counter, as the
        reference keys its trivial-mask memo (reference optimized/model.py:68-93).
        """
        if mask is None:
            return None
        version = _version_or_none(mask)
        cached = self._triv_ref() if self._triv_ref is not None else None
        if cached is mask and self._triv_version == version and self._packing is not None:
            return self._packing
        self._packing = build_packing(mask)
        self._triv_ref = weakref.ref(mask)
        self._triv_version = version
        return self._packing

    def _mask_is_trivial(self, mask: Optional[torch.Tensor]) -> bool:
        """True when every position is valid (so every mask op is a no-op)."""
        packing = self._mask_packing(mask)
        return packing is not None and packing.trivial

    def _forward_eager(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                       use_mask: bool, packing: Optional[RowPacking] = None) -> torch.Tensor:
        """The whole model with every host decision already made: capturable.

        No device->host reads and no lazily built state that outlives the call
        (graph capture's warmup builds those first). With `packing` the layers
        run on the valid rows only (optimized/packing.py) and the mask itself
        is not read.
        """
        if packing is not None:
            return self._forward_packed(x, packing)
        normed = self.layers[0].norm1(x)
        last = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            next_norm = self.final_norm if index == last else self.layers[index + 1].norm1
            x, normed = layer(x, normed, next_norm, valid_token_mask, not use_mask,
                              index == last)
        if use_mask:
            normed = normed.masked_fill(~valid_token_mask[..., None], 0)
        return normed

    def _forward_packed(self, x: torch.Tensor, packing: RowPacking) -> torch.Tensor:
        """Gather the valid rows (fused into the first LayerNorm), run every
        layer on them, and scatter back in the last add+LayerNorm, which also
        writes the padded rows' zeros."""
        x, normed = _layernorm_pack(x, self.layers[0].norm1, packing)
        last = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            next_norm = self.final_norm if index == last else self.layers[index + 1].norm1
            x, normed = layer(x, normed, next_norm, None, True, index == last, packing=packing)
        return normed

    def forward(self, x: torch.Tensor,
                valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        packing = self._mask_packing(valid_token_mask)
        use_mask = packing is not None and not packing.trivial
        if not (use_mask and config.ROW_PACKING != "off" and x.is_cuda):
            packing = None
        key = _graph_key(x, use_mask, packing)
        runner = self._graphs.get(key)
        if runner is None:
            runner = self._maybe_capture(key, x, valid_token_mask, use_mask, packing)
        if runner is not None:
            return runner.replay(x, valid_token_mask, packing)
        if config.MICROBATCH_FALLBACK and x.is_cuda and x.shape[0] > 1:
            return self._forward_chunk_on_oom(x, valid_token_mask, use_mask, packing)
        return self._forward_eager(x, valid_token_mask, use_mask, packing)

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
                              use_mask: bool,
                              packing: Optional[RowPacking] = None) -> torch.Tensor:
        """_forward_eager, retried over halving batch chunks on out-of-memory.

        The chunk size that worked is cached per shape, so results stay stable
        across calls (reference optimized/model.py:194-246). Chunks run the
        padded path: a packing covers the whole batch.
        """
        rows = x.shape[0]
        key = (rows, x.shape[1], x.shape[2], x.dtype, use_mask)
        n = self._chunk_rows.get(key)
        if n is None:
            n = self._rows_within_budget(x)
        if n >= rows:
            try:
                return self._forward_eager(x, valid_token_mask, use_mask, packing)
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
                       use_mask: bool,
                       packing: Optional[RowPacking] = None) -> Optional[_GraphRunner]:
        """Capture a graph for this key, or decide not to (failures are remembered)."""
        if key in self._graph_denied:
            return None
        if not _graph_eligible(x, len(self._graphs)):
            _graph_note_decline(x)
            return None
        runner = _capture_graph(self, x, valid_token_mask, use_mask, packing)
        if runner is None:
            self._graph_denied.add(key)
            return None
        self._graphs[key] = runner
        return runner
