"""Packed valid rows of a padded batch.

The reference runs every layer over all B*S rows of a padded batch and
zeroes the padded rows three times with masked_fill: after attention, after
the block, after the final norm (reference optimized/layers.py:185-189,
247-252; optimized/model.py:141-142). None of those rows reaches a valid
output:

  * every kernel except attention is row-local, so a valid row's LayerNorm,
    projections and FFN never read a padded row;
  * attention reads padded rows only as keys, and the key mask gives them
    probability 0;
  * the padded rows of the output are zero, whatever was computed for them.

So the layer can run on the T_valid valid rows alone. The first LayerNorm
gathers them (RowPacking.idx), attention runs over packed sequences
(RowPacking.cu), and the final add+LayerNorm scatters back, writing zero rows
for the padding (RowPacking.inv). On a prefix mask (valid[b, s] = s < len_b,
the padded-batch configs), each sequence's keys are tiled from its first row
in both layouts, so the valid rows come out bit-identical to the padded
computation. The padded rows' work is skipped: about a quarter of C2's
layer and half of C5's.

Building a packing costs one device->host read (T_valid sizes the GEMMs). It
replaces, rather than adds to, the mask.all().item() read the trivial-mask
memo makes once per new mask object (reference optimized/model.py:68-93).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class RowPacking:
    """Row maps between a [B, S] padded batch and its T_valid valid rows."""

    batch: int
    seq_len: int
    t_valid: int
    max_len: int
    min_len: int
    idx: torch.Tensor   # int32 [t_valid]: packed row -> padded row b*S + s
    inv: torch.Tensor   # int32 [B*S]: padded row -> packed row, -1 for padding
    cu: torch.Tensor    # int32 [B+1]: sequence b is packed rows cu[b] .. cu[b+1]

    @property
    def trivial(self) -> bool:
        """Every position valid: packing would change nothing."""
        return self.t_valid == self.batch * self.seq_len

    def key(self) -> tuple:
        """What a captured graph bakes in: the sizes, not the maps' contents."""
        return (self.batch, self.seq_len, self.t_valid)

    def empty_like(self) -> "RowPacking":
        """Uninitialised maps of the same sizes (a graph's static copy)."""
        return RowPacking(self.batch, self.seq_len, self.t_valid, self.max_len, self.min_len,
                          torch.empty_like(self.idx), torch.empty_like(self.inv),
                          torch.empty_like(self.cu))

    def copy_(self, other: "RowPacking") -> None:
        """Load another packing's maps (same sizes) into these tensors."""
        if other.key() != self.key():
            raise ValueError(f"packing sizes differ: {other.key()} vs {self.key()}")
        self.idx.copy_(other.idx)
        self.inv.copy_(other.inv)
        self.cu.copy_(other.cu)


def build_packing(mask: torch.Tensor) -> RowPacking:
    """The packing of a bool [B, S] mask (True = valid). One host sync."""
    if mask.dim() != 2 or mask.dtype != torch.bool:
        raise ValueError(f"valid_token_mask must be a bool [B, S] tensor, got "
                         f"{mask.dtype} {tuple(mask.shape)}")
    B, S = (int(n) for n in mask.shape)
    dev = mask.device
    flat = mask.reshape(-1)
    if B * S == 0:
        z = torch.zeros(0, dtype=torch.int32, device=dev)
        return RowPacking(B, S, 0, 0, 0, z, z.clone(), torch.zeros(B + 1, dtype=torch.int32,
                                                                    device=dev))
    pos = torch.cumsum(flat.to(torch.int32), 0, dtype=torch.int32)  # inclusive
    counts = mask.sum(dim=1, dtype=torch.int32)
    cu = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    cu[1:] = torch.cumsum(counts, 0, dtype=torch.int32)
    t_valid, max_len, min_len = (int(v) for v in
                                 torch.stack([cu[-1], counts.max(), counts.min()]).tolist())
    minus_one = torch.full_like(pos, -1)
    inv = torch.where(flat, pos - 1, minus_one)
    # Scatter each valid row's padded index to its packed slot; padded rows
    # all land in one spare slot past the end, which is then dropped.
    target = torch.where(flat, pos - 1, torch.full_like(pos, t_valid)).long()
    idx = torch.empty(t_valid + 1, dtype=torch.int32, device=dev)
    idx.scatter_(0, target, torch.arange(B * S, dtype=torch.int32, device=dev))
    return RowPacking(B, S, t_valid, max_len, min_len, idx[:t_valid], inv, cu)
