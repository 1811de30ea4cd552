"""The fused FFN with the residual add and the row LayerNorm (dotl_ffn_layernorm).

y = r + GELU(x W1^T + b1) W2^T + b2 and LayerNorm(y) from one kernel, d_model
256, must equal the two GEMMs it replaces -- linear_gelu with an fp16 output,
then linear_layernorm (the GEMM with the residual and LayerNorm epilogue) --
bit for bit: the same MFMAs over the same operands in the same k order, the
same GELU and fp16 rounding, the same epilogue. That chain is pinned against
the oracle by the layer parity tests and the GEMM / LayerNorm op tests.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS = 1e-5
D = 256


def _case(M, F, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).half().to(DEV)
    w1 = (torch.randn(F, D, generator=g) / D ** 0.5).to(DEV)
    b1 = (0.1 * torch.randn(F, generator=g)).to(DEV)
    w2 = (torch.randn(D, F, generator=g) / F ** 0.5).to(DEV)
    b2 = (0.1 * torch.randn(D, generator=g)).to(DEV)
    r = torch.randn(M, D, generator=g).to(DEV)
    lw = (1 + 0.1 * torch.randn(D, generator=g)).to(DEV)
    lb = (0.1 * torch.randn(D, generator=g)).to(DEV)
    return x, w1, b1, w2, b2, r, lw, lb


def _chain(kernels, x, w1, b1, w2, b2, r, lw, lb, normed, store_out=True):
    h = kernels.linear_gelu(x, w1, b1, -1, -1, True)
    return kernels.linear_layernorm(h, w2, b2, r, lw, lb, EPS, normed=normed,
                                    store_out=store_out, tile=18)


SHAPES = [(300, 1024), (128, 64), (1000, 512), (4096, 2048), (1, 256), (777, 1024), (85, 128)]


@pytest.mark.parametrize("M,F", SHAPES)
@pytest.mark.parametrize("normed", ["float", "half", "split"])
def test_ffn_ln_equals_the_two_gemms(kernels, M, F, normed):
    print(f"[ffn_ln] M={M} F={F} normed={normed}", flush=True)
    x, w1, b1, w2, b2, r, lw, lb = _case(M, F, 13 * M + F)
    y_ref, n_ref = _chain(kernels, x, w1, b1, w2, b2, r, lw, lb, normed)
    for store_out in (True, False):
        y, n = kernels.ffn_layernorm(x, w1, b1, w2, b2, r, lw, lb, EPS, normed=normed,
                                     store_out=store_out)
        torch.cuda.synchronize()
        assert torch.equal(n, n_ref)
        if store_out:
            assert torch.equal(y, y_ref)
        else:
            assert y is None


def test_ffn_ln_without_residual(kernels):
    x, w1, b1, w2, b2, _, lw, lb = _case(300, 1024, 3)
    y_ref, n_ref = _chain(kernels, x, w1, b1, w2, b2, None, lw, lb, "float")
    y, n = kernels.ffn_layernorm(x, w1, b1, w2, b2, None, lw, lb, EPS, store_out=True)
    assert torch.equal(y, y_ref) and torch.equal(n, n_ref)


@pytest.mark.parametrize("M,F,rows", [(300, 1024, 512), (700, 512, 1000)])
def test_ffn_ln_scatter_and_zero_rows(kernels, M, F, rows):
    """Packed rows scattered to a padded output (row m -> out_row[m]), the
    other rows zeroed by zero_rows from the inverse map: the chain's
    scattering form bit for bit, with the unwritten rows poisoned."""
    x, w1, b1, w2, b2, r, lw, lb = _case(M, F, 11)
    g = torch.Generator().manual_seed(5)
    out_row = torch.sort(torch.randperm(rows, generator=g)[:M]).values.to(torch.int32).to(DEV)
    inv = torch.full((rows,), -1, dtype=torch.int32, device=DEV)
    inv[out_row.long()] = torch.arange(M, dtype=torch.int32, device=DEV)
    h = kernels.linear_gelu(x, w1, b1, -1, -1, True)
    _, n_ref = kernels.linear_layernorm(h, w2, b2, r, lw, lb, EPS, store_out=False,
                                        out_row=out_row, normed_rows=rows)
    kernels.zero_rows(n_ref, inv)
    poison = torch.full((rows, D), float("nan"), device=DEV)
    del poison
    y, n = kernels.ffn_layernorm(x, w1, b1, w2, b2, r, lw, lb, EPS, out_row=out_row,
                                 normed_rows=rows)
    kernels.zero_rows(n, inv)
    assert y is None
    assert torch.equal(n, n_ref)
    # the kernel's own zeroing of the rows out_row skips (before the first,
    # between, after the last) equals zero_rows'
    for first in (0, 3):
        orow = out_row if first == 0 else out_row + first - int(out_row[0].item())
        if int(orow[-1].item()) >= rows:
            continue
        inv2 = torch.full((rows,), -1, dtype=torch.int32, device=DEV)
        inv2[orow.long()] = torch.arange(M, dtype=torch.int32, device=DEV)
        _, n_ref2 = kernels.linear_layernorm(h, w2, b2, r, lw, lb, EPS, store_out=False,
                                             out_row=orow, normed_rows=rows)
        kernels.zero_rows(n_ref2, inv2)
        poison = torch.full((rows, D), float("nan"), device=DEV)
        del poison
        _, n2 = kernels.ffn_layernorm(x, w1, b1, w2, b2, r, lw, lb, EPS, out_row=orow,
                                      normed_rows=rows, zero_padded=True)
        assert torch.equal(n2, n_ref2)


def test_ffn_ln_declines(kernels):
    """Shapes and operand types the kernel does not serve decline (None):
    the caller runs the two GEMMs."""
    x, w1, b1, w2, b2, r, lw, lb = _case(64, 1024, 1)
    assert kernels.ffn_layernorm(x.float(), w1, b1, w2, b2, r, lw, lb) is None
    g = torch.Generator().manual_seed(2)
    for F in (96, 4096):   # not a multiple of 64; above the staged b1
        w1f = torch.randn(F, D, generator=g).to(DEV)
        w2f = torch.randn(D, F, generator=g).to(DEV)
        b1f = torch.zeros(F, device=DEV)
        assert kernels.ffn_layernorm(x, w1f, b1f, w2f, b2, r, lw, lb) is None
    x5 = torch.randn(64, 128, device=DEV).half()
    w15 = torch.randn(512, 128, device=DEV)
    w25 = torch.randn(128, 512, device=DEV)
    assert kernels.ffn_layernorm(x5, w15, torch.zeros(512, device=DEV), w25,
                                 torch.zeros(128, device=DEV), None,
                                 torch.ones(128, device=DEV), torch.zeros(128, device=DEV)) is None
