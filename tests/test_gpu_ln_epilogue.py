"""The LayerNorm epilogue of the pipelined GEMM (dotl_linear_layernorm).

h = residual + x @ W^T + b and LayerNorm(h) from one kernel, for rows of up to
256 columns, must equal the two kernels it replaces -- linear_bias with the
residual epilogue on the same tile, then fused_layernorm (or its split-plane
and scattering forms) -- bit for bit: the epilogue repeats the LayerNorm
kernels' sums in the same order. The two-kernel chain itself is pinned
against the oracle by the layer parity tests.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS = 1e-5


def _case(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g)).half().to(DEV)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(DEV)
    b = (0.1 * torch.randn(N, generator=g)).to(DEV)
    r = torch.randn(M, N, generator=g).to(DEV)
    lw = (1 + 0.1 * torch.randn(N, generator=g)).to(DEV)
    lb = (0.1 * torch.randn(N, generator=g)).to(DEV)
    return x, w, b, r, lw, lb


SHAPES = [(300, 256, 256), (1000, 256, 1024), (513, 128, 512), (64, 64, 64), (777, 200, 128),
          (4096, 256, 256), (1, 256, 64)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("tile", [18])
@pytest.mark.parametrize("normed", ["float", "half", "split"])
def test_ln_epilogue_equals_the_two_kernels(kernels, M, N, K, tile, normed):
    print(f"[ln epilogue] M={M} N={N} K={K} tile={tile} normed={normed}", flush=True)
    x, w, b, r, lw, lb = _case(M, N, K, 7 * M + N)
    h_ref = kernels.linear_bias(x, w, b, tile, -1, residual=r)
    if normed == "split":
        n_ref = kernels.fused_layernorm_split(h_ref, lw, lb, EPS)
    else:
        n_ref = kernels.fused_layernorm(h_ref, lw, lb, EPS, normed == "half")
    for store_out in (True, False):
        h, n = kernels.linear_layernorm(x, w, b, r, lw, lb, EPS, normed=normed,
                                        store_out=store_out, tile=tile)
        torch.cuda.synchronize()
        assert torch.equal(n, n_ref)
        if store_out:
            assert torch.equal(h, h_ref)
        else:
            assert h is None


@pytest.mark.parametrize("M,N,K", [(300, 256, 256), (513, 128, 512)])
def test_ln_epilogue_without_residual(kernels, M, N, K):
    x, w, b, _, lw, lb = _case(M, N, K, 3)
    h_ref = kernels.linear_bias(x, w, b, 18, -1)
    n_ref = kernels.fused_layernorm(h_ref, lw, lb, EPS, False)
    h, n = kernels.linear_layernorm(x, w, b, None, lw, lb, EPS, tile=18)
    assert torch.equal(h, h_ref) and torch.equal(n, n_ref)


@pytest.mark.parametrize("M,N,K,rows", [(300, 256, 256, 512), (700, 128, 128, 1000)])
def test_ln_epilogue_scatter_and_zero_rows(kernels, M, N, K, rows):
    """Packed rows scattered to a padded output (row r -> out_row[r]), the
    other rows zeroed by zero_rows from the inverse map: the scattering
    LayerNorm (fused_layernorm_rows over the inverse map) bit for bit."""
    x, w, b, r, lw, lb = _case(M, N, K, 11)
    g = torch.Generator().manual_seed(5)
    out_row = torch.sort(torch.randperm(rows, generator=g)[:M]).values.to(torch.int32).to(DEV)
    inv = torch.full((rows,), -1, dtype=torch.int32, device=DEV)
    inv[out_row.long()] = torch.arange(M, dtype=torch.int32, device=DEV)
    h_ref = kernels.linear_bias(x, w, b, 18, -1, residual=r)
    _, n_ref = kernels.fused_layernorm_rows(h_ref, lw, lb, inv, EPS, "float", False)
    # the output is allocated by the call: poison the block the caching
    # allocator will hand it, so a row neither kernel writes shows as NaN
    poison = torch.full((rows, N), float("nan"), device=DEV)
    del poison
    h, n = kernels.linear_layernorm(x, w, b, r, lw, lb, EPS, store_out=False, out_row=out_row,
                                    normed_rows=rows)
    kernels.zero_rows(n, inv)
    assert h is None
    assert torch.equal(n, n_ref)


def test_ln_epilogue_declines(kernels):
    """Rows wider than a tile, or operand types the kernel does not take,
    decline (None): the caller runs the two kernels."""
    x, w, b, r, lw, lb = _case(64, 256, 64, 1)
    assert kernels.linear_layernorm(x.float(), w, b, r, lw, lb) is None
    x5, w5, b5, r5, lw5, lb5 = _case(64, 512, 64, 1)
    assert kernels.linear_layernorm(x5, w5, b5, r5, lw5, lb5) is None
    x6, w6, b6, r6, lw6, lb6 = _case(64, 256, 96, 1)   # K not a multiple of 64
    assert kernels.linear_layernorm(x6, w6, b6, r6, lw6, lb6) is None
    with pytest.raises(RuntimeError, match="tile"):
        kernels.linear_layernorm(x, w, b, r, lw, lb, tile=15)
