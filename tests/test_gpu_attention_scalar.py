"""The exact fp32 attention kernel and the impl x precision routing.

impl=1 ("scalar") and precision=fp32 run every product and sum in fp32, so
they are held to the reference's scalar tolerance against an fp64 oracle on
the same (unrounded) inputs: 5e-6 (reference csrc/attention_dispatch.cuh:
225-228, "5e-6 against an exact reference"). Tolerance used below: atol
5e-6 plus rtol 1e-5 for outputs whose magnitude exceeds 1 (a long fp32 dot
product's rounding scales with its terms).
"""

import numpy as np
import pytest
import torch

from oracle.layer import reference_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL, RTOL = 5e-6, 1e-5


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def _inputs(B, H, S, hd, seed, lens=None):
    r = np.random.default_rng(seed)
    q, k, v = (r.standard_normal((B, H, S, hd)).astype(np.float32) for _ in range(3))
    valid = None
    if lens is not None:
        valid = np.arange(S)[None, :] < np.asarray(lens)[:, None]
    return q, k, v, valid


def _want(q, k, v, valid, causal, scale):
    return reference_attention(q, k, v, valid, causal, scale, dtype=torch.float64).numpy()


# (B, H, S, head_dim, causal, key lengths)
CASES = [
    (2, 2, 64, 64, False, None),
    (1, 3, 100, 32, True, None),
    (2, 2, 77, 48, False, [77, 30]),
    (1, 2, 129, 1, True, None),
    (2, 1, 40, 3, False, [40, 17]),
    (1, 2, 70, 96, True, [70]),
    (1, 1, 65, 200, False, None),
    (1, 2, 33, 256, True, None),
    (1, 1, 20, 513, False, [11]),
    (1, 1, 18, 1000, True, None),
    (1, 1, 9, 2048, False, None),
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}H{c[1]}S{c[2]}hd{c[3]}{'c' if c[4] else ''}"
                                             f"{'m' if c[5] else ''}" for c in CASES])
def test_scalar_matches_fp64(kernels, case):
    B, H, S, hd, causal, lens = case
    q, k, v, valid = _inputs(B, H, S, hd, S * 31 + hd, lens)
    scale = hd ** -0.5
    want = _want(q, k, v, valid, causal, scale)
    mask = None if valid is None else _t(valid, torch.bool)[:, None, None, :]
    out = kernels.fused_attention_forward(_t(q), _t(k), _t(v), mask, causal, scale, 1, 0, 1)
    assert out.dtype == torch.float32 and tuple(out.shape) == (B, H, S, hd)
    np.testing.assert_allclose(out.cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    # layout 1 holds the same values in [B, S, H*hd]
    out1 = kernels.fused_attention_forward(_t(q), _t(k), _t(v), mask, causal, scale, 1, 1, 1)
    assert torch.equal(out1, out.transpose(1, 2).reshape(B, S, H * hd))


def test_scalar_general_mask_and_fully_masked_rows(kernels):
    """A query-dependent [B, 1, S, S] mask, with whole query rows masked (-> 0)."""
    B, H, S, hd = 2, 2, 90, 64
    q, k, v, _ = _inputs(B, H, S, hd, 5)
    r = np.random.default_rng(2)
    m = r.random((B, 1, S, S)) < 0.6
    m[:, :, 7, :] = False
    m[1, :, 50:60, :] = False
    qd, kd, vd = (torch.from_numpy(a).double() for a in (q, k, v))
    s = (qd @ kd.transpose(-1, -2)) * 0.17
    s = s.masked_fill(~torch.from_numpy(m), float("-inf"))
    want = torch.nan_to_num(torch.softmax(s, -1) @ vd, nan=0.0).numpy()
    got = kernels.fused_attention_forward(_t(q), _t(k), _t(v), _t(m, torch.bool), True, 0.17,
                                          1, 0, 1).cpu().numpy()
    # causal AND the mask
    tri = np.triu(np.ones((S, S), dtype=bool), 1)
    s2 = (qd @ kd.transpose(-1, -2)) * 0.17
    s2 = s2.masked_fill(torch.from_numpy(~m | tri), float("-inf"))
    want2 = torch.nan_to_num(torch.softmax(s2, -1) @ vd, nan=0.0).numpy()
    np.testing.assert_allclose(got, want2, atol=ATOL, rtol=RTOL)
    assert not np.any(got[:, :, 7, :])
    got_nc = kernels.fused_attention_forward(_t(q), _t(k), _t(v), _t(m, torch.bool), False,
                                             0.17, 1, 0, 1).cpu().numpy()
    np.testing.assert_allclose(got_nc, want, atol=ATOL, rtol=RTOL)


def test_scalar_special_cases(kernels):
    B, H, S, hd = 1, 2, 50, 40
    q, k, v, _ = _inputs(B, H, S, hd, 8)
    vt = _t(v)
    # causal row 0 is v[0] exactly (p = exp(0) = 1, l = 1)
    out = kernels.fused_attention_forward(_t(q), _t(k), vt, None, True, 0.3, 1, 0, 1)
    assert torch.equal(out[:, :, 0, :], vt[:, :, 0, :])
    # a single allowed key gives its V row exactly
    valid = np.zeros((B, S), dtype=bool)
    valid[:, 13] = True
    out = kernels.fused_attention_forward(_t(q), _t(k), vt, _t(valid, torch.bool)[:, None, None, :],
                                          False, 0.3, 1, 0, 1)
    assert torch.equal(out, vt[:, :, 13:14, :].expand(B, H, S, hd))
    # equal scores (q = 0) give the mean of V
    out = kernels.fused_attention_forward(torch.zeros_like(vt), _t(k), vt, None, False, 0.3,
                                          1, 0, 1)
    np.testing.assert_allclose(out.cpu().numpy(),
                               np.broadcast_to(v.astype(np.float64).mean(axis=2, keepdims=True),
                                               v.shape), atol=ATOL)


def test_scalar_fp16_tensors_and_strided_views(kernels):
    """fp16 q/k/v widen exactly; strided views of one projection read in place."""
    B, S, H, hd = 2, 70, 3, 40
    qkv = torch.randn(B, S, 3 * H * hd, device=DEV).half()
    q, k, v = qkv.view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4).unbind(0)
    out = kernels.fused_attention_forward(q, k, v, None, True, 0.2, 1, 1, 1)
    assert out.dtype == torch.float16
    want = _want(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                 None, True, 0.2)
    want = want.transpose(0, 2, 1, 3).reshape(B, S, H * hd)
    # the only narrowing is the fp16 store of O: half an ulp of fp16
    np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=1e-5, rtol=2 ** -11 + 1e-5)
    contig = kernels.fused_attention_forward(q.contiguous(), k.contiguous(), v.contiguous(),
                                             None, True, 0.2, 1, 1, 1)
    assert torch.equal(out, contig)


def test_scalar_packed_sequences(kernels):
    """cu_seqlens rows: each sequence attends only within itself."""
    H, hd = 2, 64
    lens = [5, 33, 1, 64]
    rows = sum(lens)
    r = np.random.default_rng(4)
    q, k, v = (r.standard_normal((rows, H, hd)).astype(np.float32) for _ in range(3))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    out = kernels.fused_attention_forward(_t(q), _t(k), _t(v), None, True, 0.125, 1, 1, 1,
                                          cu_seqlens=cu, max_seqlen=max(lens))
    got = out.cpu().numpy().reshape(rows, H, hd)
    start = 0
    for n in lens:
        sl = slice(start, start + n)
        seq = [a[sl].transpose(1, 0, 2)[None] for a in (q, k, v)]
        want = _want(*seq, None, True, 0.125)[0].transpose(1, 0, 2)
        np.testing.assert_allclose(got[sl], want, atol=ATOL, rtol=RTOL)
        start += n


def test_precision_routing(kernels):
    """impl x precision: which arithmetic each request gets (reference
    csrc/attention_dispatch.cuh:219-304, attention_wmma.cuh:2043-2084)."""
    B, H, S, hd = 1, 2, 96, 64
    q, k, v, _ = _inputs(B, H, S, hd, 6)
    want = _want(q, k, v, None, False, 0.125)
    call = lambda impl, prec, *t: kernels.fused_attention_forward(  # noqa: E731
        *(t or (_t(q), _t(k), _t(v))), None, False, 0.125, impl, 0, prec).float().cpu().numpy()
    exact = call(1, 1)
    np.testing.assert_allclose(exact, want, atol=ATOL, rtol=RTOL)
    # auto impl + fp32 precision is the exact kernel, bit for bit
    assert np.array_equal(call(0, 1), exact)
    # impl=1 with auto precision is fp32 too
    assert np.array_equal(call(1, 0), exact)
    # auto + tf32: gfx950 has no tf32 matrix instruction -> the exact kernel
    assert np.array_equal(call(0, 2), exact)
    # fp16 arithmetic (the MFMA kernel) is measurably coarser than fp32
    f16 = call(0, 3)
    assert np.abs(f16 - want).max() > 1e-4
    np.testing.assert_allclose(f16, want, atol=4e-3, rtol=4e-3)
    # bf16 operands on the MFMA kernel: 8 significant bits
    bf = call(2, 4)
    assert not np.array_equal(bf, f16)
    qb, kb, vb = (torch.from_numpy(a).bfloat16().double().numpy() for a in (q, k, v))
    want_bf = _want(qb, kb, vb, None, False, 0.125)
    np.testing.assert_allclose(bf, want_bf, atol=3e-2, rtol=3e-2)
    # fp16 TENSORS contract in fp16 whatever the MFMA precision asked for
    h = (_t(q).half(), _t(k).half(), _t(v).half())
    assert np.array_equal(call(2, 4, *h), call(2, 3, *h))
    # head_dim the MFMA kernel does not cover: auto falls to the exact kernel
    q48, k48, v48, _ = _inputs(1, 1, 40, 48, 7)
    out48 = kernels.fused_attention_forward(_t(q48), _t(k48), _t(v48), None, False, 0.2, 0, 0, 0)
    np.testing.assert_allclose(out48.cpu().numpy(), _want(q48, k48, v48, None, False, 0.2),
                               atol=ATOL, rtol=RTOL)


def test_precision_refusals(kernels):
    q = torch.randn(1, 1, 16, 64, device=DEV)
    with pytest.raises(RuntimeError, match="scalar has no fp16"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, 1, 1, 3)
    with pytest.raises(RuntimeError, match="wmma has no fp32"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, 2, 1, 1)
    with pytest.raises(RuntimeError, match="tf32"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, 2, 1, 2)
    q48 = torch.randn(1, 1, 16, 48, device=DEV)
    with pytest.raises(RuntimeError, match="head_dim=48"):
        kernels.fused_attention_forward(q48, q48, q48, None, False, 0.125, 2, 1, 3)
    big = torch.randn(1, 1, 2, 2056, device=DEV)
    with pytest.raises(RuntimeError, match="up to 2048"):
        kernels.fused_attention_forward(big, big, big, None, False, 0.125, 1, 1, 1)
