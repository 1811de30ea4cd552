"""Split-KV attention and the 16-bit tensor dtypes, on the GPU.

Split-KV (reference csrc/attention_wmma.cuh:706-759, 1783-1826): the key
range of each query block cut into splits whose partials a combine pass
merges. Checked against fp64 attention on the fp16-rounded operands, and
against the unsplit kernel; splits left empty by a causal limit or a short
packed sequence must contribute nothing (no NaN), and a row with no allowed
key stays 0.

fp16 / bf16 tensors (reference csrc/attention_dispatch.cuh:104-106,
csrc/add_layernorm.cuh:555-557): LayerNorm and add+LayerNorm in the tensor
dtype with fp32 statistics, and attention on bf16 q/k/v contracting in bf16.
References are fp64 on the same rounded inputs; tolerances are stated per
test from the output dtype's rounding.
"""

import numpy as np
import pytest
import torch

from oracle import brute
from oracle.layer import reference_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def _round(a, dtype):
    """a rounded to `dtype` (RNE) and back to float64, on the CPU."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).double().numpy()


def _qkv(B, H, S, hd, seed):
    r = np.random.default_rng(seed)
    return [r.standard_normal((B, H, S, hd)).astype(np.float32) for _ in range(3)]


# ---- split-KV -----------------------------------------------------------------------

SPLIT_CASES = [
    # B, H, S, hd, causal, padded, splits
    (1, 8, 2048, 64, False, False, 2),
    (1, 8, 2048, 64, False, False, 8),
    (1, 4, 2048, 128, False, False, 4),
    (1, 2, 1000, 128, True, False, 5),     # causal: early query blocks leave splits empty
    (2, 2, 300, 64, False, True, 4),       # key padding: the masked kernel variant
    (1, 4, 640, 32, True, True, 16),       # more splits asked than tiles: capped
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[str(c) for c in SPLIT_CASES])
def test_split_kv_parity(kernels, case):
    B, H, S, hd, causal, padded, splits = case
    q, k, v = _qkv(B, H, S, hd, S + hd + splits)
    valid = None
    if padded:
        lens = np.random.default_rng(S).integers(S // 3, S + 1, size=B)
        valid = np.arange(S)[None, :] < lens[:, None]
    scale = hd ** -0.5
    n, nbytes = kernels.attention_split_plan(B, H, S, hd, causal, torch.float16,
                                             has_mask=padded, splits=splits)
    assert 1 < n <= min(splits, (S + 63) // 64) and nbytes > 0
    want = reference_attention(_round(q, torch.float16), _round(k, torch.float16),
                               _round(v, torch.float16), valid, causal, scale,
                               dtype=torch.float64).numpy()
    mask = None if valid is None else _t(valid, torch.bool)[:, None, None, :]
    qh, kh, vh = _t(q).half(), _t(k).half(), _t(v).half()
    got = kernels.fused_attention_forward(qh, kh, vh, mask, causal, scale, 0, 0, 0,
                                          splits=splits)
    one = kernels.fused_attention_forward(qh, kh, vh, mask, causal, scale, 0, 0, 0, splits=1)
    g = got.float().cpu().numpy()
    assert np.isfinite(g).all()
    np.testing.assert_allclose(g, want, atol=3e-3, rtol=2e-3)
    # the split only reorders fp32 sums: within fp16 output rounding of unsplit
    np.testing.assert_allclose(g, one.float().cpu().numpy(), atol=2e-3, rtol=2e-3)


def test_split_kv_packed_with_empty_splits(kernels):
    """Packed sequences of lengths 1, 5, 64 and 600 under 8 forced splits of
    the 640-key range: every split past a short sequence's end is empty and
    must add nothing; every row matches its own sequence's attention."""
    lens = [1, 5, 64, 600]
    H, hd, S = 4, 64, 640
    rows = sum(lens)
    r = np.random.default_rng(4)
    q, k, v = (r.standard_normal((rows, H, hd)).astype(np.float32) for _ in range(3))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qh, kh, vh = _t(q).half(), _t(k).half(), _t(v).half()
    for causal in (False, True):
        got = kernels.fused_attention_forward(qh, kh, vh, None, causal, 0.125, 0, 1, 0,
                                              cu_seqlens=_t(cu, torch.int32), max_seqlen=S,
                                              splits=8).float().cpu().numpy()
        assert np.isfinite(got).all()
        for b, L in enumerate(lens):
            sl = slice(cu[b], cu[b + 1])
            seq = [_round(a[sl].transpose(1, 0, 2)[None], torch.float16) for a in (q, k, v)]
            want = reference_attention(*seq, None, causal, 0.125, dtype=torch.float64)
            want = want.numpy()[0].transpose(1, 0, 2).reshape(L, H * hd)
            np.testing.assert_allclose(got[sl], want, atol=3e-3, rtol=2e-3)


def test_split_kv_fully_masked_rows_stay_zero(kernels):
    B, H, S, hd = 2, 2, 512, 64
    q, k, v = _qkv(B, H, S, hd, 77)
    none = torch.zeros(B, 1, 1, S, dtype=torch.bool, device=DEV)
    out = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), _t(v).half(), none,
                                          False, 0.125, 0, 0, 0, splits=4)
    assert torch.count_nonzero(out).item() == 0


def test_split_kv_auto_on_a_small_grid(kernels):
    """The occupancy choice splits B=1, H=8, S=2048 (128 workgroups) and the
    knobs steer it, with the same answer either way."""
    kernels.wmma_set_split_kv(True)
    kernels.wmma_set_split_count(0)
    assert kernels.wmma_split_count(1, 8, 2048, 64, False) > 1
    q, k, v = (_t(a).half() for a in _qkv(1, 8, 2048, 64, 5))
    auto = kernels.fused_attention_forward(q, k, v, None, False, 0.125, 0, 1, 0)
    kernels.wmma_set_split_kv(False)
    try:
        assert kernels.wmma_split_count(1, 8, 2048, 64, False) == 1
        off = kernels.fused_attention_forward(q, k, v, None, False, 0.125, 0, 1, 0)
    finally:
        kernels.wmma_set_split_kv(True)
    np.testing.assert_allclose(auto.float().cpu().numpy(), off.float().cpu().numpy(),
                               atol=2e-3, rtol=2e-3)


# ---- 16-bit tensors: LayerNorm ---------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,D", [(300, 256), (64, 1024), (7, 2048), (33, 100)])
@pytest.mark.parametrize("with_sub", [True, False])
def test_layernorm_16bit_tensors(kernels, dtype, rows, D, with_sub):
    """x (+ sub) rounded to the tensor dtype, fp32 statistics, normed output
    in the tensor dtype: within one rounding of that dtype (2^-11 relative
    for fp16, 2^-8 for bf16, of |normed| <= ~5) of fp64 on the same values."""
    r = np.random.default_rng(rows + D)
    x = r.standard_normal((rows, D)).astype(np.float32)
    sub = r.standard_normal((rows, D)).astype(np.float32)
    w = (1 + 0.3 * r.standard_normal(D)).astype(np.float32)
    b = (0.2 * r.standard_normal(D)).astype(np.float32)
    xt, st, wt, bt = (_t(a).to(dtype) for a in (x, sub, w, b))
    xr, sr, wr, br = (_round(a, dtype) for a in (x, sub, w, b))
    if with_sub:
        total = _round(xr + sr, dtype)          # x_new is the sum in the tensor dtype
        x_new, normed = kernels.fused_add_layernorm(xt, st, wt, bt, 1e-5)
        assert x_new.dtype == dtype
        np.testing.assert_array_equal(x_new.double().cpu().numpy(), total)
    else:
        total = xr
        normed = kernels.fused_layernorm(xt, wt, bt, 1e-5)
    assert normed.dtype == dtype
    want = brute.layer_norm(total, wr, br)
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    np.testing.assert_allclose(normed.double().cpu().numpy(), want, rtol=ulp, atol=ulp)


# ---- 16-bit tensors: attention ---------------------------------------------------------

@pytest.mark.parametrize("B,H,S,hd,causal,padded", [
    (2, 4, 128, 64, False, False), (1, 2, 300, 128, True, False), (3, 2, 96, 32, False, True),
    (64, 4, 16, 64, False, True)])
def test_attention_bf16_tensors(kernels, B, H, S, hd, causal, padded):
    """bf16 q/k/v contract in bf16 on the MFMA kernel (P narrowed to bf16,
    bf16 output): within 1.5e-2 abs / 1e-2 rel of fp64 on the bf16 operands;
    the exact kernel (impl 1) on the same tensors within a bf16 output
    rounding."""
    q, k, v = _qkv(B, H, S, hd, B + S + hd)
    valid = None
    if padded:
        lens = np.random.default_rng(S).integers(1, S + 1, size=B)
        valid = np.arange(S)[None, :] < lens[:, None]
    mask = None if valid is None else _t(valid, torch.bool)[:, None, None, :]
    scale = hd ** -0.5
    want = reference_attention(*(_round(a, torch.bfloat16) for a in (q, k, v)), valid, causal,
                               scale, dtype=torch.float64).numpy()
    qb, kb, vb = (_t(a).bfloat16() for a in (q, k, v))
    got = kernels.fused_attention_forward(qb, kb, vb, mask, causal, scale, 0, 0, 0)
    assert got.dtype == torch.bfloat16
    np.testing.assert_allclose(got.double().cpu().numpy(), want, atol=1.5e-2, rtol=1e-2)
    exact = kernels.fused_attention_forward(qb, kb, vb, mask, causal, scale, 1, 0, 0)
    assert exact.dtype == torch.bfloat16
    np.testing.assert_allclose(exact.double().cpu().numpy(), want, atol=4e-3, rtol=2 ** -7)


# ---- 16-bit tensors: GEMMs -------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(300, 512, 256), (4096, 1536, 512), (77, 128, 1024)])
@pytest.mark.parametrize("act", ["none", "gelu"])
def test_gemm_16bit_tensors(kernels, dtype, M, N, K, act):
    """A 16-bit model's projection: x, W, bias and the output in the model
    dtype, one pass of fp16 / bf16 MFMAs with fp32 accumulation. Against fp64
    on the same 16-bit operands, within the output's own rounding (2^-11
    relative for fp16, 2^-8 for bf16) plus accumulation order (2e-4 |.|)."""
    r = np.random.default_rng(M + N + K)
    x = r.standard_normal((M, K)).astype(np.float32)
    w = (r.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = (0.1 * r.standard_normal(N)).astype(np.float32)
    xt, wt, bt = (_t(a).to(dtype) for a in (x, w, b))
    fn = kernels.linear_gelu if act == "gelu" else kernels.linear_bias
    out = fn(xt, wt, bt)
    assert out is not None and out.dtype == dtype
    ref = _round(x, dtype) @ _round(w, dtype).T + _round(b, dtype)
    if act == "gelu":
        ref = brute.gelu(ref)
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    np.testing.assert_allclose(out.double().cpu().numpy(), ref, rtol=ulp, atol=ulp)


def test_gemm_16bit_declines_what_it_does_not_cover(kernels):
    x = torch.randn(64, 96, device=DEV).bfloat16()          # K % 64 != 0 for bf16
    w = torch.randn(32, 96, device=DEV).bfloat16()
    b = torch.zeros(32, device=DEV).bfloat16()
    assert kernels.linear_bias(x, w, b) is None
    # a residual epilogue is fp32-only
    x = torch.randn(64, 128, device=DEV).half()
    w = torch.randn(32, 128, device=DEV).half()
    b = torch.zeros(32, device=DEV).half()
    assert kernels.linear_bias(x, w, b, residual=torch.zeros(64, 32, device=DEV)) is None
    # mixed dtypes are not a 16-bit model's projection
    assert kernels.linear_bias(x.bfloat16(), w, b) is None
