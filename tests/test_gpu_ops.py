"""Op-level parity of the HIP kernels, called through the extension (C ABI).

References are computed on the CPU in fp64 from the same seeded inputs. Where
a kernel contracts fp16 operands, the reference rounds the same operands to
fp16 with RNE first, so the check pins the arithmetic contract (which operand
is narrowed, where) and not only a loose tolerance.
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


# ---- MFMA accumulator layout ---------------------------------------------------

def test_mfma_ceiling_probe_runs(kernels):
    """The sustained-rate probe launches and times; the rate it implies stays
    under the datasheet's 2.5 PFLOP/s (the probe counts its flops right)."""
    wg, iters = 256, 16
    flops = wg * 4 * iters * 16 * 32768
    for rnd in (False, True):
        us = kernels.mfma_ceiling_us(wg, iters, random_operands=rnd, reps=5, warmup=2)
        assert us > 0
        assert flops / (us * 1e-6) < 2.6e15


def test_mfma_layout_probe(kernels):
    """The (row, col) each accumulator register holds, as the kernels assume it."""
    got = kernels.mfma_layout_probe().cpu().numpy()
    want32 = np.empty((64, 16), dtype=np.int32)
    for lane in range(64):
        for r in range(16):
            want32[lane, r] = (8 * (r // 4) + 4 * (lane // 32) + (r % 4)) * 32 + lane % 32
    want16 = np.empty((64, 4), dtype=np.int32)
    for lane in range(64):
        for r in range(4):
            want16[lane, r] = (4 * (lane // 16) + r) * 16 + lane % 16
    np.testing.assert_array_equal(got[:1024].reshape(64, 16), want32)
    np.testing.assert_array_equal(got[1024:].reshape(64, 4), want16)


def test_smoke_identity(kernels):
    x = torch.randn(1000, device=DEV)
    assert torch.equal(kernels.smoke_test_identity(x), x)


# ---- LayerNorm -------------------------------------------------------------------

LN_SHAPES = [(128, 128), (4096, 512), (1000, 1024), (37, 2048), (160, 256), (1023, 24),
             (5, 1), (3, 200), (64, 8192), (1, 4096)]


@pytest.mark.parametrize("rows,D", LN_SHAPES)
@pytest.mark.parametrize("with_sub", [True, False])
def test_layernorm_parity(kernels, rows, D, with_sub):
    r = np.random.default_rng(rows * 31 + D)
    x = r.standard_normal((rows, D)).astype(np.float32)
    sub = r.standard_normal((rows, D)).astype(np.float32)
    w = (1 + 0.3 * r.standard_normal(D)).astype(np.float32)
    b = (0.2 * r.standard_normal(D)).astype(np.float32)
    total = (x + sub) if with_sub else x  # fp32 add, as the reference rounds it
    want = brute.layer_norm(total.astype(np.float64), w, b) if rows * D <= 4096 else None
    if want is None:
        t = torch.from_numpy(total).double()
        want = torch.nn.functional.layer_norm(t, (D,), torch.from_numpy(w).double(),
                                              torch.from_numpy(b).double(), 1e-5).numpy()
    if with_sub:
        xn, nm = kernels.fused_add_layernorm(_t(x), _t(sub), _t(w), _t(b), 1e-5, False)
        assert torch.equal(xn.cpu(), torch.from_numpy(total))  # x_new is exactly x + sub
    else:
        nm = kernels.fused_layernorm(_t(x), _t(w), _t(b), 1e-5, False)
    np.testing.assert_allclose(nm.cpu().numpy(), want, atol=2e-5, rtol=1e-5)
    # fp16 output is the RNE narrowing of the fp32 result (1 ulp of slack for
    # values that land next to a rounding boundary)
    if with_sub:
        _, nh = kernels.fused_add_layernorm(_t(x), _t(sub), _t(w), _t(b), 1e-5, True)
    else:
        nh = kernels.fused_layernorm(_t(x), _t(w), _t(b), 1e-5, True)
    assert nh.dtype == torch.float16
    want16 = torch.from_numpy(want).half().float().numpy()
    ulp = np.spacing(np.abs(want16).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(nh.cpu().float().numpy() - want16) <= ulp + 1e-7)


@pytest.mark.parametrize("D", [256, 512])
def test_layernorm_tall_gather_with_dropped_rows(kernels, D):
    """The packed-row gather over a tall input (70K rows from 90K): rows whose
    index is out of range come out zero, the rest equal the dense LayerNorm
    of the indexed row."""
    in_rows = 90000
    g = torch.Generator().manual_seed(D)
    x = torch.randn(in_rows, D, generator=g).to(DEV)
    w = torch.randn(D, generator=g).to(DEV)
    b = torch.randn(D, generator=g).to(DEV)
    idx = torch.randint(0, in_rows, (70003,), generator=g, dtype=torch.int32)
    idx[::11] = -1
    idx[5::13] = in_rows + 7
    idx = idx.to(DEV)
    rows, normed = kernels.fused_layernorm_rows(x, w, b, idx, 1e-5, "float", True)
    dense = kernels.fused_layernorm(x, w, b, 1e-5, False)
    ok = (idx >= 0) & (idx < in_rows)
    assert torch.equal(rows[ok], x.index_select(0, idx[ok].long()))
    assert torch.equal(normed[ok], dense.index_select(0, idx[ok].long()))
    assert torch.count_nonzero(rows[~ok]) == 0 and torch.count_nonzero(normed[~ok]) == 0


@pytest.mark.parametrize("mean,scale", [(1e4, 1.0), (1e5, 1e-2)])
def test_layernorm_large_mean_rows(kernels, mean, scale):
    """Large-mean rows against the fp64 definition (reference verify_layernorm_warp.py:37-45)."""
    r = np.random.default_rng(7)
    x = (r.standard_normal((1024, 32)) * scale + mean).astype(np.float32)
    w, b = np.ones(32, np.float32), np.zeros(32, np.float32)
    got = kernels.fused_layernorm(_t(x), _t(w), _t(b), 1e-5, False).cpu().numpy()
    t = torch.from_numpy(x.astype(np.float64))
    want = torch.nn.functional.layer_norm(t, (32,), eps=1e-5).numpy()
    np.testing.assert_allclose(got, want, atol=2e-3)


def test_layernorm_constant_row_gives_beta(kernels):
    b = torch.linspace(-1, 1, 256, device=DEV)
    x = torch.full((8, 256), 3.0, device=DEV)
    out = kernels.fused_layernorm(x, torch.ones(256, device=DEV), b, 1e-5, False)
    assert torch.equal(out, b.expand(8, 256))


# ---- GEMM --------------------------------------------------------------------------

GEMM_SHAPES = [(128, 384, 128), (4096, 512, 512), (300, 200, 136), (64, 2048, 256),
               (1000, 1024, 256), (129, 129, 64), (7, 8, 8), (2048, 1536, 1024)]


def _gemm_case(M, N, K, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)).astype(np.float32)
    a = np.sqrt(6.0 / (N + K))
    w = r.uniform(-a, a, (N, K)).astype(np.float32)
    b = (0.1 * r.standard_normal(N)).astype(np.float32)
    return x, w, b


def _h(a):
    return a.astype(np.float16).astype(np.float64)


def _gelu64(z):
    return torch.nn.functional.gelu(torch.from_numpy(z), approximate="none").numpy()


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("act", ["none", "gelu"])
def test_gemm_fp16_math(kernels, M, N, K, act):
    """fp16 operands (x and W narrowed with RNE), fp32 accumulation."""
    x, w, b = _gemm_case(M, N, K, M + N + K)
    z = _h(x) @ _h(w).T + b
    want = _gelu64(z) if act == "gelu" else z
    fn = kernels.linear_gelu if act == "gelu" else kernels.linear_bias
    got = fn(_t(x), _t(w), _t(b), -1, -1).cpu().numpy()
    # fp32 accumulation of K products: ~sqrt(K) * 2^-24 * |x||w|
    np.testing.assert_allclose(got, want, atol=2e-5 * np.sqrt(K / 128), rtol=1e-5)
    # an fp16 x gives the same answer bit for bit (the narrowing only moved)
    got16 = fn(_t(x).half(), _t(w), _t(b), -1, -1).cpu().numpy()
    np.testing.assert_array_equal(got16, got)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES[:5])
def test_gemm_fp16x3_math(kernels, M, N, K):
    """Split fp16 hi+lo arithmetic: fp32-class products against the exact fp64 GEMM."""
    x, w, b = _gemm_case(M, N, K, 3 * M + N)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    got = kernels.linear_bias(_t(x), _t(w), _t(b), -1, 0).cpu().numpy()
    np.testing.assert_allclose(got, want, atol=3e-6 * np.sqrt(K / 128), rtol=2e-6)
    # and it is far tighter than the one-pass fp16 result
    one = kernels.linear_bias(_t(x), _t(w), _t(b), -1, -1).cpu().numpy()
    assert np.abs(got - want).max() < 0.05 * np.abs(one - want).max()


@pytest.mark.parametrize("tile", [0, 2])
def test_gemm_tiles_agree(kernels, tile):
    x, w, b = _gemm_case(777, 320, 192, 11)
    auto = kernels.linear_bias(_t(x), _t(w), _t(b), -1, -1)
    forced = kernels.linear_bias(_t(x), _t(w), _t(b), tile, -1)
    np.testing.assert_allclose(forced.cpu().numpy(), auto.cpu().numpy(), atol=1e-5)


def test_gemm_half_output_is_rne_of_fp32(kernels):
    x, w, b = _gemm_case(512, 384, 256, 5)
    f32 = kernels.linear_bias(_t(x), _t(w), _t(b), -1, -1, False)
    f16 = kernels.linear_bias(_t(x), _t(w), _t(b), -1, -1, True)
    assert f16.dtype == torch.float16
    assert torch.equal(f16, f32.half())
    # The GELU epilogue of the two instantiations may contract its multiply-adds
    # differently (<= 1 fp32 ulp apart), which can flip a tie in the fp16
    # rounding: allow one fp16 ulp.
    g32 = kernels.linear_gelu(_t(x), _t(w), _t(b), -1, -1, False)
    g16 = kernels.linear_gelu(_t(x), _t(w), _t(b), -1, -1, True)
    ref16 = g32.half().float()
    ulp = torch.from_numpy(np.spacing(np.abs(ref16.cpu().numpy()).astype(np.float16))).float()
    assert torch.all((g16.float() - ref16).abs().cpu() <= ulp)


def test_gemm_declines_uncovered(kernels):
    x, w, b = _gemm_case(16, 16, 12, 1)
    assert kernels.linear_bias(_t(x), _t(w), _t(b)) is None
    x8, w8, b8 = _gemm_case(16, 16, 8, 1)
    assert kernels.linear_bias(_t(x8).double(), _t(w8).double(), _t(b8).double()) is None


def test_gemm_weight_cache_follows_in_place_updates(kernels):
    x, w, b = _gemm_case(64, 64, 64, 2)
    wt = _t(w)
    first = kernels.linear_bias(_t(x), wt, _t(b))
    with torch.no_grad():
        wt.mul_(2.0)
    second = kernels.linear_bias(_t(x), wt, _t(b))
    bt = _t(b)
    np.testing.assert_allclose((second - bt).cpu().numpy(), 2 * (first - bt).cpu().numpy(),
                               atol=1e-5)


# ---- attention --------------------------------------------------------------------

# (label, B, H, S, head_dim, causal, padded) -- the reference's op-level cases
# (reference scripts/verify_kernel.py:39-55) at the head_dims the MFMA kernel covers,
# plus the configs' own attention shapes at reduced batch.
ATTN_CASES = [
    ("tiny", 1, 1, 8, 32, False, False),
    ("tiny causal", 1, 1, 8, 32, True, False),
    ("tiny padded", 2, 1, 8, 32, False, True),
    ("tiny causal+pad", 2, 1, 8, 32, True, True),
    ("default", 8, 8, 128, 64, False, False),
    ("default causal", 8, 8, 128, 64, True, False),
    ("default padded", 8, 8, 128, 64, False, True),
    ("default caus+pad", 8, 8, 128, 64, True, True),
    ("long seq", 1, 8, 2048, 64, False, False),
    ("long seq causal", 1, 8, 2048, 64, True, False),
    ("odd shape", 3, 5, 37, 32, True, True),
    ("wide head_dim", 2, 4, 64, 128, False, False),
    ("wide caus+pad", 2, 4, 128, 128, True, True),
    ("C1", 2, 4, 64, 32, False, False),
    ("C2", 2, 8, 512, 64, False, True),
    ("C4", 1, 4, 2048, 128, False, False),
    ("C5", 64, 4, 16, 64, False, True),
    ("ragged S", 2, 3, 200, 128, True, False),
]


def _attn_inputs(B, H, S, hd, padded, seed):
    r = np.random.default_rng(seed)
    q, k, v = (r.standard_normal((B, H, S, hd)).astype(np.float32) for _ in range(3))
    valid = None
    if padded:
        lens = r.integers(max(1, S // 4), S + 1, size=B)
        lens[0] = S
        valid = np.arange(S)[None, :] < lens[:, None]
    return q, k, v, valid


@pytest.mark.parametrize("case", ATTN_CASES, ids=[c[0] for c in ATTN_CASES])
def test_attention_parity(kernels, case):
    _, B, H, S, hd, causal, padded = case
    q, k, v, valid = _attn_inputs(B, H, S, hd, padded, B * 1000 + S + hd)
    scale = hd ** -0.5
    # reference on the fp16-rounded operands the kernel contracts, in fp64
    want = reference_attention(_h(q), _h(k), _h(v), valid, causal, scale,
                               dtype=torch.float64).numpy()
    mask = None if valid is None else _t(valid, torch.bool)[:, None, None, :]
    out = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), _t(v).half(), mask,
                                          causal, scale, 0, 0, 0)
    assert out.dtype == torch.float16 and tuple(out.shape) == (B, H, S, hd)
    got = out.float().cpu().numpy()
    # P is narrowed to fp16 between the two products and O is stored in fp16
    np.testing.assert_allclose(got, want, atol=3e-3, rtol=2e-3)
    # layout 1 is the same numbers in [B, S, H*hd]
    out1 = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), _t(v).half(), mask,
                                           causal, scale, 0, 1, 0)
    assert torch.equal(out1, out.transpose(1, 2).reshape(B, S, H * hd))


def test_attention_fp32_inputs_narrow_like_fp16(kernels):
    q, k, v, valid = _attn_inputs(2, 4, 96, 64, True, 3)
    mask = _t(valid, torch.bool)[:, None, None, :]
    o32 = kernels.fused_attention_forward(_t(q), _t(k), _t(v), mask, False, 0.125, 0, 1, 0)
    o16 = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), _t(v).half(), mask,
                                          False, 0.125, 0, 1, 0)
    assert o32.dtype == torch.float32
    np.testing.assert_allclose(o32.cpu().numpy(), o16.float().cpu().numpy(), atol=1e-3)


def test_attention_strided_views_equal_contiguous(kernels):
    """q/k/v as strided views of one [B, S, 3, H, hd] projection are read in place
    and give bit-identical output (reference verify_kernel.py:240-249)."""
    B, S, H, hd = 2, 96, 4, 64
    qkv = torch.randn(B, S, 3 * H * hd, device=DEV).half()
    q, k, v = qkv.view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4).unbind(0)
    a = kernels.fused_attention_forward(q, k, v, None, True, hd ** -0.5, 0, 1, 0)
    b = kernels.fused_attention_forward(q.contiguous(), k.contiguous(), v.contiguous(), None,
                                        True, hd ** -0.5, 0, 1, 0)
    assert torch.equal(a, b)


def test_attention_special_cases(kernels):
    B, H, S, hd = 2, 2, 80, 64
    q, k, v, _ = _attn_inputs(B, H, S, hd, False, 9)
    # a single allowed key -> that key's V row, exactly (p = exp2(0) = 1)
    valid = np.zeros((B, S), dtype=bool)
    valid[:, 5] = True
    mask = _t(valid, torch.bool)[:, None, None, :]
    vh = _t(v).half()
    out = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), vh, mask, False, 0.125,
                                          0, 0, 0)
    assert torch.equal(out, vh[:, :, 5:6, :].expand(B, H, S, hd))
    # no allowed key at all -> 0
    none = torch.zeros(B, 1, 1, S, dtype=torch.bool, device=DEV)
    out = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), vh, none, False, 0.125,
                                          0, 0, 0)
    assert torch.count_nonzero(out).item() == 0
    # constant V -> that constant
    vc = torch.full((B, H, S, hd), 0.75, device=DEV).half()
    out = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), vc, None, True, 0.125,
                                          0, 0, 0)
    np.testing.assert_allclose(out.float().cpu().numpy(), 0.75, atol=1e-3)
    # causal row 0 -> v[0]
    out = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), vh, None, True, 0.125,
                                          0, 0, 0)
    assert torch.equal(out[:, :, 0, :], vh[:, :, 0, :])


def test_attention_general_mask(kernels):
    """A query-dependent [B, 1, S, S] mask takes the per-element path."""
    B, H, S, hd = 2, 2, 70, 32
    q, k, v, _ = _attn_inputs(B, H, S, hd, False, 12)
    r = np.random.default_rng(1)
    m = r.random((B, 1, S, S)) < 0.7
    m[:, :, :, 0] = True
    # the general mask applied in an fp64 reference directly
    qd, kd, vd = (torch.from_numpy(_h(a)) for a in (q, k, v))
    s = (qd @ kd.transpose(-1, -2)) * 0.2
    s = s.masked_fill(~torch.from_numpy(m), float("-inf"))
    want = (torch.softmax(s, -1) @ vd).numpy()
    got = kernels.fused_attention_forward(_t(q).half(), _t(k).half(), _t(v).half(),
                                          _t(m, torch.bool), False, 0.2, 0, 0, 0)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=3e-3, rtol=2e-3)


def test_attention_refusals(kernels):
    q = torch.randn(1, 1, 16, 64, device=DEV).half()
    with pytest.raises(RuntimeError, match="tile"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, 3, 1, 0)
    with pytest.raises(RuntimeError, match="fp32"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, 2, 1, 1)
    with pytest.raises(RuntimeError, match="head_dim"):
        # a forced MFMA kernel declines a head_dim it has no tile for (auto
        # would run the exact fp32 kernel instead)
        q48 = torch.randn(1, 1, 16, 48, device=DEV).half()
        kernels.fused_attention_forward(q48, q48, q48, None, False, 0.125, 2, 1, 0)
    with pytest.raises(RuntimeError, match="float16, bfloat16 or float32"):
        qi = torch.zeros(1, 1, 16, 64, dtype=torch.float64, device=DEV)
        kernels.fused_attention_forward(qi, qi, qi, None, False, 0.125, 0, 1, 0)


# ---- LDS-DMA pipelined GEMM --------------------------------------------------------

def test_lds_dma_probe(kernels):
    """One global_load_lds_dwordx4: lane l's 16 bytes land at LDS offset 16 l."""
    src = torch.arange(256, dtype=torch.int32, device=DEV) * 7 + 3
    out = kernels.lds_dma_probe(src).cpu().numpy()
    np.testing.assert_array_equal(out[:256], src.cpu().numpy())
    assert np.all(out[256:] == 0)


@pytest.mark.parametrize("rows,D", [(300, 256), (64, 512), (5, 1024)])
def test_layernorm_split_planes(kernels, rows, D):
    r = np.random.default_rng(rows + D)
    x = r.standard_normal((rows, D)).astype(np.float32)
    w = (1 + 0.3 * r.standard_normal(D)).astype(np.float32)
    b = (0.2 * r.standard_normal(D)).astype(np.float32)
    planes = kernels.fused_layernorm_split(_t(x), _t(w), _t(b), 1e-5)
    assert planes.dtype == torch.float16 and tuple(planes.shape) == (2, rows, D)
    hi, lo = planes[0].float().cpu().numpy(), planes[1].float().cpu().numpy()
    want = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (D,),
                                          torch.from_numpy(w).double(),
                                          torch.from_numpy(b).double(), 1e-5).numpy()
    # hi is the fp16 rounding, hi + lo * 2^-12 the ~22-bit value
    assert np.all(np.abs(hi - want) <= np.spacing(np.abs(want).astype(np.float16)).astype(np.float64))
    np.testing.assert_allclose(hi + lo / 4096.0, want, atol=3e-6, rtol=1e-6)
    xn, planes2 = kernels.fused_add_layernorm_split(_t(x), _t(x), _t(w), _t(b), 1e-5)
    assert torch.equal(xn, _t(x) + _t(x))


DMA_SHAPES = [(300, 200, 128), (1000, 1024, 256), (64, 2048, 512), (513, 384, 64)]


ALL_TILES = [-1] + list(range(18))
SPLIT_TILES = [-1, 0, 2, 4, 5, 7, 8, 10, 13]   # the tiles built for split passes
TWO_PASS_TILES = SPLIT_TILES + [14, 19]        # 192x128 (4 / 8 waves): two passes at most


@pytest.mark.parametrize("M,N,K", DMA_SHAPES)
@pytest.mark.parametrize("tile", ALL_TILES)
def test_gemm_dma_one_pass(kernels, M, N, K, tile):
    """fp16 x on the pipelined kernel: every tile, with M and N tails."""
    x, w, b = _gemm_case(M, N, K, 7 * M + N)
    want = _h(x) @ _h(w).T + b
    got = kernels.linear_bias(_t(x).half(), _t(w), _t(b), tile, -1).cpu().numpy()
    np.testing.assert_allclose(got, want, atol=2e-5 * np.sqrt(K / 128), rtol=1e-5)
    # the register-staged kernel (tile 100 + id) gives the same numbers
    staged = kernels.linear_bias(_t(x).half(), _t(w), _t(b), 100 + (tile if 0 <= tile <= 4 else 0), -1)
    np.testing.assert_allclose(got, staged.cpu().numpy(), atol=2e-5 * np.sqrt(K / 128))


@pytest.mark.parametrize("M,N,K", DMA_SHAPES)
@pytest.mark.parametrize("tile", TWO_PASS_TILES)
def test_gemm_dma_split_weight(kernels, M, N, K, tile):
    """fp16 x with the fp16x3 math: two passes, x * (hi + 2^-12 lo) of the fp32 W."""
    x, w, b = _gemm_case(M, N, K, 5 * M + N)
    want = _h(x) @ w.astype(np.float64).T + b
    got = kernels.linear_bias(_t(x).half(), _t(w), _t(b), tile, 0).cpu().numpy()
    np.testing.assert_allclose(got, want, atol=3e-6 * np.sqrt(K / 128), rtol=2e-6)


@pytest.mark.parametrize("M,N,K", DMA_SHAPES)
@pytest.mark.parametrize("tile", TWO_PASS_TILES)
def test_gemm_dma_split_x_only(kernels, M, N, K, tile):
    """Split-plane x with an fp16 W (the fp16x2 arithmetic): two passes,
    (hi + 2^-12 lo)(x) * fp16(W), against the fp64 GEMM of those operands."""
    x, w, b = _gemm_case(M, N, K, 11 * M + N)
    xt = _t(x)
    hi = xt.half()
    lo = ((xt - hi.float()) * 4096.0).half()
    planes = torch.stack([hi, lo])
    xr = hi.double().cpu().numpy() + lo.double().cpu().numpy() / 4096.0
    want = xr @ _h(w).T + b
    got = kernels.linear_bias_split(planes, _t(w), _t(b), tile, False, split_weight=False)
    np.testing.assert_allclose(got.cpu().numpy(), want, atol=3e-6 * np.sqrt(K / 128), rtol=2e-6)
    # and it differs from the three-pass arithmetic by W's fp16 rounding
    if tile in SPLIT_TILES:
        three = kernels.linear_bias_split(planes, _t(w), _t(b), tile, False).cpu().numpy()
        assert np.abs(three - got.cpu().numpy()).max() > 1e-5
    else:
        with pytest.raises(RuntimeError, match="not built for split passes"):
            kernels.linear_bias_split(planes, _t(w), _t(b), tile, False)


@pytest.mark.parametrize("M,N,K", DMA_SHAPES)
@pytest.mark.parametrize("tile", SPLIT_TILES)
@pytest.mark.parametrize("act", ["none", "half_out"])
def test_gemm_dma_split_planes(kernels, M, N, K, tile, act):
    """Split-plane x: three passes, fp32-class products against the fp64 GEMM."""
    x, w, b = _gemm_case(M, N, K, 3 * M + N)
    xt = _t(x)
    hi = xt.half()
    lo = ((xt - hi.float()) * 4096.0).half()
    planes = torch.stack([hi, lo])
    xr = hi.double().cpu().numpy() + lo.double().cpu().numpy() / 4096.0
    want = xr @ w.astype(np.float64).T + b
    got = kernels.linear_bias_split(planes, _t(w), _t(b), tile, act == "half_out")
    if act == "half_out":
        want16 = want.astype(np.float16).astype(np.float64)
        # one fp16 ulp, or the fp32 accumulation's absolute error where the
        # result is small enough for that to exceed an ulp (cancellation)
        ulp = np.maximum(np.spacing(np.abs(want16).astype(np.float16)).astype(np.float64),
                         3e-6 * np.sqrt(K / 128))
        g = got.double().cpu().numpy()
        bad = np.abs(g - want16) > ulp
        if bad.any():
            i = np.unravel_index(np.argmax(np.abs(g - want16) - ulp), g.shape)
            raise AssertionError(f"{int(bad.sum())} elements off by more than 1 ulp; worst at {i}: "
                                 f"got {g[i]!r} want {want[i]!r} want16 {want16[i]!r} ulp {ulp[i]!r}")
    else:
        np.testing.assert_allclose(got.cpu().numpy(), want, atol=3e-6 * np.sqrt(K / 128), rtol=2e-6)


@pytest.mark.parametrize("M,N,K", [(128, 768, 256), (300, 200, 128), (513, 384, 64)])
@pytest.mark.parametrize("half_out", [False, True])
@pytest.mark.parametrize("split_weight", [False, True])
def test_gemm_planes_in_place(kernels, M, N, K, half_out, split_weight):
    """linear_bias_planes: the first M rows of [2, rows, K] planes, read in
    place, written into the first M rows of a larger output, equal
    linear_bias_split on a compacted copy of those rows bit for bit; the
    output's other rows are untouched."""
    rows = M + 77
    x, w, b = _gemm_case(rows, N, K, 13 * M + N)
    xt = _t(x)
    hi = xt.half()
    lo = ((xt - hi.float()) * 4096.0).half()
    planes = torch.stack([hi, lo])
    want = kernels.linear_bias_split(planes[:, :M].contiguous(), _t(w), _t(b), -1, half_out,
                                     split_weight=split_weight)
    out = torch.full((rows, N), 7.0, device=DEV, dtype=torch.float16 if half_out else torch.float32)
    got = kernels.linear_bias_planes(planes[0, :M], planes[1, :M], _t(w), _t(b), out[:M],
                                     split_weight=split_weight)
    assert got is not None and got.data_ptr() == out.data_ptr()
    torch.cuda.synchronize()
    assert torch.equal(out[:M], want)
    assert bool((out[M:] == 7.0).all())


@pytest.mark.parametrize("M,N,K", DMA_SHAPES)
@pytest.mark.parametrize("tile", [-1, 3, 5, 9, 10, 12, 13, 15, 16, 17])
def test_gemm_residual_epilogue(kernels, M, N, K, tile):
    """linear_bias(residual=R) = R + linear_bias() bit for bit: the epilogue adds
    the same fp32 values in the same order as a separate add would."""
    x, w, b = _gemm_case(M, N, K, 13 * M + N)
    r = np.random.default_rng(M + K).standard_normal((M, N)).astype(np.float32)
    xh, rt = _t(x).half(), _t(r)
    plain = kernels.linear_bias(xh, _t(w), _t(b), tile, -1)
    fused = kernels.linear_bias(xh, _t(w), _t(b), tile, -1, residual=rt)
    assert torch.equal(fused, rt + plain)
    # fp32 x takes the register-staged kernel, which declines the residual
    assert kernels.linear_bias(_t(x), _t(w), _t(b), -1, -1, residual=rt) is None
    with pytest.raises(RuntimeError, match="residual"):
        kernels.linear_bias(xh, _t(w), _t(b), tile, -1, out_half=True, residual=rt)
