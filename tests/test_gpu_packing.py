"""The packed-row path of a padded batch, on the GPU.

A padded batch runs on its valid rows only (optimized/packing.py): the first
LayerNorm gathers them, attention runs over packed sequences, the last
add+LayerNorm scatters back with zero padded rows. Each piece is checked
against the padded computation it replaces. On prefix masks (the padded-batch
configs) the valid rows must agree bit for bit; padded rows must be exact
zeros. Whole-layer parity against the oracle at C2 and C5 (which take this
path by default) is in test_gpu_layer.py.
"""

import numpy as np
import pytest
import torch

from layer_runner import TransformerConfig, build_model, to_device
from optimized import config as ocfg
from optimized import kernels as okernels
from optimized.packing import build_packing
from oracle.compare import compare_outputs
from oracle.inputs import CONFIGS, LayerConfig, make_case
from oracle.layer import reference_layer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _prefix_mask(B, S, seed, lo=0):
    r = np.random.default_rng(seed)
    lengths = r.integers(lo, S + 1, B)
    lengths[0] = S          # one full sequence
    if B > 2:
        lengths[1] = 0      # one empty sequence
    return torch.from_numpy(np.arange(S)[None, :] < lengths[:, None]).to(DEV)


@pytest.mark.parametrize("B,H,S,hd,causal", [
    (4, 2, 200, 64, False), (4, 2, 200, 64, True), (6, 4, 16, 64, False),
    (3, 2, 130, 32, False), (3, 2, 300, 128, True), (2, 1, 1, 64, False)])
def test_packed_attention_equals_padded(kernels, B, H, S, hd, causal):
    print(f"[packed attention] B={B} H={H} S={S} hd={hd} causal={causal}", flush=True)
    torch.manual_seed(B * 1000 + S + hd)
    mask = _prefix_mask(B, S, S + hd)
    pk = build_packing(mask)
    qkv = torch.randn(B, S, 3, H, hd, device=DEV).half()
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    scale = hd ** -0.5
    padded = kernels.fused_attention_forward(q, k, v, mask[:, None, None, :], causal, scale,
                                             0, 1, 0)          # [B, S, H*hd]
    packed_qkv = qkv.reshape(B * S, 3, H, hd).index_select(0, pk.idx.long())
    pq, pk_, pv = packed_qkv.unbind(1)
    packed = kernels.fused_attention_forward(pq, pk_, pv, None, causal, scale, 0, 1, 0,
                                             cu_seqlens=pk.cu, max_seqlen=S)
    assert packed.shape == (pk.t_valid, H * hd)
    want = padded.reshape(B * S, H * hd).index_select(0, pk.idx.long())
    assert torch.equal(packed, want)


def test_packed_attention_refusals(kernels):
    q = torch.zeros(8, 2, 64, device=DEV, dtype=torch.float16)
    cu = torch.tensor([0, 8], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="max_seqlen"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, cu_seqlens=cu)
    with pytest.raises(RuntimeError, match="no attn_mask"):
        kernels.fused_attention_forward(q, q, q, torch.ones(1, 1, 1, 8, dtype=torch.bool,
                                                            device=DEV),
                                        False, 0.125, cu_seqlens=cu, max_seqlen=8)
    with pytest.raises(RuntimeError, match="int32"):
        kernels.fused_attention_forward(q, q, q, None, False, 0.125, cu_seqlens=cu.long(),
                                        max_seqlen=8)


@pytest.mark.parametrize("D,kind", [(512, "split"), (512, "half"), (512, "float"),
                                    (256, "split"), (130, "float")])
def test_layernorm_gather_equals_padded(kernels, D, kind):
    B, S = 5, 37
    torch.manual_seed(D)
    x = torch.randn(B, S, D, device=DEV)
    w = torch.randn(D, device=DEV)
    b = torch.randn(D, device=DEV)
    pk = build_packing(_prefix_mask(B, S, D))
    rows, normed = kernels.fused_layernorm_rows(x, w, b, pk.idx, 1e-5, kind, True)
    x2 = x.reshape(-1, D)
    assert torch.equal(rows, x2.index_select(0, pk.idx.long()))
    if kind == "split":
        full = kernels.fused_layernorm_split(x2, w, b)
        assert torch.equal(normed, full.index_select(1, pk.idx.long()))
    else:
        full = kernels.fused_layernorm(x2, w, b, 1e-5, kind == "half")
        assert torch.equal(normed, full.index_select(0, pk.idx.long()))


@pytest.mark.parametrize("D", [512, 256, 130])
def test_add_layernorm_scatter(kernels, D):
    B, S = 6, 29
    torch.manual_seed(D + 1)
    pk = build_packing(_prefix_mask(B, S, D + 1))
    x = torch.randn(pk.t_valid, D, device=DEV)
    sub = torch.randn(pk.t_valid, D, device=DEV)
    w = torch.randn(D, device=DEV)
    b = torch.randn(D, device=DEV)
    out = kernels.fused_add_layernorm_rows(x, sub, w, b, pk.inv, 1e-5)
    assert out.shape == (B * S, D) and out.dtype == torch.float32
    _, dense = kernels.fused_add_layernorm(x, sub, w, b, 1e-5, False)
    valid = pk.inv >= 0
    assert torch.equal(out[valid], dense)
    assert torch.count_nonzero(out[~valid]) == 0


def test_row_index_out_of_range_writes_zeros(kernels):
    D = 64
    x = torch.randn(4, D, device=DEV)
    w = torch.ones(D, device=DEV)
    b = torch.zeros(D, device=DEV)
    idx = torch.tensor([3, 4, -2, 0], dtype=torch.int32, device=DEV)
    rows, normed = kernels.fused_layernorm_rows(x, w, b, idx, 1e-5, "float", True)
    assert torch.equal(rows[0], x[3]) and torch.equal(rows[3], x[0])
    assert torch.count_nonzero(rows[1:3]) == 0 and torch.count_nonzero(normed[1:3]) == 0


def _model_out(cfg, x, mask, params, packing, graph="off"):
    prev = (ocfg.ROW_PACKING, ocfg.CUDA_GRAPH)
    ocfg.ROW_PACKING, ocfg.CUDA_GRAPH = packing, graph
    try:
        model = build_model(TransformerConfig(x.shape[0], cfg.seq_len, cfg.d_model,
                                              cfg.num_heads, cfg.ffn_dim, 1, cfg.causal), params)
        xt, mt = to_device(x, mask)
        with torch.inference_mode():
            out = model(xt, mt)
        torch.cuda.synchronize()
        return out.cpu().numpy(), model, xt, mt
    finally:
        ocfg.ROW_PACKING, ocfg.CUDA_GRAPH = prev


SMALL = {
    "C2s": LayerConfig("C2s", 4, 256, 512, 8, 2048, False, "keypad", 128, 1.0, 21),
    "C5s": LayerConfig("C5s", 600, 16, 256, 4, 1024, False, "keypad", 1, 1.0, 25),
    "C3s": LayerConfig("C3s", 3, 512, 256, 4, 1024, True, "keypad", 200, 1.0, 23),
}


@pytest.mark.parametrize("name", list(SMALL))
def test_model_packed_equals_padded_path(kernels, name):
    cfg = SMALL[name]
    print(f"[model packed] {cfg}", flush=True)
    x, mask, params = make_case(cfg)
    okernels.fallback_counts.clear()
    packed, model, _, _ = _model_out(cfg, x, mask, params, "auto")
    assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    padded, _, _, _ = _model_out(cfg, x, mask, params, "off")
    np.testing.assert_array_equal(packed, padded)
    assert not np.any(packed[~mask])
    ref = reference_layer(x, mask, params, cfg).numpy()
    res = compare_outputs(ref, packed)
    assert res.passed and res.failed_elements == 0, res


def test_model_packed_non_prefix_mask(kernels):
    """A mask with holes: still the reference's answer (keys tile differently,
    so only the tolerance, not bit equality, is promised)."""
    cfg = SMALL["C2s"]
    _, _, params = make_case(cfg)
    r = np.random.default_rng(5)
    mask = r.random((cfg.batch_size, cfg.seq_len)) < 0.7
    # fresh x: make_case's x is already zero past its own prefix lengths, and
    # a valid all-zero row is a degenerate input (its final LayerNorm divides
    # by the tiny spread of an attention-only residual)
    x = r.standard_normal((cfg.batch_size, cfg.seq_len, cfg.d_model)).astype(np.float32)
    x = np.where(mask[..., None], x, 0).astype(np.float32)
    got, _, _, _ = _model_out(cfg, x, mask, params, "auto")
    assert not np.any(got[~mask])
    ref = reference_layer(x, mask, params, cfg).numpy()
    res = compare_outputs(ref, got)
    assert res.passed and res.failed_elements == 0, res


def test_packed_graph_reloads_maps_for_a_new_mask(kernels):
    """Two masks with the same valid-row count share one graph; the second
    must reload the row maps, not reuse the first mask's."""
    cfg = SMALL["C2s"]
    x, mask, params = make_case(cfg)
    B, S = mask.shape
    prev = (ocfg.ROW_PACKING, ocfg.CUDA_GRAPH)
    ocfg.ROW_PACKING, ocfg.CUDA_GRAPH = "auto", "always"
    try:
        model = build_model(TransformerConfig(B, S, cfg.d_model, cfg.num_heads, cfg.ffn_dim, 1,
                                              cfg.causal), params)
        xt, mt = to_device(x, mask)
        # the same number of valid rows, moved between two sequences
        m2 = mask.copy()
        l0, l1 = int(mask[0].sum()), int(mask[1].sum())
        shift = min(l0 - 1, S - l1, 7)
        assert shift > 0
        m2[0] = np.arange(S) < l0 - shift
        m2[1] = np.arange(S) < l1 + shift
        _, mt2 = to_device(x, m2)
        with torch.inference_mode():
            g1 = model(xt, mt).clone()
            g2 = model(xt, mt2).clone()
            g1b = model(xt, mt).clone()
        assert len(model._graphs) == 1
        ocfg.CUDA_GRAPH = "off"
        with torch.inference_mode():
            e1 = model(xt, mt)
            e2 = model(xt, mt2)
        assert torch.equal(g1, e1) and torch.equal(g1b, e1) and torch.equal(g2, e2)
        assert not torch.equal(e1, e2)
    finally:
        ocfg.ROW_PACKING, ocfg.CUDA_GRAPH = prev


@pytest.mark.parametrize("S", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_short_sequence_kernel_equals_tiled(kernels, S, hd, causal):
    """Sequences of <= 32 keys take the one-wave-per-(sequence, head) kernel;
    it must agree with the tiled kernel (forced through the pipeline knob)
    to fp16 rounding of the output, packed and padded."""
    B, H = 7, 3
    torch.manual_seed(S * 100 + hd)
    mask = _prefix_mask(B, S, S + hd, lo=1)
    pk = build_packing(mask)
    qkv = torch.randn(B, S, 3, H, hd, device=DEV).half()
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    pq, pk_, pv = qkv.reshape(B * S, 3, H, hd).index_select(0, pk.idx.long()).unbind(1)
    scale = hd ** -0.5
    outs = []
    for forced in (False, True):
        kernels.attention_set_pipeline(0, 1 if forced else 0)
        try:
            dense = kernels.fused_attention_forward(q, k, v, mask[:, None, None, :], causal,
                                                    scale, 0, 1, 0)
            packed = kernels.fused_attention_forward(pq, pk_, pv, None, causal, scale, 0, 1, 0,
                                                     cu_seqlens=pk.cu, max_seqlen=S)
            torch.cuda.synchronize()
        finally:
            kernels.attention_set_pipeline(0, 0)
        outs.append((dense.float(), packed.float()))
    (d0, p0), (d1, p1) = outs
    ulp = 2.0 ** -10
    assert (d0 - d1).abs().max().item() <= ulp * max(1.0, d1.abs().max().item())
    assert (p0 - p1).abs().max().item() <= ulp * max(1.0, p1.abs().max().item())
    # and packed equals the padded kernel on the valid rows, bit for bit
    assert torch.equal(p0, d0.reshape(B * S, H * hd).index_select(0, pk.idx.long()))
