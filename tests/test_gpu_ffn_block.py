"""The fused post-attention block (fused_ffn_block, reference csrc/ffn_block.cuh).

Two checks per shape:
  * the fused kernel equals the unfused kernel chain (add+LayerNorm with fp16
    output, linear_gelu with fp16 output, linear_bias, add+LayerNorm) bit for
    bit: same operand roundings, same accumulation order, so fusing is a pure
    speed choice;
  * both agree with an fp64 oracle that applies the same fp16 roundings
    (LayerNorm output, weights, GELU output) within 1e-3 absolute plus 1e-3
    relative. Beyond fp32 accumulation order and GELU's 1.5e-7 in erf, an fp32
    value next to an fp16 rounding boundary can round one fp16 ulp (up to
    2e-3 at |v| ~ 2) away from the fp64 oracle's, moving an output by
    ~|w_in| |w_out| ulp ~ 2e-4.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS = 1e-5


def _params(D, F, seed):
    g = torch.Generator().manual_seed(seed)
    u = lambda *s: (torch.rand(*s, generator=g) * 2 - 1)  # noqa: E731
    p = dict(w1=1 + 0.1 * u(D), b1=0.1 * u(D), win=u(F, D) * (6 / (D + F)) ** 0.5,
             bin=0.1 * u(F), wout=u(D, F) * (6 / (D + F)) ** 0.5, bout=0.1 * u(D),
             w2=1 + 0.1 * u(D), b2=0.1 * u(D))
    return {k: v.float().to(DEV) for k, v in p.items()}


def _chain(kx, x, a, p):
    x1, n1 = kx.fused_add_layernorm(x, a, p["w1"], p["b1"], EPS, True)
    h = kx.linear_gelu(n1, p["win"], p["bin"], -1, -1, True)
    y = kx.linear_bias(h, p["wout"], p["bout"], -1, -1, False)
    return kx.fused_add_layernorm(x1, y, p["w2"], p["b2"], EPS, False)


def _oracle(x, a, p):
    """fp64, with the kernels' fp16 roundings applied where they happen."""
    d = {k: v.double().cpu() for k, v in p.items()}
    r16 = lambda t: t.half().double()  # noqa: E731
    x1 = (x + a).double().cpu()   # the kernels' fp32 add, then exact

    def ln(t, w, b):
        m = t.mean(-1, keepdim=True)
        var = ((t - m) ** 2).mean(-1, keepdim=True)
        return (t - m) / torch.sqrt(var + EPS) * w + b

    n1 = r16(ln(x1, d["w1"], d["b1"]))
    z = n1 @ r16(d["win"]).T + d["bin"]
    h = r16(0.5 * z * (1 + torch.erf(z / 2 ** 0.5)))
    x2 = x1 + (h @ r16(d["wout"]).T + d["bout"])
    return x2, ln(x2, d["w2"], d["b2"])


SHAPES = [(16, 16), (32, 32), (48, 48), (64, 64), (128, 128), (40, 96), (128, 24), (8, 8),
          # d_ff above 128: the padded 256 and 512 instances (C1 is 128 x 512)
          (128, 512), (64, 256), (128, 384), (96, 200)]


@pytest.mark.parametrize("rows", [1, 64, 130, 1000])
@pytest.mark.parametrize("D,F", SHAPES)
def test_fused_block_equals_chain_and_oracle(kernels, D, F, rows):
    torch.manual_seed(rows * 7 + D)
    x = torch.randn(rows, D, device=DEV)
    a = torch.randn(rows, D, device=DEV) * 0.5
    p = _params(D, F, D * 131 + F)
    got = kernels.fused_ffn_block(x, a, p["w1"], p["b1"], p["win"], p["bin"], p["wout"],
                                  p["bout"], p["w2"], p["b2"], EPS)
    assert len(got) == 2
    x2, n2 = got
    cx2, cn2 = _chain(kernels, x, a, p)
    assert torch.equal(x2, cx2) and torch.equal(n2, cn2)
    ox2, on2 = _oracle(x, a, p)
    np.testing.assert_allclose(x2.cpu().numpy(), ox2.numpy(), atol=1e-3, rtol=1e-3)
    np.testing.assert_allclose(n2.cpu().numpy(), on2.numpy(), atol=1e-3, rtol=1e-3)


def test_fused_block_batched_shape_and_declines(kernels):
    D = F = 64
    x = torch.randn(3, 50, D, device=DEV)
    a = torch.randn(3, 50, D, device=DEV)
    p = _params(D, F, 1)
    x2, n2 = kernels.fused_ffn_block(x, a, p["w1"], p["b1"], p["win"], p["bin"], p["wout"],
                                     p["bout"], p["w2"], p["b2"], EPS)
    assert x2.shape == x.shape and n2.shape == x.shape
    cx2, cn2 = _chain(kernels, x.view(-1, D), a.view(-1, D), p)
    assert torch.equal(x2.view(-1, D), cx2) and torch.equal(n2.view(-1, D), cn2)
    # widths outside the kernel: the empty-list decline
    pw = _params(256, 256, 2)
    xw = torch.randn(4, 256, device=DEV)
    assert kernels.fused_ffn_block(xw, xw, pw["w1"], pw["b1"], pw["win"], pw["bin"], pw["wout"],
                                   pw["bout"], pw["w2"], pw["b2"], EPS) == []
    pw = _params(128, 640, 3)
    xw = torch.randn(4, 128, device=DEV)
    assert kernels.fused_ffn_block(xw, xw, pw["w1"], pw["b1"], pw["win"], pw["bin"], pw["wout"],
                                   pw["bout"], pw["w2"], pw["b2"], EPS) == []
    with pytest.raises(RuntimeError, match="must match"):
        kernels.fused_ffn_block(x, a[:1], p["w1"], p["b1"], p["win"], p["bin"], p["wout"],
                                p["bout"], p["w2"], p["b2"], EPS)


def test_model_uses_fused_block_with_same_output(kernels):
    """A narrow layer (d_model 64 = the "auto" gate) runs the fused block; the
    model's output equals FFN_BLOCK="off" exactly and passes the layer oracle."""
    from layer_runner import TransformerConfig, build_model, to_device
    import optimized.layers as olayers
    from optimized import config as ocfg
    from oracle.compare import compare_outputs
    from oracle.inputs import LayerConfig, make_case
    from oracle.layer import reference_layer

    cfg = LayerConfig("narrow", 3, 40, 64, 2, 64, False, "none", 40, 1.0, 9)
    x, mask, params = make_case(cfg)
    tcfg = TransformerConfig(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads,
                             cfg.ffn_dim, 1, cfg.causal)
    saved = (ocfg.FFN_BLOCK, ocfg.CUDA_GRAPH)
    outs = {}
    try:
        ocfg.CUDA_GRAPH = "off"
        for mode in ("auto", "off"):
            ocfg.FFN_BLOCK = mode
            model = build_model(tcfg, params)
            xt, mt = to_device(x, mask)
            calls = []
            orig = olayers._ffn_block

            def spy(*a, **k):
                r = orig(*a, **k)
                calls.append(r is not None)
                return r

            olayers._ffn_block = spy
            try:
                with torch.inference_mode():
                    outs[mode] = model(xt, mt).cpu()
            finally:
                olayers._ffn_block = orig
            if mode == "auto":
                assert calls == [True]
    finally:
        ocfg.FFN_BLOCK, ocfg.CUDA_GRAPH = saved
    assert torch.equal(outs["auto"], outs["off"])
    ref = reference_layer(x, mask, params, cfg).numpy()
    assert compare_outputs(ref, outs["auto"].numpy()).passed
