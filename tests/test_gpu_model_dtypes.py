"""The whole model with float16 and bfloat16 tensors (the harness's --dtype,
reference torch_transformer_benchmark.py:314-320), on the GPU.

The model is cast to the dtype (weights, LayerNorm parameters, biases) and
fed the input in that dtype; every kernel then keeps it: LayerNorm and
add+LayerNorm with fp32 statistics, one-pass fp16 / bf16 MFMA GEMMs, attention
contracting in the tensor dtype, the residual stream in the tensor dtype. The
check is against the fp32 oracle on the same 16-bit-rounded weights and
input, so what is measured is the 16-bit arithmetic itself. Its error budget
is set by the residual stream's rounding (|h| reaches a few units, rounded at
every add): for fp16 (unit roundoff 2^-11) |err| <= 1e-2 or 2% relative; for
bf16 (2^-8) |err| <= 6e-2 or 6% relative. No torch fallback may run.
"""

import os

import numpy as np
import pytest
import torch

from layer_runner import TransformerConfig
from optimized import OptimizedTransformer
from optimized import kernels as okernels
from oracle.compare import compare_outputs
from oracle.inputs import CONFIGS, make_case, stack_layers
from oracle.layer import reference_layer

pytestmark = pytest.mark.gpu

TOL = {torch.float16: (1e-2, 0.02), torch.bfloat16: (6e-2, 0.06)}


def _rounded(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).float().numpy()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("name,batch,layers", [("C1", None, 1), ("C2", None, 1), ("C1", None, 2),
                                               ("C5", 2000, 1), ("C3", None, 1)])
def test_model_16bit(kernels, dtype, name, batch, layers):
    cfg = CONFIGS[name]
    print(f"[16-bit model] {name} batch={batch} layers={layers} {dtype}", flush=True)
    x, mask, params = make_case(cfg, batch=batch)
    params = stack_layers(params, layers)
    p16 = {k: _rounded(v, dtype) for k, v in params.items()}
    x16 = _rounded(x, dtype)
    B = x.shape[0]
    model = OptimizedTransformer(TransformerConfig(B, cfg.seq_len, cfg.d_model, cfg.num_heads,
                                                   cfg.ffn_dim, layers, cfg.causal))
    model.load_state_dict({k: torch.from_numpy(v) for k, v in p16.items()}, strict=True)
    model = model.to(device="cuda", dtype=dtype).eval()
    xt = torch.from_numpy(x16).to("cuda", dtype)
    mt = None if mask is None else torch.from_numpy(mask).cuda()
    okernels.fallback_counts.clear()
    with torch.inference_mode():
        out = model(xt, mt)
    assert out.dtype == dtype
    assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = reference_layer(x16, mask, p16, cfg).numpy()
    atol, rtol = TOL[dtype]
    res = compare_outputs(ref, out.float().cpu().numpy(), atol=atol, rtol=rtol)
    print(f"[16-bit model] {name} L={layers} {dtype}: failed={res.failed_elements}/"
          f"{res.total_elements} max_abs={res.max_abs_error:.3e} "
          f"mean_abs={res.mean_abs_error:.3e}", flush=True)
    assert res.passed, res
    if mask is not None:
        assert torch.count_nonzero(out.float().cpu()[~torch.from_numpy(mask)]) == 0
