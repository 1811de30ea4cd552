"""The committed golden fixtures agree with the oracle and the input generator.

Fixtures are data written by tests/golden/make_golden.py; these checks make
sure a change to the oracle or the generator cannot pass unnoticed.
"""

import os

import numpy as np
import pytest
import torch

from oracle.inputs import CONFIGS, make_case
from oracle.layer import gelu, layer_norm, linear, reference_attention, reference_layer

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail(f"missing fixture {name}; run tests/golden/make_golden.py")
    return np.load(path, allow_pickle=False)


def _check_inputs(fx, cfg):
    x, mask, params = make_case(cfg)
    assert x.astype(np.float64).sum() == fx["x_sum"]
    assert np.abs(x.astype(np.float64)).sum() == fx["x_abs_sum"]
    np.testing.assert_array_equal(x.reshape(-1)[:64], fx["x_head"])
    for name in ("layers.0.attention.q_proj.weight", "layers.0.ffn_out.weight"):
        assert params[name].astype(np.float64).sum() == fx["w_sum." + name]
    if mask is not None:
        np.testing.assert_array_equal(mask.sum(1), fx["lengths"])
    return x, mask, params


def test_ops_known_answers():
    k = _load("ops_kat.npz")
    d = torch.float64
    t = lambda a: torch.from_numpy(a).to(d)  # noqa: E731
    np.testing.assert_allclose(layer_norm(t(k["ln_x"]), t(k["ln_w"]), t(k["ln_b"])).numpy(),
                               k["ln_out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(linear(t(k["lin_x"]), t(k["lin_w"]), t(k["lin_b"])).numpy(),
                               k["lin_out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gelu(t(k["gelu_x"])).numpy(), k["gelu_out"], rtol=1e-13, atol=1e-15)
    q, kk, v = k["att_q"], k["att_k"], k["att_v"]
    np.testing.assert_allclose(reference_attention(q, kk, v, dtype=d).numpy(), k["att_out"],
                               atol=1e-12)
    np.testing.assert_allclose(reference_attention(q, kk, v, causal=True, dtype=d).numpy(),
                               k["att_out_causal"], atol=1e-12)
    np.testing.assert_allclose(reference_attention(q, kk, v, k["att_valid"], dtype=d).numpy(),
                               k["att_out_masked"], atol=1e-12)


def test_c1_full_output():
    fx = _load("c1_layer.npz")
    cfg = CONFIGS["C1"]
    x, mask, params = _check_inputs(fx, cfg)
    out = reference_layer(x, mask, params, cfg).numpy()
    np.testing.assert_allclose(out, fx["out32"], atol=1e-5)
    # the fp32 oracle sits within fp32 noise of the fp64 brute-force layer
    np.testing.assert_allclose(out, fx["out64"], atol=2e-5)


@pytest.mark.parametrize("name", ["C2", "C3", "C5"])
def test_sampled_rows(name):
    fx = _load(f"rows_{name}.npz")
    cfg = CONFIGS[name]
    x, mask, params = _check_inputs(fx, cfg)
    out = reference_layer(x, mask, params, cfg).numpy()
    got = np.stack([out[b, s] for b, s in fx["rows"]])
    np.testing.assert_allclose(got, fx["values"], atol=1e-5)


def test_c4_inputs():
    """C4's oracle takes minutes on a CPU; its inputs are pinned here and its
    sampled rows are checked against the GPU output in the GPU suite."""
    fx = _load("rows_C4.npz")
    _check_inputs(fx, CONFIGS["C4"])
