"""The harness-compatible runner (transformer_benchmark.py), on the CPU.

Its baseline model is pinned against the oracle (the same layer, restated
independently), its chunked scoring against its own unchunked scoring, its
inputs against the reference harness's case rules, and its planning and
argument handling directly. The GPU run (accuracy PASS and timing lines on a
product preset) is in test_gpu_runner.py.
"""

import numpy as np
import pytest
import torch

import transformer_benchmark as tb
from oracle.inputs import CONFIGS, stack_layers
from oracle.layer import reference_layer


def _cfg(B=2, S=24, D=32, H=4, F=64, L=2, causal=True):
    return tb.TransformerConfig(B, S, D, H, F, L, causal)


def test_presets_table():
    assert len(tb.PRESETS) == 14 and tb.PRESETS_CAUSAL
    assert tb.find_preset("1")[0] == "1 - base"
    assert tb.find_preset("14 - seq 100000")[1:] == (32, 100000, 1024, 16, 1024, 2)
    for name, B, S, D, H, F, L in tb.PRESETS:
        assert D % H == 0 and F == D and L == (2 if name.startswith("14") else 4)
    with pytest.raises(ValueError):
        tb.find_preset("15")


def test_preset_flags_and_explicit_overrides():
    a = tb.parse_args(["--preset", "8"])
    assert (a.batch_size, a.seq_len, a.d_model, a.heads, a.ffn_dim, a.layers, a.causal) == \
        (64, 128, 1024, 4, 1024, 4, True)
    b = tb.parse_args(["--preset", "14", "--batch-size", "1", "--seq-len", "2048"])
    assert (b.batch_size, b.seq_len, b.d_model) == (1, 2048, 1024)
    c = tb.parse_args([])
    assert (c.batch_size, c.seq_len, c.d_model, c.layers, c.causal) == (8, 128, 512, 6, False)
    d = tb.parse_args(["--attn-impl", "wmma", "--qkv-precision", "fp16x3"])
    assert d.attn_impl == "wmma" and d.qkv_precision == "fp16x3"


@pytest.mark.parametrize("causal,padding", [(False, 0.0), (True, 0.0), (True, 0.5)])
def test_baseline_equals_the_oracle(causal, padding):
    """The runner's baseline and the oracle are two restatements of the same
    reference layer stack: equal to fp64 rounding."""
    cfg = _cfg(causal=causal)
    torch.manual_seed(0)
    base = tb.BaselineTransformer(cfg).double()
    x, valid = tb.make_case(cfg, torch.device("cpu"), torch.float64, 7, padding, 1.0)
    with torch.no_grad():
        got = base(x, valid if padding > 0 else None).numpy()
    params = {k: v.numpy() for k, v in base.state_dict().items()}
    ocfg = CONFIGS["C1"].__class__("t", cfg.batch_size, cfg.seq_len, cfg.d_model,
                                   cfg.num_heads, cfg.ffn_dim, cfg.causal, "none", 1, 1.0, 0)
    want = reference_layer(x.numpy(), valid.numpy() if padding > 0 else None, params, ocfg,
                           dtype=torch.float64).numpy()
    # the baseline's softmax runs in fp32 whatever the model dtype (the
    # reference harness's cast), so an fp64 run agrees to fp32 rounding
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("block", [1, 5, 16])
def test_chunked_baseline_is_the_same_arithmetic(causal, block):
    cfg = _cfg(causal=causal, S=37)
    torch.manual_seed(1)
    base = tb.BaselineTransformer(cfg).double()
    x, valid = tb.make_case(cfg, torch.device("cpu"), torch.float64, 3, 0.4, 1.0)
    with torch.no_grad():
        whole = base(x, valid)
        base.set_query_block(block)
        chunked = base(x, valid)
    # the same values up to the fp32 softmax's summation order over the
    # (causal: fewer, the dropped ones exactly 0) columns of a block
    np.testing.assert_allclose(chunked.numpy(), whole.numpy(), rtol=1e-6, atol=1e-6)


def test_state_dict_loads_strictly_into_the_optimized_model():
    base, opt = tb.build_models(_cfg(), torch.device("cpu"), torch.float32, 5)
    assert set(base.state_dict()) == set(opt.state_dict())
    for k, v in base.state_dict().items():
        assert torch.equal(v, opt.state_dict()[k])


def test_case_rules():
    cfg = _cfg(B=64, S=40)
    x, valid = tb.make_case(cfg, torch.device("cpu"), torch.float32, 11, 0.25, 2.0)
    lengths = valid.sum(1)
    assert int(lengths.min()) >= round(40 * 0.75) and int(lengths.max()) <= 40
    assert torch.equal(valid, torch.arange(40)[None, :] < lengths[:, None])
    assert torch.count_nonzero(x[~valid]) == 0
    x2, valid2 = tb.make_case(cfg, torch.device("cpu"), torch.float32, 11, 0.25, 2.0)
    assert torch.equal(x, x2) and torch.equal(valid, valid2)
    _, full = tb.make_case(cfg, torch.device("cpu"), torch.float32, 11, 0.0, 1.0)
    assert bool(full.all())


def test_element_rule():
    ref = torch.tensor([1.0, 0.0, 10.0, 1.0])
    opt = torch.tensor([1.0015, 0.0019, 10.15, float("nan")])
    r = tb.compare(ref, opt, 0.02, 0.002)
    assert r.failed == 1 and not r.passed          # the NaN
    r = tb.compare(ref[:3], opt[:3], 0.02, 0.002)
    assert r.passed
    r = tb.compare(torch.tensor([0.0]), torch.tensor([0.0021]), 0.02, 0.002)
    assert not r.passed                             # not isclose's atol + rtol * ref


def test_iteration_trimming():
    assert tb.trim_iterations(1.0, 20, 100, 3) == (20, 100, 3)
    w, r, n = tb.trim_iterations(2000.0, 20, 100, 3)     # 2 s a pass
    assert w >= 1 and r >= 3 and 1 <= n <= 3
    assert 2.0 * (w + r * n) <= tb.BENCHMARK_BUDGET_S * 1.1


def test_memory_planning(monkeypatch):
    cfg = _cfg(B=100, S=1000, D=1024, H=16, F=1024, L=2)
    monkeypatch.setattr(tb, "free_budget", lambda device: 1 << 40)
    dev = torch.device("cpu")
    assert tb.plan_slice_rows(cfg, dev, torch.float32) == 100
    assert tb.plan_query_block(cfg, dev, torch.float32, 100, 0) == 0
    monkeypatch.setattr(tb, "free_budget", lambda device: 8 << 30)
    rows = tb.plan_slice_rows(cfg, dev, torch.float32)
    assert 1 <= rows < 100
    block = tb.plan_query_block(cfg, dev, torch.float32, rows, 0)
    assert block > 0 and block & (block - 1) == 0 and block < cfg.seq_len
    assert tb.plan_query_block(cfg, dev, torch.float32, rows, 64) == 64
    assert tb.plan_query_block(cfg, dev, torch.float32, rows, -1) == 0
    monkeypatch.setattr(tb, "free_budget", lambda device: 1 << 20)
    assert tb.plan_query_block(cfg, dev, torch.float32, 1, 0) == -1
