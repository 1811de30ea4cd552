"""Whole-layer parity on the GPU at all five configs, plus graph replay.

The optimized model (optimized/ on libdotl_hip.so) runs the layer on the
device; the oracle runs the reference layer on this machine's CPU cores on the
same seeded inputs; every element must pass the harness rule (finite AND
|err| <= 2e-3 OR |err| <= 2% |ref|) with zero failures, which is the north-star
gate. The committed golden rows are checked too, so a box whose CPU oracle
disagreed with the one that wrote them would be caught.
"""

import os

import numpy as np
import pytest
import torch

import kernel_ext
from layer_runner import TransformerConfig, build_model, to_device
from optimized import config as ocfg
from optimized import kernels as okernels
from oracle.compare import compare_outputs, gate_ratio
from oracle.inputs import CONFIGS, make_case, stack_layers as params_for
from oracle.layer import reference_layer

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Margin regression bound: the share of the 2e-3 / 2% allowance the worst
# element may use. Measured on MI355X with the default arithmetic: C4 0.76,
# C5 0.77, C3 0.49, C2 0.52 (C4 seed 404: 0.77, C5 seed 505: 0.72); the tail
# comes from the FFN GEMMs' fp16 operands (both in the split fp16x3
# arithmetic, C4 drops to 0.09). A change that eats into the margin fails
# here before it can fail the rule on another draw.
MAX_GATE_RATIO = 0.85


def _tcfg(cfg, batch=None, layers=1):
    return TransformerConfig(batch or cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads,
                             cfg.ffn_dim, layers, cfg.causal)


def _run_gpu(cfg, x, mask, params, graph="off"):
    prev = ocfg.CUDA_GRAPH
    ocfg.CUDA_GRAPH = graph
    try:
        model = build_model(_tcfg(cfg, x.shape[0]), params)
        xt, mt = to_device(x, mask)
        with torch.inference_mode():
            out = model(xt, mt)
        torch.cuda.synchronize()
        return out.cpu().numpy(), model
    finally:
        ocfg.CUDA_GRAPH = prev


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_layer_parity(kernels, name):
    cfg = CONFIGS[name]
    print(f"[layer parity] {name} {cfg}", flush=True)
    x, mask, params = make_case(cfg)
    okernels.fallback_counts.clear()
    got, _ = _run_gpu(cfg, x, mask, params)
    assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = reference_layer(x, mask, params, cfg).numpy()
    res = compare_outputs(ref, got)
    gate = gate_ratio(ref, got)
    print(f"[layer parity] {name}: failed={res.failed_elements}/{res.total_elements} "
          f"max_abs={res.max_abs_error:.3e} mean_abs={res.mean_abs_error:.3e} "
          f"gate={gate:.3f} worst={res.worst_index}", flush=True)
    assert res.passed, res
    assert gate <= MAX_GATE_RATIO, f"{name}: the worst element uses {gate:.3f} of the allowance"
    if mask is not None:
        assert np.all(got[~mask] == 0.0)
    fx = np.load(os.path.join(GOLDEN, f"rows_{name}.npz" if name != "C1" else "c1_layer.npz"),
                 allow_pickle=False)
    if name == "C1":
        assert compare_outputs(fx["out64"], got).passed
    else:
        rows = np.stack([got[b, s] for b, s in fx["rows"]])
        assert compare_outputs(fx["values"], rows).passed


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name,seed,batch", [("C2", 101, None), ("C2", 202, None),
                                             ("C3", 303, None), ("C4", 404, 1),
                                             ("C5", 505, 3000), ("C5", 606, 3000)])
def test_layer_parity_other_seeds(kernels, name, seed, batch):
    """The north-star rule on freshly drawn inputs and weights beyond the fixed
    seeds (C4 at one sequence, C5 at 3000, to keep the CPU oracle short): zero
    failing elements, so the fp16 margin is not a property of one draw."""
    cfg = CONFIGS[name]
    x, mask, params = make_case(cfg, seed=seed, batch=batch)
    print(f"[layer parity, seed {seed}] {name} batch {x.shape[0]}", flush=True)
    okernels.fallback_counts.clear()
    got, _ = _run_gpu(cfg, x, mask, params)
    assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = reference_layer(x, mask, params, cfg).numpy()
    res = compare_outputs(ref, got)
    gate = gate_ratio(ref, got)
    print(f"[layer parity, seed {seed}] {name}: failed={res.failed_elements}/{res.total_elements} "
          f"max_abs={res.max_abs_error:.3e} gate={gate:.3f}", flush=True)
    assert res.passed, res
    assert gate <= MAX_GATE_RATIO, f"{name} seed {seed}: the worst element uses {gate:.3f}"
    if mask is not None:
        assert np.all(got[~mask] == 0.0)


@pytest.mark.parametrize("name", ["C1", "C2"])
def test_layer_nonzero_affine(kernels, name):
    """Non-zero biases and LayerNorm affine exercise every epilogue term."""
    cfg = CONFIGS[name]
    x, mask, params = make_case(cfg, batch=2, nonzero_affine=True)
    got, _ = _run_gpu(cfg, x, mask, params)
    ref = reference_layer(x, mask, params, cfg).numpy()
    res = compare_outputs(ref, got)
    assert res.passed, res


def test_layer_precision_knobs(kernels):
    """All-fp16 arithmetic still passes at C1; the fp32-class split path is far tighter."""
    cfg = CONFIGS["C1"]
    x, mask, params = make_case(cfg)
    ref = reference_layer(x, mask, params, cfg).numpy()
    saved = (ocfg.QKV_PRECISION, ocfg.LINEAR_BIAS, ocfg.LINEAR_GELU)
    try:
        ocfg.QKV_PRECISION = "fp16"
        fast, _ = _run_gpu(cfg, x, mask, params)
        ocfg.QKV_PRECISION, ocfg.LINEAR_BIAS, ocfg.LINEAR_GELU = "fp16x3", "tf32", "tf32"
        tight, _ = _run_gpu(cfg, x, mask, params)
    finally:
        ocfg.QKV_PRECISION, ocfg.LINEAR_BIAS, ocfg.LINEAR_GELU = saved
    r_fast, r_tight = compare_outputs(ref, fast), compare_outputs(ref, tight)
    assert r_fast.passed and r_tight.passed
    assert r_tight.max_abs_error < r_fast.max_abs_error


@pytest.mark.parametrize("name", ["C1", "C2"])
def test_layer_fp32_class_end_to_end(kernels, name):
    """Exact fp32 attention (ATTENTION_PRECISION="fp32", the scalar kernel; at C2
    over packed rows) with the split fp16x3 GEMMs: the whole layer at fp32-class
    error. Bound: 5e-5 absolute, against ~1e-3 for the fp16 path."""
    cfg = CONFIGS[name]
    x, mask, params = make_case(cfg, batch=2)
    ref = reference_layer(x, mask, params, cfg).numpy()
    saved = (ocfg.ATTENTION_PRECISION, ocfg.LINEAR_BIAS, ocfg.LINEAR_GELU)
    try:
        ocfg.LINEAR_BIAS, ocfg.LINEAR_GELU = "tf32", "tf32"
        half_attn, _ = _run_gpu(cfg, x, mask, params)
        ocfg.ATTENTION_PRECISION = "fp32"
        okernels.fallback_counts.clear()
        exact, _ = _run_gpu(cfg, x, mask, params)
        assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    finally:
        ocfg.ATTENTION_PRECISION, ocfg.LINEAR_BIAS, ocfg.LINEAR_GELU = saved
    r_half, r_exact = compare_outputs(ref, half_attn), compare_outputs(ref, exact)
    print(f"[fp32-class] {name}: fp16 attention max_abs={r_half.max_abs_error:.3e}, "
          f"fp32 attention max_abs={r_exact.max_abs_error:.3e}", flush=True)
    assert r_exact.passed and r_exact.max_abs_error < 5e-5
    assert r_exact.max_abs_error < r_half.max_abs_error
    if mask is not None:
        assert np.all(exact[~mask] == 0.0)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name,batch,layers,packing", [
    ("C1", None, 2, "auto"), ("C1", None, 4, "auto"), ("C2", None, 2, "auto"),
    ("C2", None, 4, "auto"), ("C2", 4, 2, "off"), ("C5", 3000, 2, "auto"),
    ("C5", 3000, 4, "auto"), ("C3", None, 2, "auto")])
def test_multi_layer_parity(kernels, name, batch, layers, packing):
    """L stacked blocks against the oracle's L-block model: the cross-layer
    edges (the next block's norm1 fused into this block's last add, as split
    fp16 planes for the QKV projection; packed rows kept between blocks) and
    the final norm. Zero failing elements at 2e-3 / 2%."""
    cfg = CONFIGS[name]
    print(f"[multi-layer parity] {name} batch={batch} layers={layers} packing={packing}",
          flush=True)
    x, mask, params = make_case(cfg, batch=batch)
    p_l = params_for(params, layers)
    saved = ocfg.ROW_PACKING
    ocfg.ROW_PACKING = packing
    try:
        okernels.fallback_counts.clear()
        got = _eager_out(cfg, x, mask, params, layers)
        assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    finally:
        ocfg.ROW_PACKING = saved
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = reference_layer(x, mask, p_l, cfg).numpy()
    res = compare_outputs(ref, got)
    print(f"[multi-layer parity] {name} L={layers}: failed={res.failed_elements}/"
          f"{res.total_elements} max_abs={res.max_abs_error:.3e} "
          f"mean_abs={res.mean_abs_error:.3e}", flush=True)
    assert res.passed, res
    if mask is not None:
        assert np.all(got[~mask] == 0.0)


def _eager_out(cfg, x, mask, params, layers=1):
    prev = ocfg.CUDA_GRAPH
    ocfg.CUDA_GRAPH = "off"
    try:
        model = build_model(_tcfg(cfg, x.shape[0], layers), params_for(params, layers))
        xt, mt = to_device(x, mask)
        with torch.inference_mode():
            return model(xt, mt).cpu().numpy()
    finally:
        ocfg.CUDA_GRAPH = prev


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name,batch,layers,packing", [
    ("C1", None, 1, "auto"), ("C1", None, 2, "auto"), ("C2", None, 1, "auto"),
    ("C2", 4, 1, "off"), ("C3", None, 1, "auto"), ("C5", None, 1, "auto")])
def test_graph_replay_matches_eager(kernels, name, batch, layers, packing):
    """A captured forward equals the eager forward bit for bit, on repeated
    replays with eager work and synchronisations between them, and a fresh
    input reaches the graph. Full C1/C2/C3/C5 shapes; the packed path binds
    input and output to the graph's I/O slot, the masked path with row
    packing off copies them."""
    cfg = CONFIGS[name]
    print(f"[graph replay] {name} batch={batch} layers={layers} packing={packing}", flush=True)
    x, mask, params = make_case(cfg, batch=batch)
    saved = (ocfg.CUDA_GRAPH, ocfg.ROW_PACKING)
    ocfg.ROW_PACKING = packing
    try:
        eager = _eager_out(cfg, x, mask, params, layers)
        ocfg.CUDA_GRAPH = "always"
        model = build_model(_tcfg(cfg, x.shape[0], layers), params_for(params, layers))
        xt, mt = to_device(x, mask)
        with torch.inference_mode():
            outs = []
            for i in range(4):
                outs.append(model(xt, mt).cpu().numpy())
                _ = torch.randn(1000, device="cuda").sum().item()  # eager work in between
            assert len(model._graphs) == 1, model._graph_log
            (log,) = model._graph_log.values()
            runner = next(iter(model._graphs.values()))
            assert runner.replays == 4
            # the entry norm always reads the bound input; the output is bound
            # unless the forward ends in masked_fill (the masked padded path)
            assert runner.in_bound, log
            assert runner.out_bound == (packing == "auto" or mask is None), log
            x2, _, _ = make_case(cfg, seed=555, batch=x.shape[0])
            if mask is not None:
                x2 = np.where(mask[..., None], x2, 0).astype(np.float32)
            out2 = model(to_device(x2, mask)[0], mt).cpu().numpy()
        eager2 = _eager_out(cfg, x2, mask, params, layers)
    finally:
        ocfg.CUDA_GRAPH, ocfg.ROW_PACKING = saved
    print(f"[graph replay] {name}: {log}", flush=True)
    for o in outs:
        np.testing.assert_array_equal(o, eager)
    np.testing.assert_array_equal(out2, eager2)


@pytest.mark.parametrize("name", ["C1", "C2"])
def test_graph_auto_keeps_only_a_faster_graph(kernels, name):
    """In "auto" every capture is timed against eager and the outcome logged;
    a kept graph measured faster, a declined one not, and the output is the
    eager one either way."""
    cfg = CONFIGS[name]
    x, mask, params = make_case(cfg)
    eager = _eager_out(cfg, x, mask, params)
    prev = ocfg.CUDA_GRAPH
    ocfg.CUDA_GRAPH = "auto"
    try:
        model = build_model(_tcfg(cfg), params)
        xt, mt = to_device(x, mask)
        with torch.inference_mode():
            got = [model(xt, mt).cpu().numpy() for _ in range(2)]
    finally:
        ocfg.CUDA_GRAPH = prev
    (log,) = model._graph_log.values()
    print(f"[graph auto] {name}: {log}", flush=True)
    assert "eager_us" in log and "replay_us" in log
    kept = log["replay_us"] <= log["eager_us"] * (1.0 - ocfg._GRAPH_MIN_GAIN)
    assert (log["outcome"] == "captured") == kept
    assert (len(model._graphs) == 1) == (log["outcome"] == "captured")
    for g in got:
        np.testing.assert_array_equal(g, eager)


def test_native_library_is_loaded(kernels):
    """The product path runs libdotl_hip.so from the source tree, not a fallback."""
    maps = open("/proc/self/maps").read()
    assert kernel_ext.library_path() in maps


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_residual_epilogue_is_bit_identical(kernels, name):
    """out_proj and ffn_out adding the residual stream in their epilogues, then
    plain LayerNorms or (rows of <= 256: C1, C5) the LayerNorms in the same
    epilogues, give the add+LayerNorm chain's output bit for bit, on the
    unpadded (C1, C3) and packed-row (C2, C5) paths; no torch fallback runs."""
    cfg = CONFIGS[name]
    x, mask, params = make_case(cfg, batch=min(cfg.batch_size, 64))
    saved = (ocfg.RESIDUAL_EPILOGUE, ocfg._RESIDUAL_EPILOGUE_MIN_D, ocfg.LN_EPILOGUE,
             ocfg._LN_EPILOGUE_MIN_ROWS)
    try:
        outs = {}
        ocfg._RESIDUAL_EPILOGUE_MIN_D = 0   # every width, whatever the default threshold
        ocfg._LN_EPILOGUE_MIN_ROWS = 0      # every row count, likewise
        # residual epilogue with the LayerNorms in the same epilogues (C1,
        # C5: rows of <= 256), with separate LayerNorms, and neither
        for mode, ln in (("auto", "auto"), ("auto", "off"), ("off", "off")):
            ocfg.RESIDUAL_EPILOGUE, ocfg.LN_EPILOGUE = mode, ln
            okernels.fallback_counts.clear()
            outs[(mode, ln)], _ = _run_gpu(cfg, x, mask, params)
            assert not okernels.fallback_counts, dict(okernels.fallback_counts)
    finally:
        (ocfg.RESIDUAL_EPILOGUE, ocfg._RESIDUAL_EPILOGUE_MIN_D, ocfg.LN_EPILOGUE,
         ocfg._LN_EPILOGUE_MIN_ROWS) = saved
    assert np.array_equal(outs[("auto", "auto")], outs[("off", "off")])
    assert np.array_equal(outs[("auto", "off")], outs[("off", "off")])
    assert compare_outputs(reference_layer(x, mask, params, cfg).numpy(),
                           outs[("auto", "auto")]).passed
