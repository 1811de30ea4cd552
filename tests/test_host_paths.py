"""Host-side failure handling of the optimized package, forced on the CPU.

The memory-pressure ladder (an out-of-memory error raised from a stand-in
forward), kernel declines (a fake extension answering None / []), and graph
capture that is refused or fails. None of these needs a device: each test
replaces exactly the piece that would touch one.
"""

import math

import pytest
import torch

import optimized.graphs as graphs
import optimized.kernels as okernels
import optimized.model as omodel
from layer_runner import TransformerConfig
from optimized import config


def _model(B=8, S=4, D=16, H=2, F=32, L=1):
    return omodel.OptimizedTransformer(TransformerConfig(B, S, D, H, F, L, False))


# -- memory planning ----------------------------------------------------------

def test_plan_batch_chunks():
    assert omodel.plan_batch_chunks(8, 100, 10_000) == 1
    assert omodel.plan_batch_chunks(8, 100, 400) == 2          # 800 B into 400 B
    assert omodel.plan_batch_chunks(8, 100, 399) == 3
    assert omodel.plan_batch_chunks(8, 100, 1) == 8            # never below one row a chunk
    assert omodel.plan_batch_chunks(8, 100, 10_000, min_chunks=4) == 4
    assert omodel.plan_batch_chunks(1, 10**9, 1) == 1


def test_forward_bytes_per_token_bounds_every_dtype():
    fp32 = omodel.forward_bytes_per_token(512, 2048, 4)
    assert omodel.forward_bytes_per_token(512, 2048, 2) <= fp32
    assert omodel.forward_bytes_per_token(1024, 2048, 4) > fp32
    assert omodel.forward_bytes_per_token(512, 4096, 4) > fp32
    # at least the residual stream, the output and the FFN hidden activation
    assert fp32 >= 512 * 4 * 2 + 2048 * 2


def _fake_forward(limit_rows, calls):
    """A forward that runs out of memory above `limit_rows` sequences and
    otherwise returns x * 2 (+ 1 on masked-out positions)."""
    def fwd(x, mask, use_mask, packing=None):
        calls.append(x.shape[0])
        if x.shape[0] > limit_rows:
            raise torch.OutOfMemoryError("simulated")
        out = x * 2
        if mask is not None:
            out = out + (~mask)[..., None].to(out.dtype)
        return out
    return fwd


def test_oom_ladder_doubles_chunks_and_remembers():
    m = _model(B=8)
    calls = []
    m._forward_eager = _fake_forward(2, calls)
    m._free_device_bytes = lambda x: 1 << 50
    x = torch.randn(8, 4, 16)
    out = m._forward_chunk_on_oom(x, None, False)
    assert torch.equal(out, x * 2)
    # 1 chunk (8 rows) fails, 2 chunks (4 rows) fail, 4 chunks of 2 succeed
    assert calls[:2] == [8, 4] and calls[2:] == [2, 2, 2, 2]
    key = (tuple(x.shape), x.dtype, False, False)
    assert m._chunks[key] == 4
    calls.clear()
    assert torch.equal(m._forward_chunk_on_oom(x, None, False), x * 2)
    assert calls == [2, 2, 2, 2]            # the settled count, no retries


def test_oom_ladder_slices_the_mask_with_the_batch():
    m = _model(B=6)
    calls = []
    m._forward_eager = _fake_forward(2, calls)
    m._free_device_bytes = lambda x: 1 << 50
    x = torch.randn(6, 4, 16)
    mask = torch.rand(6, 4) > 0.3
    out = m._forward_chunk_on_oom(x, mask, True)
    assert torch.equal(out, x * 2 + (~mask)[..., None].float())


def test_oom_at_one_sequence_a_chunk_is_raised():
    m = _model(B=4)
    m._forward_eager = _fake_forward(0, [])
    m._free_device_bytes = lambda x: 1 << 50
    with pytest.raises(torch.OutOfMemoryError):
        m._forward_chunk_on_oom(torch.randn(4, 4, 16), None, False)


def test_plan_chunks_before_any_oom():
    m = _model(B=8, S=4, D=16, F=32)
    calls = []
    m._forward_eager = _fake_forward(100, calls)
    per_row = 4 * omodel.forward_bytes_per_token(16, 32, 4)
    m._free_device_bytes = lambda x: 3 * per_row       # room for three sequences
    x = torch.randn(8, 4, 16)
    assert torch.equal(m._forward_chunk_on_oom(x, None, False), x * 2)
    assert calls == [3, 3, 2]                          # ceil(8 / 3) chunks, planned up front


def test_uneven_last_chunk():
    m = _model(B=5)
    calls = []
    m._forward_eager = _fake_forward(2, calls)
    m._free_device_bytes = lambda x: 1 << 50
    x = torch.randn(5, 4, 16)
    assert torch.equal(m._forward_chunk_on_oom(x, None, False), x * 2)
    assert sum(calls[-math.ceil(5 / 2):]) == 5


# -- kernel declines ----------------------------------------------------------

class _DecliningKernels:
    """An extension that declines every GEMM and the fused FFN block."""

    def linear_bias(self, *a, **k):
        return None

    def linear_gelu(self, *a, **k):
        return None

    def fused_ffn_block(self, *a, **k):
        return []


class _ResidualDecliningKernels(_DecliningKernels):
    """Runs plain GEMMs but declines the residual epilogue."""

    def linear_bias(self, x, weight, bias, tile=-1, math=-1, out_half=False, residual=None):
        if residual is not None:
            return None
        return torch.nn.functional.linear(x, weight, bias)


@pytest.fixture
def fallbacks(monkeypatch):
    okernels.fallback_counts.clear()
    yield okernels.fallback_counts
    okernels.fallback_counts.clear()


def test_declined_gemm_falls_back_and_is_counted(monkeypatch, fallbacks):
    monkeypatch.setattr(okernels, "_custom_kernels", lambda: _DecliningKernels())
    x, w, b = torch.randn(5, 16), torch.randn(8, 16), torch.randn(8)
    got = okernels._linear_bias(x, w, b)
    assert torch.allclose(got, torch.nn.functional.linear(x, w, b))
    assert fallbacks["linear_bias"] == 1
    lin = torch.nn.Linear(16, 8)
    got = okernels._linear_gelu(x, lin)
    assert torch.allclose(got, torch.nn.functional.gelu(lin(x)))
    assert fallbacks["linear_gelu"] == 1


def test_declined_residual_epilogue_adds_on_the_host(monkeypatch, fallbacks):
    monkeypatch.setattr(okernels, "_custom_kernels", lambda: _ResidualDecliningKernels())
    x, w, b, r = torch.randn(5, 16), torch.randn(8, 16), torch.randn(8), torch.randn(5, 8)
    got = okernels._linear_bias(x, w, b, residual=r)
    assert torch.allclose(got, r + torch.nn.functional.linear(x, w, b))
    assert fallbacks["linear_bias_residual"] == 1 and fallbacks["linear_bias"] == 0


def test_declined_ffn_block_runs_unfused(monkeypatch):
    monkeypatch.setattr(okernels, "_custom_kernels", lambda: _DecliningKernels())
    norm = omodel.MyLayerNorm(16)
    ffn_in, ffn_out = torch.nn.Linear(16, 32), torch.nn.Linear(32, 16)
    x = torch.randn(4, 16)
    assert okernels._ffn_block(x, x, norm, ffn_in, ffn_out, norm) is None


def test_fused_ffn_gate(monkeypatch):
    """_ffn_ln_wanted: the one-kernel FFN exactly where the two GEMMs it
    replaces would be the one-pass GELU GEMM (fp16 out) and the GEMM with the
    LayerNorm epilogue, at d_model 256 and d_ff a multiple of 64 up to 2048."""
    rows = config._LN_EPILOGUE_MIN_ROWS
    x = torch.empty(rows, 256, dtype=torch.float16)
    ffn_in, ffn_out = torch.nn.Linear(256, 1024), torch.nn.Linear(1024, 256)
    assert okernels._ffn_ln_wanted(x, ffn_in, ffn_out)
    assert not okernels._ffn_ln_wanted(x.float(), ffn_in, ffn_out)            # fp32 input
    assert not okernels._ffn_ln_wanted(x[: rows - 1], ffn_in, ffn_out)         # too few rows
    x128 = torch.empty(rows, 128, dtype=torch.float16)
    assert not okernels._ffn_ln_wanted(x128, torch.nn.Linear(128, 512),
                                       torch.nn.Linear(512, 128))              # d_model 128
    for d_ff in (96, 4096):                                                    # d_ff % 64, > 2048
        assert not okernels._ffn_ln_wanted(x, torch.nn.Linear(256, d_ff),
                                           torch.nn.Linear(d_ff, 256))
    assert not okernels._ffn_ln_wanted(x, torch.nn.Linear(256, 1024, bias=False), ffn_out)
    for knob, value in (("FFN_LN", "off"), ("LN_EPILOGUE", "off"), ("LINEAR_GELU", "tf32"),
                        ("GELU_FP16", "off")):
        monkeypatch.setattr(config, knob, value)
        assert not okernels._ffn_ln_wanted(x, ffn_in, ffn_out), knob
        monkeypatch.undo()


class _FfnKernels:
    """Records the fused FFN call; declines (None) when asked to."""

    def __init__(self, decline):
        self.decline, self.calls = decline, []

    def ffn_layernorm(self, x, *a, **k):
        self.calls.append(k)
        if self.decline:
            return None
        rows = x.shape[0]
        return None, torch.full((rows, 256), 7.0)


def test_fused_ffn_used_where_wanted(monkeypatch):
    kx = _FfnKernels(decline=False)
    monkeypatch.setattr(okernels, "_custom_kernels", lambda: kx)
    monkeypatch.setattr(okernels, "_ffn_ln_wanted", lambda *a: True)
    norm = omodel.MyLayerNorm(256)
    x = torch.empty(4, 256, dtype=torch.float16)
    h, out = okernels._ffn_norm(x, torch.nn.Linear(256, 1024), torch.nn.Linear(1024, 256),
                                torch.zeros(4, 256), norm, "float", store_out=False)
    assert h is None and bool((out == 7.0).all())
    assert kx.calls and kx.calls[0]["normed"] == "float"


def test_declined_fused_ffn_runs_the_two_gemms(monkeypatch):
    kx = _FfnKernels(decline=True)
    monkeypatch.setattr(okernels, "_custom_kernels", lambda: kx)
    monkeypatch.setattr(okernels, "_ffn_ln_wanted", lambda *a: True)
    seen = []
    monkeypatch.setattr(okernels, "_linear_gelu", lambda x, lin, out_half=False: seen.append("gelu") or x)
    monkeypatch.setattr(okernels, "_linear_norm",
                        lambda hidden, lin, r, norm, kind, *a, **k: seen.append("norm") or ("h", "n"))
    x = torch.empty(4, 256, dtype=torch.float16)
    got = okernels._ffn_norm(x, torch.nn.Linear(256, 1024), torch.nn.Linear(1024, 256),
                             torch.zeros(4, 256), omodel.MyLayerNorm(256), "float")
    assert len(kx.calls) == 1 and seen == ["gelu", "norm"] and got == ("h", "n")


def test_attention_without_the_library_raises(monkeypatch):
    import kernel_ext

    monkeypatch.setattr(kernel_ext, "get_kernels", lambda verbose=False: None)
    q = torch.zeros(1, 1, 4, 32)
    with pytest.raises(RuntimeError, match="libdotl_hip.so"):
        okernels._attention_dispatch(q, q, q, None, False, 1.0)


# -- graph capture refused or failing -----------------------------------------

def test_cpu_tensors_are_never_captured():
    assert not graphs._graph_eligible(torch.zeros(2, 4, 16), 0)


class _DeviceTensorStandIn:
    """What _graph_eligible reads of a [2, 4, 16] tensor on cuda:0."""

    device = torch.device("cuda", 0)

    def dim(self):
        return 3

    def numel(self):
        return 2 * 4 * 16


def test_knob_off_and_entry_cap(monkeypatch):
    monkeypatch.setattr(graphs.torch.cuda, "is_current_stream_capturing", lambda: False)
    x = _DeviceTensorStandIn()
    monkeypatch.setattr(config, "CUDA_GRAPH", "off")
    assert not graphs._graph_eligible(x, 0)
    monkeypatch.setattr(config, "CUDA_GRAPH", "auto")
    assert graphs._graph_eligible(x, 0)
    assert not graphs._graph_eligible(x, config._GRAPH_MAX_ENTRIES)
    monkeypatch.setattr(config, "_GRAPH_MAX_ACTIVATION", 10)
    assert not graphs._graph_eligible(x, 0)
    monkeypatch.setattr(config, "CUDA_GRAPH", "always")
    assert graphs._graph_eligible(x, 0)


def test_refused_capture_is_logged_and_not_retried(monkeypatch):
    m = _model(B=2)
    attempts = []

    def refuse(model, x, mask, use_mask, packing=None, log=None):
        attempts.append(tuple(x.shape))
        log["outcome"] = "declined: replay not faster than eager"
        return None

    monkeypatch.setattr(omodel, "_graph_eligible", lambda x, n: True)
    monkeypatch.setattr(omodel, "_capture_graph", refuse)
    monkeypatch.setattr(config, "MICROBATCH_FALLBACK", False)
    m._forward_eager = lambda x, mask, use_mask, packing=None: x + 1
    x = torch.zeros(2, 4, 16)
    for _ in range(3):
        assert torch.equal(m(x), x + 1)
    assert attempts == [(2, 4, 16)]
    (entry,) = m._graph_log.values()
    assert entry["outcome"].startswith("declined")
    assert not m._graphs


def test_ineligible_calls_are_not_logged(monkeypatch):
    m = _model(B=2)
    monkeypatch.setattr(config, "MICROBATCH_FALLBACK", False)
    m._forward_eager = lambda x, mask, use_mask, packing=None: x
    m(torch.zeros(2, 4, 16))
    assert m._graph_log == {}       # a later CUDA_GRAPH change is still honoured


def test_capture_without_the_library_declines(monkeypatch):
    monkeypatch.setattr(graphs, "_custom_kernels", lambda: None)
    log = {}
    assert graphs._capture_graph(_model(), torch.zeros(2, 4, 16), None, False, log=log) is None
    assert log["outcome"] == "extension not loaded"


def test_failed_capture_on_a_healthy_device_is_noted(monkeypatch):
    monkeypatch.setattr(graphs, "_device_still_runs", lambda dev: True)
    monkeypatch.setattr(graphs.torch.cuda, "empty_cache", lambda: None)
    log = {}
    graphs._abandon_capture(RuntimeError("operation not permitted when stream is capturing"),
                            torch.device("cpu"), log)
    assert log["outcome"].startswith("capture failed: RuntimeError")


def test_failed_capture_on_a_broken_device_raises(monkeypatch):
    monkeypatch.setattr(graphs, "_device_still_runs", lambda dev: False)
    with pytest.raises(RuntimeError, match="no longer runs work"):
        graphs._abandon_capture(RuntimeError("boom"), torch.device("cpu"), {})


def test_graph_io_binding_marks_only_the_forward_input():
    slot = torch.zeros(2, dtype=torch.int64)
    x = torch.zeros(2, 4, 16)
    io = graphs._GraphIO(slot, x)
    okernels._graph_io = io
    try:
        assert okernels._input_io(torch.zeros(2, 4, 16)) is None   # another tensor
        assert not io.in_bound
        assert okernels._input_io(x) == (slot, 1) and io.in_bound
        assert okernels._output_io() == (slot, 2)
        y = torch.zeros(3)
        assert okernels._note_output(y, (slot, 2)) is y and io.out_ptr == y.data_ptr()
    finally:
        okernels._graph_io = None
    assert okernels._output_io() is None and okernels._input_io(x) is None
