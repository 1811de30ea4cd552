"""hipGraph capture and replay of the forward pass.

The names the rest of the package (and the reference's scripts) use are kept
from the reference's module (optimized/graphs.py:27-460): `_GraphRunner`
with `replay()` / `release()`, `_graph_key`, `_graph_eligible`,
`_graph_note_decline`, `_capture_graph`, `_graph_release_all`. The design
behind them is this build's:

* Bound I/O. A captured forward does not own its input and output buffers.
  Its entry LayerNorm reads x, and its output LayerNorm writes y, through a
  device-resident slot (int64 [2]) that those two kernels dereference at run
  time; one tiny kernel (`Kernels.bind_io`) writes the caller's addresses into
  the slot, in stream order, before each replay. A replay is then two
  launches and moves no activation bytes beyond the forward's own: nothing is
  copied into a static input and no static output is cloned (at the padded
  mass-batch shape those two copies were ~0.5 GB of traffic per call). A
  forward whose last op is not such a LayerNorm (the masked path with row
  packing off ends in masked_fill) binds only what it can and copies the
  rest.
* Proof before use. A graph is installed only if (1) a replay on the input
  the forward was captured with reproduces the eager output bit for bit,
  (2) a replay on a second input, the first one negated (padded rows stay
  zero, so the mask stays valid), reproduces eager on that input bit for
  bit -- which shows that the graph reads the bound input, not a stale copy,
  and writes the bound output -- and (3) no weight cache was rebuilt inside
  the capture (a cache built there would live in the graph's private pool).
* Measured keep/decline. In "auto" a proven graph is then timed against the
  eager forward on the same input (HIP events, alternating samples, median
  of five); it is kept only if it is at least config._GRAPH_MIN_GAIN faster. "always" keeps every proven graph. Each
  outcome and its timings go to `model._graph_log[key]`.
* Failure isolation. An exception while capturing ends the capture (torch's
  context manager), then a one-element kernel checks the device still runs
  work: if it does not, the error is raised, since nothing else will work
  either; otherwise the key is denied and the call runs eagerly.

torch.cuda.CUDAGraph is hipGraph on ROCm; every kernel of this build
launches on torch's current stream read at call time, so the forward records
into one graph, with the intermediates in the graph's private memory pool.
"""

from __future__ import annotations

import atexit
import statistics
import weakref
from typing import Dict, Optional, Tuple

import torch

from . import config
from . import kernels as _kernels_mod
from .kernels import _custom_kernels

# One [info] line per process for each kind of event, not one per shape.
_said: set = set()


def _say_once(kind: str, msg: str) -> None:
    if kind not in _said:
        _said.add(kind)
        print(f"[info] {msg}")


class _GraphIO:
    """The capture-time record of which kernels were bound to the I/O slot.

    Set as `kernels._graph_io` while a forward is being captured: the entry
    LayerNorm that receives `x_stand_in` reads through `slot[0]` and sets
    `in_bound`; the output LayerNorm writes through `slot[1]` and records
    the address of the tensor that stands for its output in `out_ptr`.
    """

    __slots__ = ("slot", "x_stand_in", "in_bound", "out_ptr")

    def __init__(self, slot: torch.Tensor, x_stand_in: torch.Tensor) -> None:
        self.slot = slot
        self.x_stand_in = x_stand_in
        self.in_bound = False
        self.out_ptr: Optional[int] = None


class _GraphRunner:
    """A proven graph and what its replays need.

    Holds the graph (its executable and private pool), the I/O slot, the
    stand-in tensors whose addresses the graph baked in for anything not
    bound (the input copy target, the output, a mask, the row maps), and
    `keepalive`, the cached weight copies the graph reads.
    """

    __slots__ = ("graph", "slot", "x_buf", "out_buf", "mask_buf", "maps_buf", "maps_src",
                 "in_bound", "out_bound", "out_shape", "out_dtype", "keepalive", "replays",
                 "timing", "bound_to", "__weakref__")

    def __init__(self) -> None:
        self.graph = None
        self.slot = None
        self.x_buf = None
        self.out_buf = None
        self.mask_buf = None
        self.maps_buf = None
        self.maps_src = None
        self.in_bound = False
        self.out_bound = False
        self.out_shape = None
        self.out_dtype = None
        self.keepalive: Tuple = ()
        self.replays = 0
        self.timing: Dict[str, float] = {}
        # (input address, output address, stream) the slot holds: a replay
        # with the same three needs no bind (the caching allocator usually
        # hands the output the block the previous one released)
        self.bound_to: Optional[Tuple] = None

    def replay(self, x: torch.Tensor, mask: Optional[torch.Tensor],
               packing=None) -> torch.Tensor:
        """Run the graph on `x` (and `mask` / `packing`); returns a new tensor."""
        kx = _custom_kernels()
        if self.in_bound:
            src = x if x.is_contiguous() else x.contiguous()
        else:
            self.x_buf.copy_(x)
            src = None
        out = (torch.empty(self.out_shape, dtype=self.out_dtype, device=x.device)
               if self.out_bound else None)
        if src is not None or out is not None:
            stream = torch.cuda.current_stream(x.device)
            want = (src.data_ptr() if src is not None else 0,
                    out.data_ptr() if out is not None else 0, stream.cuda_stream)
            if want != self.bound_to:
                kx.bind_io(self.slot, src, out)
                self.bound_to = want
        if self.mask_buf is not None:
            self.mask_buf.copy_(mask)
        if self.maps_buf is not None and packing is not self.maps_src:
            self.maps_buf.copy_(packing)
            self.maps_src = packing
        self.graph.replay()
        self.replays += 1
        return out if out is not None else self.out_buf.clone()

    def release(self) -> None:
        """Drop the graph and every tensor of its pool, then return the pool's
        memory to the device (a pool is freed only when the graph is reset
        and none of its tensors is referenced any more)."""
        graph, self.graph = self.graph, None
        if graph is not None:
            try:
                graph.reset()
            except RuntimeError:
                pass
        for name in ("slot", "x_buf", "out_buf", "mask_buf", "maps_buf", "maps_src"):
            setattr(self, name, None)
        self.keepalive = ()
        torch.cuda.empty_cache()


def _graph_key(x: torch.Tensor, use_mask: bool, packing=None) -> Tuple:
    """What a capture freezes: the input's shape, dtype and device; the mask
    mode (and the packed row count, which sizes the packed path's GEMMs);
    and every knob that selects a kernel or an arithmetic."""
    return (tuple(x.shape), x.dtype, x.device.index, use_mask,
            None if packing is None else packing.key(), config.ROW_PACKING,
            config.RESIDUAL_EPILOGUE, config.LN_EPILOGUE, config.FFN_LN, config.ATTENTION_IMPL, config.LINEAR_GELU,
            config.LINEAR_BIAS, config.LAYERNORM, config.QKV_FP16, config.NORMED_FP16,
            config.CP_ASYNC, config.ATTENTION_PRECISION, config.QKV_PRECISION, config.GELU_FP16,
            _kernels_mod._stack_precision, _kernels_mod._qkv_few_keys,
            _kernels_mod._qkv_split_prefix)


def _graph_eligible(x: torch.Tensor, entries: int) -> bool:
    """Whether to try a capture for this call: host-side checks only."""
    mode = config.CUDA_GRAPH
    if mode == "off" or x.device.type != "cuda" or x.dim() != 3:
        return False
    if torch.compiler.is_compiling() or torch.cuda.is_current_stream_capturing():
        return False
    if entries >= config._GRAPH_MAX_ENTRIES:
        return False
    return mode == "always" or x.numel() <= config._GRAPH_MAX_ACTIVATION


def _graph_note_decline(x: torch.Tensor) -> None:
    """Say (once) why a capture is not tried."""
    if config.CUDA_GRAPH == "off" or x.device.type != "cuda":
        return
    if x.numel() > config._GRAPH_MAX_ACTIVATION and config.CUDA_GRAPH == "auto":
        _say_once("too-big", f"no graph for shape {tuple(x.shape)}: {x.numel()} activation "
                             f"elements exceed the {config._GRAPH_MAX_ACTIVATION} up to which "
                             f"'auto' captures; running eagerly (same results)")
    else:
        _say_once("not-eligible", f"no graph for shape {tuple(x.shape)}; running eagerly "
                                  f"(same results)")


def _weight_generation(model) -> Tuple:
    """Counts of weight-cache (re)builds: changes iff a cache was rebuilt."""
    kx = _custom_kernels()
    kgen = kx.cache_generation() if kx is not None and hasattr(kx, "cache_generation") else 0
    return (kgen,) + tuple(layer.attention._qkv_generation for layer in model.layers)


def _weight_keepalive(model) -> Tuple:
    """The cached weight tensors a captured graph reads by address."""
    held = []
    for layer in model.layers:
        held.extend(t for t in (layer.attention._qkv_weight, layer.attention._qkv_bias)
                    if t is not None)
    kx = _custom_kernels()
    if kx is not None and hasattr(kx, "weight_cache_tensors"):
        held.extend(kx.weight_cache_tensors())
    return tuple(held)


def _time_calls(fn, n: int) -> float:
    """Device time (ms) per call of `n` back-to-back calls of `fn`."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(n):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / n


def _compare_timing(eager_call, replay_call, samples: int = 5) -> Tuple[float, float]:
    """Median per-call device time (ms) of eager and replay, measured in
    alternating samples of enough calls for ~10 ms each, so clock and
    thermal drift hit both alike."""
    single = max(_time_calls(eager_call, 1), 1e-3)
    n = max(3, min(200, int(10.0 / single)))
    eager, replay = [], []
    for _ in range(samples):
        eager.append(_time_calls(eager_call, n))
        replay.append(_time_calls(replay_call, n))
    return statistics.median(eager), statistics.median(replay)


def _device_still_runs(device: torch.device) -> bool:
    """One tiny kernel and a synchronize: False if the context is broken."""
    try:
        if torch.cuda.is_current_stream_capturing():
            return False
        probe = torch.zeros(1, device=device)
        probe.add_(1.0)
        torch.cuda.synchronize(device)
        return bool(probe.item() == 1.0)
    except RuntimeError:
        return False


def _abandon_capture(exc: BaseException, device: torch.device, log: Dict) -> None:
    """After a failed capture: raise if the device is unusable, else note why."""
    if not _device_still_runs(device):
        raise RuntimeError("hipGraph capture failed and the device no longer runs work; "
                           "rerun with CUDA_GRAPH='off' (--cuda-graph off). Capture error: "
                           f"{type(exc).__name__}: {exc}") from exc
    torch.cuda.empty_cache()
    log["outcome"] = f"capture failed: {type(exc).__name__}: {exc}"
    _say_once("failed", f"graph capture failed ({type(exc).__name__}: {exc}); running eagerly "
                        f"(same results)")


def _capture_graph(model, x: torch.Tensor, mask: Optional[torch.Tensor], use_mask: bool,
                   packing=None, log: Optional[Dict] = None) -> Optional[_GraphRunner]:
    """Capture, prove and (in "auto") time a graph of model._forward_eager.

    Returns an installed-ready runner, or None (with the reason in `log`)
    when the call should stay eager.
    """
    log = {} if log is None else log
    device = x.device
    kx = _custom_kernels()
    if kx is None or not hasattr(kx, "bind_io"):
        log["outcome"] = "extension not loaded"
        return None
    free, total = torch.cuda.mem_get_info(device)
    if free < config._GRAPH_MIN_FREE_BYTES:
        log["outcome"] = f"only {free >> 20} MiB free"
        return None

    runner = _GraphRunner()
    graph = None
    try:
        with torch.inference_mode(False), torch.no_grad():
            x_in = x.contiguous().clone()
            mask_in = mask.clone() if (use_mask and packing is None) else None
            maps_in = None
            if packing is not None:
                maps_in = packing.empty_like()
                maps_in.copy_(packing)
            slot = torch.zeros(2, dtype=torch.int64, device=device)

            # Eager reference on the real input, run on the capture stream
            # first so every lazily built cache exists before capture.
            side = torch.cuda.Stream(device=device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                for _ in range(config._GRAPH_WARMUP_ITERS):
                    ref = model._forward_eager(x_in, mask_in, use_mask, maps_in)
            torch.cuda.current_stream(device).wait_stream(side)
            torch.cuda.synchronize(device)
            gen_before = _weight_generation(model)
            reserved_before = torch.cuda.memory_reserved(device)

            io = _GraphIO(slot, x_in)
            graph = torch.cuda.CUDAGraph()
            _kernels_mod._graph_io = io
            try:
                with torch.cuda.graph(graph, stream=side):
                    out_stand_in = model._forward_eager(x_in, mask_in, use_mask, maps_in)
            finally:
                _kernels_mod._graph_io = None
            if _weight_generation(model) != gen_before:
                log["outcome"] = "a weight cache was rebuilt during capture"
                return None

            runner.graph = graph
            runner.slot = slot
            runner.in_bound = io.in_bound
            runner.out_bound = (io.out_ptr is not None
                                and out_stand_in.data_ptr() == io.out_ptr)
            runner.out_shape = tuple(out_stand_in.shape)
            runner.out_dtype = out_stand_in.dtype
            runner.x_buf = None if runner.in_bound else x_in
            runner.out_buf = None if runner.out_bound else out_stand_in
            runner.mask_buf = mask_in
            runner.maps_buf = maps_in
            runner.maps_src = packing
            runner.keepalive = _weight_keepalive(model)

            # Proof: the captured input, then a different one, each against eager.
            x_alt = torch.neg(x_in)
            for probe in (x, x_alt):
                want = model._forward_eager(probe.contiguous(), mask_in, use_mask, maps_in)
                got = runner.replay(probe, mask_in if mask_in is not None else mask, packing)
                torch.cuda.synchronize(device)
                if not torch.equal(got, want):
                    diff = (got.float() - want.float()).abs().max().item()
                    log["outcome"] = f"replay differs from eager by {diff:.3e}"
                    _say_once("mismatch", f"graph replay differed from eager ({diff:.3e}); "
                                          f"discarded, running eagerly (same results)")
                    runner.release()
                    return None
            runner.replays = 0
            pool = max(0, torch.cuda.memory_reserved(device) - reserved_before)
            log["pool_mib"] = round(pool / (1 << 20), 1)
            log["io"] = ("bound" if runner.in_bound else "copied") + " in, " + \
                        ("bound" if runner.out_bound else "cloned") + " out"
            if config.CUDA_GRAPH != "always" and pool > total * config._GRAPH_POOL_SAFETY_FRACTION:
                log["outcome"] = f"pool of {pool >> 20} MiB over the cap"
                runner.release()
                return None

            if config.CUDA_GRAPH == "auto":
                eager_call = lambda: model._forward_eager(x, mask, use_mask, packing)  # noqa: E731
                replay_call = lambda: runner.replay(x, mask, packing)  # noqa: E731
                eager_ms, replay_ms = _compare_timing(eager_call, replay_call)
                runner.replays = 0
                runner.timing = {"eager_us": eager_ms * 1e3, "replay_us": replay_ms * 1e3}
                log.update(runner.timing)
                if replay_ms > eager_ms * (1.0 - config._GRAPH_MIN_GAIN):
                    log["outcome"] = "declined: replay not faster than eager"
                    runner.release()
                    return None
            log["outcome"] = "captured"
            _say_once("captured", f"graph captured for shape {tuple(x.shape)} "
                                  f"({log['io']}; replay equals eager on two inputs)")
            _live.add(runner)
            _register_atexit()
            return runner
    except (RuntimeError, torch.OutOfMemoryError) as exc:
        runner.release()
        _abandon_capture(exc, device, log)
        return None


# Live runners, weakly held, released at exit while the HIP runtime is up.
_live: "weakref.WeakSet[_GraphRunner]" = weakref.WeakSet()
_atexit_done = False


def _register_atexit() -> None:
    global _atexit_done
    if not _atexit_done:
        _atexit_done = True
        atexit.register(_graph_release_all)


def _graph_release_all() -> None:
    """Release every live graph (registered with atexit on first capture)."""
    for runner in list(_live):
        try:
            runner.release()
        except RuntimeError:
            pass
    _live.clear()
