"""hipGraph capture and replay of the forward pass (reference optimized/graphs.py).

torch.cuda.CUDAGraph is hipGraph on ROCm, and every kernel in this build
launches on torch's current stream read at call time, so the whole forward
(our kernels plus the few torch elementwise ops of the padded path) records
into one graph. A graph is installed only after a replay is shown to equal
the eager forward bit for bit; on any doubt capture declines and the caller
stays eager.
"""

from __future__ import annotations

import atexit
import weakref
from typing import Optional, Tuple

import torch

from . import config
from .kernels import _custom_kernels

_graph_warned = False
_graph_noted = False
_graph_declined_noted = False


class _GraphRunner:
    """One captured graph plus every buffer whose address it baked in."""

    __slots__ = ("graph", "stream", "static_x", "static_mask", "static_out", "needs_mask",
                 "static_packing", "loaded_packing", "replays", "pinned", "__weakref__")

    def __init__(self, graph, stream, static_x, static_mask, static_out, needs_mask, pinned,
                 static_packing=None, loaded_packing=None):
        self.graph = graph
        self.stream = stream
        self.static_x = static_x
        self.static_mask = static_mask
        self.static_out = static_out
        self.needs_mask = needs_mask
        self.pinned = pinned
        # Packed-row graphs read the row maps instead of the mask; the maps
        # are reloaded only when the model hands in a different packing
        # (a new mask object), not on every replay.
        self.static_packing = static_packing
        self.loaded_packing = loaded_packing
        self.replays = 0

    def replay(self, x: torch.Tensor, mask: Optional[torch.Tensor],
               packing=None) -> torch.Tensor:
        """Copy the inputs in, replay, return a clone of the output."""
        self.static_x.copy_(x)
        if self.needs_mask:
            self.static_mask.copy_(mask)
        if self.static_packing is not None and packing is not self.loaded_packing:
            self.static_packing.copy_(packing)
            self.loaded_packing = packing
        self.graph.replay()
        self.replays += 1
        return self.static_out.clone()

    def release(self) -> None:
        """Give the private pool back: reset, drop every pool tensor, empty the cache."""
        try:
            self.graph.reset()
        except Exception:  # noqa: BLE001 - reset on a half-captured graph may throw
            pass
        self.graph = None
        self.stream = None
        self.static_x = None
        self.static_mask = None
        self.static_out = None
        self.static_packing = None
        self.loaded_packing = None
        self.pinned = None
        torch.cuda.empty_cache()


def _graph_key(x: torch.Tensor, use_mask: bool, packing=None) -> Tuple:
    """Everything a capture freezes: shape/dtype/device, mask mode (and the
    packed row count, which sizes the packed path's GEMMs) and the knobs."""
    return (tuple(x.shape), x.dtype, x.device.index, use_mask,
            None if packing is None else packing.key(), config.ROW_PACKING, config.RESIDUAL_EPILOGUE,
            config.ATTENTION_IMPL, config.LINEAR_GELU, config.LINEAR_BIAS, config.LAYERNORM,
            config.QKV_FP16, config.NORMED_FP16, config.CP_ASYNC, config.ATTENTION_PRECISION,
            config.QKV_PRECISION, config.GELU_FP16)


def _graph_pool_cap_bytes(device: torch.device) -> int:
    total = torch.cuda.get_device_properties(device).total_memory
    return int(total * config._GRAPH_POOL_SAFETY_FRACTION)


def _graph_eligible(x: torch.Tensor, entries: int) -> bool:
    """Cheap per-call gate: pure Python comparisons, no GPU calls."""
    if config.CUDA_GRAPH == "off":
        return False
    if x.device.type != "cuda" or x.dim() != 3:
        return False
    if torch.compiler.is_compiling():
        return False
    if torch.cuda.is_current_stream_capturing():
        return False
    if entries >= config._GRAPH_MAX_ENTRIES:
        return False
    if config.CUDA_GRAPH == "always":
        return True
    return x.shape[0] * x.shape[1] * x.shape[2] <= config._GRAPH_MAX_ACTIVATION


def _graph_note_decline(x: torch.Tensor) -> None:
    """Say once why "auto" is not capturing."""
    global _graph_declined_noted
    if _graph_declined_noted or config.CUDA_GRAPH == "off":
        return
    if x.device.type != "cuda" or torch.compiler.is_compiling():
        return
    _graph_declined_noted = True
    activation = x.shape[0] * x.shape[1] * x.shape[2]
    if activation > config._GRAPH_MAX_ACTIVATION:
        print(f"[info] graph capture declined for shape {tuple(x.shape)}: batch*seq*d_model "
              f"is {activation}, over the {config._GRAPH_MAX_ACTIVATION} above which the GPU "
              f"hides launch cost. Running eagerly; results are unaffected. "
              f"(--cuda-graph always captures anyway.)")
    else:
        print(f"[info] graph capture declined for shape {tuple(x.shape)}, running eagerly "
              f"(results are unaffected).")


def _graph_cache_ptrs(model) -> Tuple:
    """Addresses of the lazily built caches a graph bakes in."""
    out = []
    for layer in model.layers:
        attn = layer.attention
        for t in (attn._qkv_weight, attn._qkv_bias):
            out.append(None if t is None else t.data_ptr())
    kernels = _custom_kernels()
    if kernels is not None and hasattr(kernels, "weight_cache_tensors"):
        out.extend(sorted(t.data_ptr() for t in kernels.weight_cache_tensors()))
    return tuple(out)


def _graph_pinned_refs(model) -> Tuple:
    """Strong references keeping those caches alive as long as the graph."""
    out = []
    for layer in model.layers:
        attn = layer.attention
        out.extend((attn._qkv_weight, attn._qkv_bias))
    kernels = _custom_kernels()
    if kernels is not None and hasattr(kernels, "weight_cache_tensors"):
        out.extend(kernels.weight_cache_tensors())
    return tuple(out)


def _graph_release(g) -> None:
    if g is not None:
        try:
            g.reset()
        except Exception:  # noqa: BLE001
            pass


def _capture_graph(model, x: torch.Tensor, mask: Optional[torch.Tensor],
                   use_mask: bool, packing=None) -> Optional[_GraphRunner]:
    """Capture model._forward_eager, or return None and leave the run eager.

    With `packing` the graph runs the packed-row path on static copies of the
    row maps (loaded from `packing`) and never reads the mask.
    """
    global _graph_noted, _graph_warned
    dev = x.device
    g = None
    static_x = static_mask = static_out = ref = static_packing = None
    needs_mask = use_mask and packing is None
    try:
        if _custom_kernels() is None:
            return None
        torch.cuda.get_device_properties(dev)
        free_bytes, _ = torch.cuda.mem_get_info(dev)
        if free_bytes < config._GRAPH_MIN_FREE_BYTES:
            return None
        torch.cuda.empty_cache()
        reserved_before = torch.cuda.memory_reserved(dev)

        with torch.inference_mode(False):
            static_x = torch.empty(x.shape, dtype=x.dtype, device=dev)
            static_mask = (torch.empty(mask.shape, dtype=torch.bool, device=dev)
                           if needs_mask else None)
            gen = torch.Generator(device=dev)
            gen.manual_seed(config._GRAPH_SEED)
            static_x.normal_(generator=gen)
            if needs_mask:
                static_mask.fill_(True)
                static_mask[:, static_mask.shape[1] // 2:] = False
            if packing is not None:
                static_packing = packing.empty_like()
                static_packing.copy_(packing)

            with torch.no_grad():
                # Warmup on the capture stream: builds the fused QKV weight and
                # the fp16 weight copies in the general pool, not the graph's.
                side = torch.cuda.Stream(device=dev)
                side.wait_stream(torch.cuda.current_stream(dev))
                with torch.cuda.stream(side):
                    for _ in range(config._GRAPH_WARMUP_ITERS):
                        model._forward_eager(static_x, static_mask, use_mask, static_packing)
                torch.cuda.current_stream(dev).wait_stream(side)
                torch.cuda.synchronize(dev)
                ptrs_before = _graph_cache_ptrs(model)

                ref = model._forward_eager(static_x, static_mask, use_mask,
                                           static_packing).clone()

                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=side):
                    static_out = model._forward_eager(static_x, static_mask, use_mask,
                                                      static_packing)

                # Prove the graph computes what eager computes, on more than one
                # replay (a replay-dependent node would show on the second).
                delta = 0.0
                for _ in range(2):
                    g.replay()
                    torch.cuda.synchronize(dev)
                    delta = max(delta, (static_out.float() - ref.float()).abs().max().item())
                ptrs_after = _graph_cache_ptrs(model)

        if ptrs_after != ptrs_before:
            _graph_release(g)
            if not _graph_warned:
                _graph_warned = True
                print("[info] graph capture rebuilt a weight cache inside the capture region, "
                      "so it was discarded and this run stays eager (results are correct).")
            return None
        if delta != 0.0:
            _graph_release(g)
            if not _graph_warned:
                _graph_warned = True
                print(f"[info] graph replay differs from eager by {delta:.3e}, so the graph was "
                      f"discarded and this run stays eager (results are correct).")
            return None
        pool_bytes = torch.cuda.memory_reserved(dev) - reserved_before
        budget = _graph_pool_cap_bytes(dev)
        if config.CUDA_GRAPH != "always" and pool_bytes > budget:
            _graph_release(g)
            if not _graph_warned:
                _graph_warned = True
                print(f"[info] graph for shape {tuple(x.shape)} reserved "
                      f"{pool_bytes / (1 << 20):.0f} MiB, over the {budget / (1 << 20):.0f} MiB "
                      f"cap; released, this shape runs eagerly.")
            return None

        runner = _GraphRunner(graph=g, stream=side, static_x=static_x, static_mask=static_mask,
                              static_out=static_out, needs_mask=needs_mask,
                              pinned=_graph_pinned_refs(model), static_packing=static_packing,
                              loaded_packing=packing)
        _graph_register(runner)
        if not _graph_noted:
            _graph_noted = True
            pool_mib = (torch.cuda.memory_reserved(dev) - reserved_before) / (1 << 20)
            print(f"[info] graph captured: shape={tuple(x.shape)} "
                  f"{str(x.dtype).replace('torch.', '')} mask={'on' if use_mask else 'off'}"
                  f"{' (packed rows)' if packing is not None else ''}, "
                  f"pool +{pool_mib:.1f} MiB, replay matches eager exactly")
        return runner

    except Exception as exc:  # noqa: BLE001
        _graph_release(g)
        del static_x, static_mask, static_out, ref, static_packing
        try:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("stream is still capturing")
            torch.cuda.synchronize(dev)
            torch.empty(1, device=dev).fill_(1.0)
            torch.cuda.synchronize(dev)
        except Exception as fatal:  # noqa: BLE001
            raise RuntimeError(
                "graph capture failed and left the device context unusable; re-run with "
                f"--cuda-graph off. Original failure: {exc}") from fatal
        torch.cuda.empty_cache()
        if not _graph_warned:
            _graph_warned = True
            print(f"[info] graph capture failed for shape {tuple(x.shape)}, running eagerly "
                  f"(results are correct). Reason: {type(exc).__name__}: {exc}")
        return None


# Every live graph, weakly held, torn down at exit while the runtime is still up.
_graph_live: "weakref.WeakSet" = weakref.WeakSet()
_graph_atexit_registered = False


def _graph_register(runner: _GraphRunner) -> None:
    global _graph_atexit_registered
    _graph_live.add(runner)
    if not _graph_atexit_registered:
        _graph_atexit_registered = True
        atexit.register(_graph_release_all)


def _graph_release_all() -> None:
    for runner in list(_graph_live):
        try:
            runner.release()
        except Exception:  # noqa: BLE001
            pass
    _graph_live.clear()
