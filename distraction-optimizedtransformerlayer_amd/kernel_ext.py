"""Loader for the gfx950 kernels: the reference's extension surface over a C ABI.

The reference's `kernel_ext.get_kernels()` JIT-builds a pybind CUDA module and
returns it, or None when it cannot (reference kernel_ext.py:363-491). This
module keeps that contract -- `get_kernels()` returns an object whose methods
have the pybind module's names, arguments and return conventions
(reference csrc/fused_attention.cu:118-376), `load_error()` says why it is
None -- but the object is a thin ctypes layer over `libdotl_hip.so`, the
C-ABI library declared in include/dotl.h:

  * device memory and streams are torch's: outputs are allocated with
    torch.empty on the input's device, and every launch goes to
    torch.cuda.current_stream() read at call time, so a call made under
    torch.cuda.graph() capture is recorded into the graph;
  * the C entry points return 0 (launched), 1 (declined: the reference's
    undefined tensor / empty list, i.e. None / [] here) or a negative error
    (the reference's TORCH_CHECK raise, i.e. RuntimeError here);
  * W is narrowed to fp16 once per weight version and cached here (the
    reference narrows it inside every GEMM launch); `weight_cache_tensors()`
    lists the cached buffers so graph capture can pin them.

There is no CPU fallback anywhere in this module: a missing library makes
get_kernels() return None, and the callers that cannot decline (attention)
raise, exactly as the reference does.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading
import weakref
from typing import Dict, List, Optional, Tuple

_THIS_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_THIS_DIR, "libdotl_hip.so")
_CSRC = os.path.join(_THIS_DIR, "csrc")

ABI_VERSION = 3

DOTL_OK = 0
DOTL_DECLINED = 1
DOTL_F32 = 0
DOTL_F16 = 1
DOTL_F16X2 = 2
DOTL_BF16 = 3
DOTL_ACT_NONE = 0
DOTL_ACT_GELU = 1
DOTL_MATH_FP16 = 0
DOTL_MATH_FP16X3 = 1
DOTL_MATH_FP16X2 = 2

# Every symbol include/dotl.h declares.
EXPORTED_SYMBOLS = (
    "dotl_last_error", "dotl_abi_version", "dotl_target", "dotl_smoke_test_identity",
    "dotl_mfma_layout_probe", "dotl_mfma_ceiling_probe", "dotl_layernorm", "dotl_weight_split", "dotl_linear",
    "dotl_attention_forward", "dotl_ffn_block", "dotl_wmma_set_fp16", "dotl_wmma_fp16",
    "dotl_wmma_set_cp_async", "dotl_wmma_cp_async_mode", "dotl_lds_dma_probe",
    "dotl_attention_set_pipeline", "dotl_linear_residual", "dotl_bind_io",
    "dotl_attention_split_plan", "dotl_wmma_set_split_kv", "dotl_wmma_split_kv_enabled",
    "dotl_wmma_set_split_count", "dotl_attention_forward_noalloc",
    "dotl_attention_noalloc_scratch_bytes", "dotl_linear_layernorm", "dotl_zero_rows",
    "dotl_linear_planes", "dotl_ffn_layernorm",
)

_kernels = None
_load_attempted = False
_load_error: Optional[BaseException] = None
_lock = threading.Lock()


def library_path() -> str:
    return _LIB_PATH


def build(verbose: bool = False, jobs: int = 8, force: bool = True) -> str:
    """Compile libdotl_hip.so for gfx950 with the Makefile in csrc/ (hipcc).

    Needs no GPU: hipcc cross-compiles. `force` (the default) recompiles every
    source (make -B, ~4 minutes on 8 cores), so a build check never passes on
    objects left from an earlier build. Returns the library path.
    """
    cmd = ["make", "-C", _CSRC, f"-j{jobs}"] + (["-B"] if force else [])
    res = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or res.returncode != 0:
        print(res.stdout)
        print(res.stderr)
    if res.returncode != 0:
        raise RuntimeError(f"building libdotl_hip.so failed (exit {res.returncode}):\n"
                           f"{res.stderr[-4000:]}")
    return _LIB_PATH


def _declare(lib) -> None:
    c = ctypes
    i64, vp, i32 = c.c_int64, c.c_void_p, c.c_int
    lib.dotl_last_error.restype = c.c_char_p
    lib.dotl_last_error.argtypes = []
    lib.dotl_abi_version.restype = i32
    lib.dotl_target.restype = c.c_char_p
    lib.dotl_smoke_test_identity.restype = i32
    lib.dotl_smoke_test_identity.argtypes = [vp, vp, i64, vp]
    lib.dotl_mfma_layout_probe.restype = i32
    lib.dotl_mfma_layout_probe.argtypes = [vp, vp]
    lib.dotl_mfma_ceiling_probe.restype = i32
    lib.dotl_mfma_ceiling_probe.argtypes = [i64, i32, i32, vp, vp]
    lib.dotl_lds_dma_probe.restype = i32
    lib.dotl_lds_dma_probe.argtypes = [vp, vp, vp]
    lib.dotl_layernorm.restype = i32
    lib.dotl_layernorm.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, c.c_double, i32,
                                   i32, vp, i32, vp]
    lib.dotl_bind_io.restype = i32
    lib.dotl_bind_io.argtypes = [vp, vp, vp, vp]
    lib.dotl_weight_split.restype = i32
    lib.dotl_weight_split.argtypes = [vp, vp, vp, i64, vp]
    lib.dotl_linear.restype = i32
    lib.dotl_linear.argtypes = [vp, i32, vp, vp, vp, vp, i32, i64, i64, i64, i32, i32, i32, vp]
    lib.dotl_linear_residual.restype = i32
    lib.dotl_linear_residual.argtypes = [vp, i32, vp, vp, vp, vp, vp, i64, i64, i64, i32, i32,
                                         i32, vp]
    lib.dotl_linear_planes.restype = i32
    lib.dotl_linear_planes.argtypes = [vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i32, i32, vp]
    lib.dotl_linear_layernorm.restype = i32
    lib.dotl_linear_layernorm.argtypes = [vp, i32, vp, vp, vp, vp, vp, vp, c.c_double, vp, i32,
                                          vp, i64, vp, i64, i64, i64, i32, vp]
    lib.dotl_ffn_layernorm.restype = i32
    lib.dotl_ffn_layernorm.argtypes = [vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, c.c_double, vp,
                                       i32, vp, i64, i32, vp, i64, i64, i64, vp]
    lib.dotl_zero_rows.restype = i32
    lib.dotl_zero_rows.argtypes = [vp, vp, i64, i64, vp, vp]
    lib.dotl_attention_forward.restype = i32
    lib.dotl_attention_forward.argtypes = [vp, vp, vp, i32, c.POINTER(i64), vp, c.POINTER(i64),
                                           vp, i32, i32, i32, i32, i32, i32, i32, c.c_double,
                                           i32, i32, vp, i64, i32, vp, i64, vp]
    lib.dotl_attention_forward_noalloc.restype = i32
    lib.dotl_attention_forward_noalloc.argtypes = [vp, vp, vp, i32, c.POINTER(i64), vp,
                                                   c.POINTER(i64), vp, i32, i32, i32, i32, i32,
                                                   i32, i32, c.c_double, i32, i32, vp, i64, i32,
                                                   vp]
    lib.dotl_attention_noalloc_scratch_bytes.restype = i64
    lib.dotl_attention_noalloc_scratch_bytes.argtypes = []
    lib.dotl_attention_split_plan.restype = i32
    lib.dotl_attention_split_plan.argtypes = [i32, i32, i32, i32, i32, i32, i32, i64, i32, i32,
                                              i32, c.POINTER(i32), c.POINTER(i64)]
    lib.dotl_wmma_set_split_kv.restype = None
    lib.dotl_wmma_set_split_kv.argtypes = [i32]
    lib.dotl_wmma_split_kv_enabled.restype = i32
    lib.dotl_wmma_set_split_count.restype = None
    lib.dotl_wmma_set_split_count.argtypes = [i32]
    lib.dotl_ffn_block.restype = i32
    lib.dotl_ffn_block.argtypes = [vp] * 12 + [i64, i64, i64, c.c_double, vp]
    lib.dotl_wmma_set_fp16.restype = None
    lib.dotl_wmma_set_fp16.argtypes = [i32]
    lib.dotl_wmma_fp16.restype = i32
    lib.dotl_wmma_set_cp_async.restype = None
    lib.dotl_wmma_set_cp_async.argtypes = [i32]
    lib.dotl_wmma_cp_async_mode.restype = i32
    lib.dotl_attention_set_pipeline.restype = None
    lib.dotl_attention_set_pipeline.argtypes = [i32, i32]


def load_library(path: Optional[str] = None):
    """dlopen the C-ABI library (after torch, so it binds torch's HIP runtime)."""
    import torch  # noqa: F401  -- the HIP runtime must be loaded first

    lib = ctypes.CDLL(path or _LIB_PATH)
    _declare(lib)
    got = lib.dotl_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"libdotl_hip.so ABI {got}, this loader speaks {ABI_VERSION}; rebuild")
    return lib


def _version_or_none(t) -> Optional[int]:
    try:
        return t._version
    except RuntimeError:
        return None


def _dtype_code(t) -> Optional[int]:
    import torch

    if t.dtype == torch.float32:
        return DOTL_F32
    if t.dtype == torch.float16:
        return DOTL_F16
    if t.dtype == torch.bfloat16:
        return DOTL_BF16
    return None


class Kernels:
    """The extension module: same entry points as the reference's pybind module."""

    def __init__(self, lib) -> None:
        self._lib = lib
        self._wcache: Dict[int, Tuple[weakref.ReferenceType, tuple, object, object]] = {}
        self._wcache_builds = 0
        self._tile_split_kv = False
        self._layernorm_knobs = {"block_threads": 0, "warp_width": -1, "warp_rows": 0,
                                 "fused_reduce": True}
        self._wmma_flags = {"softmax_mode": 1, "mask_classify": True, "acc_formula": True,
                            "direct_o": True, "causal_reverse": True}

    # -- plumbing ----------------------------------------------------------------

    def _err(self) -> str:
        msg = self._lib.dotl_last_error()
        return msg.decode() if msg else ""

    def _check(self, rc: int) -> int:
        if rc < 0:
            raise RuntimeError(self._err())
        return rc

    @staticmethod
    def _stream(device) -> int:
        import torch

        return torch.cuda.current_stream(device).cuda_stream

    @staticmethod
    def _require_cuda(who: str, *tensors) -> None:
        for t in tensors:
            if t is not None and not t.is_cuda:
                raise RuntimeError(f"{who}: all inputs must be CUDA tensors")

    def raw(self):
        """The ctypes library handle, for tests that call the C ABI directly."""
        return self._lib

    # -- build smoke test (reference csrc/fused_attention.cu:96-114) ---------------

    def smoke_test_identity(self, x):
        import torch

        self._require_cuda("smoke_test_identity", x)
        if x.dtype != torch.float32:
            raise RuntimeError("smoke_test_identity: float32 only")
        xc = x.contiguous()
        out = torch.empty_like(xc)
        self._check(self._lib.dotl_smoke_test_identity(
            xc.data_ptr(), out.data_ptr(), xc.numel(), self._stream(x.device)))
        return out

    def mfma_layout_probe(self, device=None):
        import torch

        out = torch.empty(1280, dtype=torch.int32, device=device or "cuda")
        self._check(self._lib.dotl_mfma_layout_probe(out.data_ptr(), self._stream(out.device)))
        return out

    def mfma_ceiling_us(self, workgroups, iters, random_operands=True, reps=20, warmup=10,
                        device=None):
        """Average launch time (us, HIP events on this library's stream) of
        dotl_mfma_ceiling_probe; flops per launch = workgroups * 4 * iters * 16
        * 32768. Not in the reference's surface: a roofline measurement aid."""
        import torch

        dev = torch.device(device or "cuda")
        sink = torch.zeros(1, dtype=torch.float32, device=dev)
        stream = torch.cuda.current_stream(dev)

        def launch():
            self._check(self._lib.dotl_mfma_ceiling_probe(int(workgroups), int(iters),
                                                          1 if random_operands else 0,
                                                          sink.data_ptr(), self._stream(dev)))

        for _ in range(warmup):
            launch()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            launch()
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) * 1000.0 / reps

    def lds_dma_probe(self, src):
        """LDS contents after one wave's 16-byte-per-lane LDS-DMA load of src (256 int32)."""
        import torch

        out = torch.empty(512, dtype=torch.int32, device=src.device)
        self._check(self._lib.dotl_lds_dma_probe(src.data_ptr(), out.data_ptr(),
                                                 self._stream(src.device)))
        return out

    # -- LayerNorm (reference csrc/add_layernorm.cuh:491-692) -----------------------

    def _layernorm(self, who, x, sub, weight, bias, eps, normed_half, write_xnew=True,
                   split=False, row_index=None, io=None, copy_x=False):
        """Shared body of the LayerNorm methods.

        x_new is written when `write_xnew` and either a residual is added or a
        row index is given (then it is the gathered x). With `row_index`
        (int32 [rows], device), x/sub are read as [in_rows, D] and both
        outputs are [rows, D]; an entry outside [0, in_rows) gives zero rows.
        x may be float32, float16 or bfloat16 (weight and bias in the same
        dtype); x_new and the normed output then have x's dtype, except that
        a float32 x may ask for an fp16 (`normed_half`) or split (`split`)
        normed output.

        `io` = (slot, mode) binds the kernel's x (mode bit 0) and/or normed
        (bit 1) pointer to the device int64 [2] `slot` (a graph I/O slot,
        see bind_io): the kernel then reads/writes there instead of x /
        the normed tensor returned here, which only stands in for its shape.
        """
        import torch

        self._require_cuda(who, x, sub, weight, bias, row_index)
        if x.dim() < 1:
            raise RuntimeError(f"{who}: x needs at least one dimension")
        D = x.shape[-1]
        if weight.numel() != D or bias.numel() != D:
            raise RuntimeError(f"{who}: weight/bias must have {D} elements")
        if weight.dtype != x.dtype or bias.dtype != x.dtype:
            raise RuntimeError(f"{who}: weight/bias must share x's dtype")
        if sub is not None:
            if tuple(sub.shape) != tuple(x.shape):
                raise RuntimeError(f"{who}: x and sub must have identical shapes, got "
                                   f"{tuple(x.shape)} and {tuple(sub.shape)}")
            if sub.dtype != x.dtype:
                raise RuntimeError(f"{who}: x and sub must share a dtype")
        if (normed_half or split) and x.dtype != torch.float32:
            raise RuntimeError(f"{who}: normed_half is only defined for an fp32 input, got {x.dtype}")
        xcode = _dtype_code(x)
        if xcode is None:
            raise RuntimeError(f"{who}: x must be float32, float16 or bfloat16, got {x.dtype}")
        xc = x.contiguous()
        sc = sub.contiguous() if sub is not None else None
        wc, bc = weight.contiguous(), bias.contiguous()
        in_rows = xc.numel() // D if D else 0
        if row_index is not None:
            if row_index.dtype != torch.int32 or row_index.dim() != 1:
                raise RuntimeError(f"{who}: row_index must be a 1-D int32 tensor")
            ri = row_index.contiguous()
            rows = ri.numel()
            out_shape = (rows, D)
        else:
            ri = None
            rows = in_rows
            out_shape = tuple(xc.shape)
        want_xnew = (write_xnew and (sc is not None or ri is not None)) or copy_x
        x_new = torch.empty(out_shape, dtype=xc.dtype, device=xc.device) if want_xnew else None
        if split:
            normed = torch.empty((2, *out_shape), dtype=torch.float16, device=xc.device)
            ncode = DOTL_F16X2
        elif normed_half:
            normed = torch.empty(out_shape, dtype=torch.float16, device=xc.device)
            ncode = DOTL_F16
        else:
            normed = torch.empty(out_shape, dtype=xc.dtype, device=xc.device)
            ncode = xcode
        slot_ptr, mode = None, 0
        if io is not None:
            slot, mode = io
            if slot.dtype != torch.int64 or slot.numel() < 2 or not slot.is_cuda:
                raise RuntimeError(f"{who}: the io slot must be a CUDA int64 tensor of 2")
            slot_ptr = slot.data_ptr()
        rc = self._lib.dotl_layernorm(
            xc.data_ptr(), sc.data_ptr() if sc is not None else None, wc.data_ptr(),
            bc.data_ptr(), x_new.data_ptr() if x_new is not None else None, normed.data_ptr(),
            ri.data_ptr() if ri is not None else None, in_rows, rows, D, float(eps), xcode,
            ncode, slot_ptr, int(mode), self._stream(x.device))
        self._check(rc)
        if rc == DOTL_DECLINED:
            raise RuntimeError(self._err())
        return x_new, normed

    def bind_io(self, slot, src, dst) -> None:
        """slot[0] = src's address, slot[1] = dst's (either may be None: 0),
        written in stream order on the current stream: rebinds the kernels
        of a captured graph that read/write through `slot` (the `io`
        argument of the LayerNorm methods). Not in the reference's surface."""
        import torch

        if slot.dtype != torch.int64 or slot.numel() < 2 or not slot.is_cuda:
            raise RuntimeError("bind_io: the slot must be a CUDA int64 tensor of 2")
        self._check(self._lib.dotl_bind_io(
            slot.data_ptr(), src.data_ptr() if src is not None else None,
            dst.data_ptr() if dst is not None else None, self._stream(slot.device)))

    def fused_layernorm_rows(self, x, weight, bias, row_index, eps=1e-5, normed="float",
                             copy_x=True, io=None):
        """[x[row_index], LayerNorm(x[row_index])]: the gather into packed rows.

        Not in the reference's surface. `x` is [..., D] read as [in_rows, D];
        `row_index` int32 [rows] on the device; `normed` is "float", "half" or
        "split" (fp16 hi/lo planes [2, rows, D]); `copy_x` also returns the
        gathered rows of x (else None).
        """
        x_rows, out = self._layernorm("fused_layernorm", x, None, weight, bias, eps,
                                      normed == "half", write_xnew=copy_x,
                                      split=normed == "split", row_index=row_index, io=io)
        return [x_rows, out]

    def fused_add_layernorm_rows(self, x, sub, weight, bias, row_index, eps=1e-5, io=None):
        """LayerNorm(x + sub)[row_index] in fp32, zero rows where row_index < 0.

        Not in the reference's surface: the scatter back from packed rows to
        the padded layout, fused with the model's last add+LN and the
        reference's final masked_fill. The residual sum is not stored.
        """
        _, out = self._layernorm("fused_add_layernorm", x, sub, weight, bias, eps, False,
                                 write_xnew=False, row_index=row_index, io=io)
        return out

    def fused_add_layernorm(self, x, sub, weight, bias, eps=1e-5, normed_half=False):
        """[x + sub, LayerNorm(x + sub)] in one kernel."""
        if sub is None:
            raise RuntimeError("fused_add_layernorm: sub is required")
        x_new, normed = self._layernorm("fused_add_layernorm", x, sub, weight, bias, eps,
                                        normed_half)
        return [x_new, normed]

    def fused_add_layernorm_final(self, x, sub, weight, bias, eps=1e-5, io=None):
        """LayerNorm(x + sub) only: the residual sum is not stored.

        For the model's last add+LN, whose sum nothing reads. Same kernel as
        fused_add_layernorm with the x_new store compiled out.
        """
        _, normed = self._layernorm("fused_add_layernorm", x, sub, weight, bias, eps, False,
                                    write_xnew=False, io=io)
        return normed

    def fused_layernorm(self, x, weight, bias, eps=1e-5, out_half=False, io=None):
        """Plain LayerNorm over the last dimension."""
        _, normed = self._layernorm("fused_layernorm", x, None, weight, bias, eps, out_half,
                                    io=io)
        return normed

    def fused_layernorm_copy(self, x, weight, bias, eps=1e-5, normed="float", io=None):
        """[copy of x, LayerNorm(x)] from one read of x. Not in the reference's
        surface: a captured graph's entry norm, which reads the caller's x
        through the io slot and keeps the copy as the residual stream.
        `normed` is "float", "half" or "split"."""
        x_copy, out = self._layernorm("fused_layernorm", x, None, weight, bias, eps,
                                      normed == "half", split=normed == "split", io=io,
                                      copy_x=True)
        return [x_copy, out]

    def fused_layernorm_split(self, x, weight, bias, eps=1e-5, io=None):
        """LayerNorm as split fp16 planes [2, *x.shape]: hi, then lo = (v - hi) * 2^12.

        Not in the reference's surface: the input form of linear_bias_split,
        the fp32-class (fp16x3) projection. Same bytes as an fp32 output.
        """
        _, planes = self._layernorm("fused_layernorm", x, None, weight, bias, eps, False,
                                    split=True, io=io)
        return planes

    def fused_add_layernorm_split(self, x, sub, weight, bias, eps=1e-5):
        """[x + sub, LayerNorm(x + sub) as split fp16 planes]."""
        x_new, planes = self._layernorm("fused_add_layernorm", x, sub, weight, bias, eps, False,
                                        split=True)
        return [x_new, planes]

    # -- GEMM (reference csrc/linear_gelu.cuh:598-756) -------------------------------

    def weight_half(self, weight, want_lo: bool):
        """(w_hi, w_lo) fp16 copies of an fp32 [N, K] weight, cached per version."""
        import torch

        key = (weight.data_ptr(), tuple(weight.shape), str(weight.device),
               _version_or_none(weight))
        ent = self._wcache.get(id(weight))
        if ent is not None and ent[0]() is weight and ent[1] == key and (ent[3] is not None or not want_lo):
            return ent[2], ent[3]
        wc = weight.detach().contiguous()
        hi = torch.empty(wc.shape, dtype=torch.float16, device=wc.device)
        lo = torch.empty(wc.shape, dtype=torch.float16, device=wc.device) if want_lo else None
        self._check(self._lib.dotl_weight_split(
            wc.data_ptr(), hi.data_ptr(), lo.data_ptr() if lo is not None else None,
            wc.numel(), self._stream(wc.device)))
        if len(self._wcache) > 256:
            self._wcache = {k: v for k, v in self._wcache.items() if v[0]() is not None}
        self._wcache[id(weight)] = (weakref.ref(weight), key, hi, lo)
        self._wcache_builds += 1
        return hi, lo

    def cache_generation(self) -> int:
        """Number of weight-cache entries built so far (it moves iff one was)."""
        return self._wcache_builds

    def weight_cache_tensors(self) -> List[object]:
        """Every live cached weight (and 16-bit bias) copy (graph capture pins these)."""
        out = []
        for ref, _, hi, lo in self._wcache.values():
            if ref() is not None:
                out.append(hi)
                if lo is not None:
                    out.append(lo)
        return out

    def _gemm(self, who, x, weight, bias, tile, math, act, out_half, residual=None):
        import torch

        self._require_cuda(who, x, weight, bias)
        if weight.dim() != 2:
            raise RuntimeError(f"{who}: weight must be 2-D [N, K]")
        if x.dim() < 1 or x.shape[-1] != weight.shape[1]:
            raise RuntimeError(f"{who}: x's last dimension must match weight's, got "
                               f"{tuple(x.shape)} and {tuple(weight.shape)}")
        if bias.numel() != weight.shape[0]:
            raise RuntimeError(f"{who}: bias must have {weight.shape[0]} elements")
        xcode = _dtype_code(x)
        K, N = weight.shape[1], weight.shape[0]
        if K % 8 != 0 or K == 0:
            return None
        if weight.dtype in (torch.float16, torch.bfloat16):
            return self._gemm16(who, x, weight, bias, tile, act, residual)
        if (xcode not in (DOTL_F32, DOTL_F16) or weight.dtype != torch.float32
                or bias.dtype != torch.float32):
            return None  # declined: the caller falls back
        # math: -1 auto -> fp16 operands; 0 (the reference's tf32 slot) -> the
        # split fp16x3 path, which needs an fp32 x.
        m = DOTL_MATH_FP16 if math in (-1, None) else DOTL_MATH_FP16X3
        xc = x.contiguous()
        M = xc.numel() // K
        hi, lo = self.weight_half(weight, m == DOTL_MATH_FP16X3)
        bc = bias.contiguous()
        out = torch.empty((*xc.shape[:-1], N), dtype=torch.float16 if out_half else torch.float32,
                          device=xc.device)
        if residual is not None:
            if out_half or residual.dtype != torch.float32 or tuple(residual.shape) != tuple(out.shape):
                raise RuntimeError(f"{who}: residual must be float32 with the output's shape "
                                   f"{tuple(out.shape)}, and the output float32")
            rc_ = residual.contiguous()
            rc = self._check(self._lib.dotl_linear_residual(
                xc.data_ptr(), xcode, hi.data_ptr(), lo.data_ptr() if lo is not None else None,
                bc.data_ptr(), rc_.data_ptr(), out.data_ptr(), M, N, K, act, m, int(tile),
                self._stream(x.device)))
        else:
            rc = self._check(self._lib.dotl_linear(
                xc.data_ptr(), xcode, hi.data_ptr(), lo.data_ptr() if lo is not None else None,
                bc.data_ptr(), out.data_ptr(), DOTL_F16 if out_half else DOTL_F32, M, N, K, act,
                m, int(tile), self._stream(x.device)))
        if rc == DOTL_DECLINED:
            return None
        return out

    def linear_layernorm(self, x, weight, bias, residual, ln_weight, ln_bias, eps=1e-5,
                         normed="float", store_out=True, out_row=None, normed_rows=None,
                         tile=-1, io=None):
        """(h, LayerNorm(h)) with h = residual + x @ weight^T + bias, in one
        GEMM whose epilogue normalises each row (rows of up to 256 columns).

        Not in the reference's surface: linear_bias(residual=...) followed by
        fused_layernorm, bit for bit. `x` fp16 [..., K]; `normed` "float",
        "half" or "split" (fp16 hi/lo planes [2, rows, N]); `store_out` False
        skips h (None is returned for it). With `out_row` (int32 [M], device)
        row r of the normed output goes to row out_row[r] of a [normed_rows,
        N] fp32 tensor whose other rows are left as allocated (zero them with
        zero_rows). `io` = (slot, 2) binds the normed pointer to a graph I/O
        slot as the LayerNorm methods do. Returns None where the kernel
        declines (the caller runs the two ops)."""
        import torch

        who = "linear_layernorm"
        self._require_cuda(who, x, weight, bias, residual, ln_weight, ln_bias, out_row)
        if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
            raise RuntimeError(f"{who}: x [..., K] and weight [N, K] required")
        if x.dtype != torch.float16 or weight.dtype != torch.float32 or bias.dtype != torch.float32:
            return None
        N, K = weight.shape
        if (ln_weight.numel() != N or ln_bias.numel() != N or ln_weight.dtype != torch.float32
                or ln_bias.dtype != torch.float32):
            raise RuntimeError(f"{who}: LayerNorm weight/bias must be float32 with {N} elements")
        xc = x.contiguous()
        M = xc.numel() // K
        shape = (*xc.shape[:-1], N)
        hi, _ = self.weight_half(weight, False)
        rc_ = None
        if residual is not None:
            if residual.dtype != torch.float32 or tuple(residual.shape) != tuple(shape):
                raise RuntimeError(f"{who}: residual must be float32 of shape {tuple(shape)}")
            rc_ = residual.contiguous()
        out = torch.empty(shape, dtype=torch.float32, device=xc.device) if store_out else None
        nout, ncode, normed_rows, slot_ptr, orc = self._ln_outputs(
            who, xc.device, shape, M, N, normed, out_row, normed_rows, io)
        rc = self._check(self._lib.dotl_linear_layernorm(
            xc.data_ptr(), DOTL_F16, hi.data_ptr(), bias.contiguous().data_ptr(),
            rc_.data_ptr() if rc_ is not None else None,
            out.data_ptr() if out is not None else None, ln_weight.contiguous().data_ptr(),
            ln_bias.contiguous().data_ptr(), float(eps), nout.data_ptr(), ncode,
            orc.data_ptr() if orc is not None else None, int(normed_rows), slot_ptr, M, N, K,
            int(tile), self._stream(x.device)))
        if rc == DOTL_DECLINED:
            return None
        return out, nout

    @staticmethod
    def _ln_outputs(who, device, shape, M, N, normed, out_row, normed_rows, io):
        """The normed output of a LayerNorm epilogue (linear_layernorm,
        ffn_layernorm) and its arguments: (tensor, dtype code, normed_rows,
        graph I/O slot pointer or None, out_row contiguous or None)."""
        import torch

        if out_row is not None:
            if out_row.dtype != torch.int32 or out_row.numel() != M or normed != "float":
                raise RuntimeError(f"{who}: out_row must be int32 [{M}] with a float normed output")
            if normed_rows is None:
                raise RuntimeError(f"{who}: out_row needs normed_rows")
            nshape = (int(normed_rows), N)
        else:
            normed_rows = M
            nshape = shape
        if normed == "split":
            nout = torch.empty((2, *nshape), dtype=torch.float16, device=device)
            ncode = DOTL_F16X2
        elif normed == "half":
            nout = torch.empty(nshape, dtype=torch.float16, device=device)
            ncode = DOTL_F16
        elif normed == "float":
            nout = torch.empty(nshape, dtype=torch.float32, device=device)
            ncode = DOTL_F32
        else:
            raise RuntimeError(f"{who}: normed must be 'float', 'half' or 'split'")
        slot_ptr = None
        if io is not None:
            slot, mode = io
            if mode != 2 or slot.dtype != torch.int64 or slot.numel() < 2 or not slot.is_cuda:
                raise RuntimeError(f"{who}: io must be (a CUDA int64 slot of 2, 2)")
            slot_ptr = slot.data_ptr()
        orc = out_row.contiguous() if out_row is not None else None
        return nout, ncode, int(normed_rows), slot_ptr, orc

    def ffn_layernorm(self, x, w1, b1, w2, b2, residual, ln_weight, ln_bias, eps=1e-5,
                      normed="float", store_out=False, out_row=None, normed_rows=None, io=None,
                      zero_padded=False):
        """(y, LayerNorm(y)) with y = residual + GELU(x @ w1^T + b1) @ w2^T + b2
        in one kernel, for d_model 256 and d_ff a multiple of 64 up to 2048.

        Not in the reference's surface: linear_gelu(x, w1, b1, out_half=True)
        followed by linear_layernorm(h, w2, b2, residual, ...), bit for bit.
        `x` fp16 [..., 256]; w1 [d_ff, 256], w2 [256, d_ff] fp32 (their fp16
        copies come from the weight cache); `residual` fp32 like y or None;
        `normed`, `out_row`, `normed_rows` and `io` as in linear_layernorm;
        `zero_padded` (with an increasing out_row): the rows out_row does not
        name are zeroed too (no zero_rows call needed). y is returned only
        with store_out (else None). Returns None where the kernel declines
        (the caller runs the two GEMMs)."""
        import torch

        who = "ffn_layernorm"
        self._require_cuda(who, x, w1, b1, w2, b2, residual, ln_weight, ln_bias, out_row)
        if (w1.dim() != 2 or w2.dim() != 2 or x.shape[-1] != w1.shape[1]
                or tuple(w2.shape) != (w1.shape[1], w1.shape[0])):
            raise RuntimeError(f"{who}: x [..., D], w1 [F, D] and w2 [D, F] required")
        if (x.dtype != torch.float16 or w1.dtype != torch.float32 or w2.dtype != torch.float32
                or b1.dtype != torch.float32 or b2.dtype != torch.float32):
            return None
        F, D = w1.shape
        if (ln_weight.numel() != D or ln_bias.numel() != D or ln_weight.dtype != torch.float32
                or ln_bias.dtype != torch.float32 or b1.numel() != F or b2.numel() != D):
            raise RuntimeError(f"{who}: biases and LayerNorm weight/bias must be float32 of "
                               f"{F} / {D} elements")
        xc = x.contiguous()
        M = xc.numel() // D
        shape = (*xc.shape[:-1], D)
        w1h, _ = self.weight_half(w1, False)
        w2h, _ = self.weight_half(w2, False)
        rc_ = None
        if residual is not None:
            if residual.dtype != torch.float32 or tuple(residual.shape) != tuple(shape):
                raise RuntimeError(f"{who}: residual must be float32 of shape {tuple(shape)}")
            rc_ = residual.contiguous()
        out = torch.empty(shape, dtype=torch.float32, device=xc.device) if store_out else None
        nout, ncode, normed_rows, slot_ptr, orc = self._ln_outputs(
            who, xc.device, shape, M, D, normed, out_row, normed_rows, io)
        rc = self._check(self._lib.dotl_ffn_layernorm(
            xc.data_ptr(), DOTL_F16, w1h.data_ptr(), b1.contiguous().data_ptr(), w2h.data_ptr(),
            b2.contiguous().data_ptr(), rc_.data_ptr() if rc_ is not None else None,
            out.data_ptr() if out is not None else None, ln_weight.contiguous().data_ptr(),
            ln_bias.contiguous().data_ptr(), float(eps), nout.data_ptr(), ncode,
            orc.data_ptr() if orc is not None else None, normed_rows,
            1 if (zero_padded and orc is not None) else 0, slot_ptr, M, D, F,
            self._stream(x.device)))
        if rc == DOTL_DECLINED:
            return None
        return out, nout

    def zero_rows(self, out, row_map, io=None):
        """Zero row r of the fp32 [rows, width] `out` wherever row_map[r] < 0
        (int32 [rows]): the padded rows of a scattered output. `io` = (slot,
        2): out is the slot's bound output. Not in the reference's surface."""
        import torch

        self._require_cuda("zero_rows", out, row_map)
        if out.dtype != torch.float32 or row_map.dtype != torch.int32:
            raise RuntimeError("zero_rows: out float32 and row_map int32 required")
        width = out.shape[-1]
        rows = out.numel() // width if width else 0
        if row_map.numel() != rows:
            raise RuntimeError(f"zero_rows: row_map must have {rows} entries")
        slot_ptr = io[0].data_ptr() if io is not None else None
        self._check(self._lib.dotl_zero_rows(out.data_ptr(), row_map.contiguous().data_ptr(),
                                             rows, width, slot_ptr, self._stream(out.device)))

    def bias_f32(self, bias):
        """An fp32 copy of a 16-bit bias (the epilogue adds in fp32), cached
        per tensor and version like the weight copies."""
        import torch

        key = (bias.data_ptr(), bias.numel(), str(bias.device), _version_or_none(bias))
        ent = self._wcache.get(("bias", id(bias)))
        if ent is not None and ent[0]() is bias and ent[1] == key:
            return ent[2]
        b32 = bias.detach().to(torch.float32).contiguous()
        self._wcache[("bias", id(bias))] = (weakref.ref(bias), key, b32, None)
        self._wcache_builds += 1
        return b32

    def _gemm16(self, who, x, weight, bias, tile, act, residual):
        """A 16-bit model's projection: x, W (as it is) and the output in the
        weight's dtype, one MFMA pass (fp16 or bf16 operands), fp32
        accumulation, bias and GELU. The residual epilogue is fp32-only:
        with one the call declines and the caller adds it."""
        import torch

        if x.dtype != weight.dtype or residual is not None:
            return None
        code = DOTL_F16 if weight.dtype == torch.float16 else DOTL_BF16
        K, N = weight.shape[1], weight.shape[0]
        xc, wc = x.contiguous(), weight.detach().contiguous()
        M = xc.numel() // K
        b32 = self.bias_f32(bias)
        out = torch.empty((*xc.shape[:-1], N), dtype=weight.dtype, device=xc.device)
        rc = self._check(self._lib.dotl_linear(
            xc.data_ptr(), code, wc.data_ptr(), None, b32.data_ptr(), out.data_ptr(), code, M, N,
            K, act, DOTL_MATH_FP16, int(tile), self._stream(x.device)))
        if rc == DOTL_DECLINED:
            return None
        return out

    def linear_bias_split(self, planes, weight, bias, tile=-1, out_half=False,
                          split_weight=True):
        """x @ weight^T + bias with x given as split fp16 planes [2, ..., K]
        (fused_layernorm_split's output). split_weight=True: the fp16x3
        arithmetic, three MFMA passes, fp32-class products; False: fp16x2,
        hi(x)*W + lo(x)*W with W in fp16, two passes. Not in the reference's
        surface.
        """
        import torch

        who = "linear_bias"
        self._require_cuda(who, planes, weight, bias)
        if planes.dtype != torch.float16 or planes.dim() < 2 or planes.shape[0] != 2:
            raise RuntimeError(f"{who}: split input must be float16 [2, ..., K]")
        if planes.shape[-1] != weight.shape[1] or bias.numel() != weight.shape[0]:
            raise RuntimeError(f"{who}: shapes disagree: {tuple(planes.shape)}, "
                               f"{tuple(weight.shape)}, {tuple(bias.shape)}")
        K, N = weight.shape[1], weight.shape[0]
        pc = planes.contiguous()
        M = pc[0].numel() // K
        hi, lo = self.weight_half(weight, bool(split_weight))
        out = torch.empty((*pc.shape[1:-1], N), dtype=torch.float16 if out_half else torch.float32,
                          device=pc.device)
        rc = self._check(self._lib.dotl_linear(
            pc.data_ptr(), DOTL_F16X2, hi.data_ptr(), lo.data_ptr() if lo is not None else None,
            bias.contiguous().data_ptr(), out.data_ptr(), DOTL_F16 if out_half else DOTL_F32,
            M, N, K, DOTL_ACT_NONE, DOTL_MATH_FP16X3 if split_weight else DOTL_MATH_FP16X2,
            int(tile), self._stream(pc.device)))
        if rc == DOTL_DECLINED:
            return None
        return out

    def linear_bias_planes(self, hi, lo, weight, bias, out, split_weight=False):
        """linear_bias_split with the two planes as separate [M, K] fp16
        tensors (each contiguous; e.g. a block of rows of a [2, rows, K]
        LayerNorm output) and the result written into `out` ([M, N], fp16 or
        fp32, contiguous; e.g. a block of rows of a larger output). Not in
        the reference's surface. Returns `out`, or None where declined."""
        import torch

        who = "linear_bias"
        self._require_cuda(who, hi, lo, weight, bias, out)
        K, N = weight.shape[1], weight.shape[0]
        if (hi.dtype != torch.float16 or lo.dtype != torch.float16 or hi.shape != lo.shape
                or hi.shape[-1] != K or not hi.is_contiguous() or not lo.is_contiguous()):
            raise RuntimeError(f"{who}: hi and lo must be contiguous float16 [M, {K}] planes")
        M = hi.numel() // K
        if (out.dtype not in (torch.float16, torch.float32) or not out.is_contiguous()
                or out.numel() != M * N):
            raise RuntimeError(f"{who}: out must be a contiguous float16/float32 [{M}, {N}]")
        whi, wlo = self.weight_half(weight, bool(split_weight))
        rc = self._check(self._lib.dotl_linear_planes(
            hi.data_ptr(), lo.data_ptr(), whi.data_ptr(), wlo.data_ptr() if wlo is not None else None,
            bias.contiguous().data_ptr(), out.data_ptr(),
            DOTL_F16 if out.dtype == torch.float16 else DOTL_F32, M, N, K,
            DOTL_MATH_FP16X3 if split_weight else DOTL_MATH_FP16X2, -1, self._stream(hi.device)))
        if rc == DOTL_DECLINED:
            return None
        return out

    def linear_bias(self, x, weight, bias, tile=-1, math=-1, out_half=False, residual=None):
        """x @ weight^T + bias, or None when the shape/dtype is not covered.

        `residual` (not in the reference's signature; appended, default None):
        an fp32 tensor of the output's shape added in the epilogue, the
        residual add of the add+LayerNorm that follows out_proj / ffn_out.
        """
        return self._gemm("linear_bias", x, weight, bias, tile, math, DOTL_ACT_NONE, out_half,
                          residual)

    def linear_gelu(self, x, weight, bias, tile=-1, math=-1, out_half=False):
        """GELU_erf(x @ weight^T + bias), or None when not covered.

        `out_half` (not in the reference's signature; appended, default off)
        stores the GELU output as fp16 for a consumer that narrows it anyway.
        """
        return self._gemm("linear_gelu", x, weight, bias, tile, math, DOTL_ACT_GELU, out_half)

    # -- attention (reference csrc/attention_dispatch.cuh:332-519) -------------------

    def attention_split_plan(self, B, H, S, head_dim, is_causal=False, dtype=None,
                             has_mask=False, rows=None, impl=0, precision=0, splits=0):
        """(splits, workspace bytes) a call with these arguments resolves to.
        `splits`: 0 the library's choice, 1 none, n forced. Not in the
        reference's surface (its split choice is internal)."""
        import torch

        code = DOTL_F16 if dtype is None else _dtype_code(torch.empty(0, dtype=dtype))
        n = ctypes.c_int32(1)
        nbytes = ctypes.c_int64(0)
        rows = B * S if rows is None else rows
        self._check(self._lib.dotl_attention_split_plan(
            int(B), int(H), int(S), int(head_dim), 1 if is_causal else 0, int(code),
            1 if has_mask else 0, int(rows), int(impl), int(precision), int(splits),
            ctypes.byref(n), ctypes.byref(nbytes)))
        return int(n.value), int(nbytes.value)

    def fused_attention_forward(self, q, k, v, attn_mask=None, is_causal=False, scale=None,
                                impl=0, out_layout=0, precision=0, cu_seqlens=None,
                                max_seqlen=None, splits=0):
        """softmax(q k^T * scale + mask) v (reference csrc/attention_dispatch.cuh:332-519).

        q/k/v are [B, H, S, head_dim] of float32, float16 or bfloat16. Beyond
        the reference's arguments: with `cu_seqlens` (int32 [B + 1] on the
        device) they are packed sequences instead, [rows, H, head_dim] with
        sequence b at rows cu_seqlens[b] .. cu_seqlens[b + 1], `max_seqlen`
        (a host int) must bound every sequence's length (rows of a longer one
        past it are not computed), there is no mask, and the output is
        [rows, H * head_dim]. `splits`: key-range splits for the fp16 MFMA
        kernel (0 the library's choice from occupancy and the split knobs,
        1 none, n forced); the partials' workspace comes from torch's
        allocator on the current stream.
        """
        import torch

        who = "fused_attention_forward"
        if scale is None:
            raise TypeError(f"{who}: scale is required")
        if out_layout not in (0, 1):
            raise RuntimeError(f"{who}: out_layout must be 0 ([B,H,S,head_dim]) or 1 ([B,S,H*head_dim])")
        if not (0 <= impl <= 3):
            raise RuntimeError(f"{who}: impl must be 0 (auto), 1 (scalar), 2 (wmma) or 3 (tile)")
        if not (0 <= precision <= 4):
            raise RuntimeError(f"{who}: precision must be 0 (auto), 1 (fp32), 2 (tf32), 3 (fp16) or 4 (bf16)")
        if not (q.is_cuda and k.is_cuda and v.is_cuda):
            raise RuntimeError(f"{who}: q/k/v must be CUDA tensors")
        packed = cu_seqlens is not None
        want_dim = 3 if packed else 4
        if q.dim() != want_dim or k.dim() != want_dim or v.dim() != want_dim:
            raise RuntimeError(f"{who}: q/k/v must be " + (
                "3-D [rows, H, head_dim] with cu_seqlens" if packed else "4-D [B, H, S, head_dim]"))
        if q.shape != k.shape or q.shape != v.shape:
            raise RuntimeError(f"{who}: q/k/v must have identical shapes")
        if q.dtype != k.dtype or q.dtype != v.dtype:
            raise RuntimeError(f"{who}: q/k/v must share a dtype")
        code = _dtype_code(q)
        hd = int(q.shape[-1])
        if code is None:
            raise RuntimeError(f"{who}: impl={impl}, precision={precision} does not cover "
                               f"dtype={q.dtype}, head_dim={hd}: the kernels take float16, "
                               f"bfloat16 or float32 tensors")
        last = want_dim - 1
        pass_strided = (q.stride(last) == 1 and k.stride(last) == 1 and v.stride(last) == 1
                        and q.stride() == k.stride() and q.stride() == v.stride())
        if not pass_strided:
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        if any((st * q.element_size()) % 16 for st in q.stride()[:last]):
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        cu_ptr = None
        if packed:
            if attn_mask is not None:
                raise RuntimeError(f"{who}: packed sequences (cu_seqlens) take no attn_mask")
            if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or not cu_seqlens.is_cuda:
                raise RuntimeError(f"{who}: cu_seqlens must be a 1-D int32 CUDA tensor")
            if max_seqlen is None or int(max_seqlen) < 0:
                raise RuntimeError(f"{who}: max_seqlen (a host int) is required with cu_seqlens")
            cu = cu_seqlens.contiguous()
            cu_ptr = cu.data_ptr()
            rows, H = int(q.shape[0]), int(q.shape[1])
            B, S = cu.numel() - 1, int(max_seqlen)
            strides = (ctypes.c_int64 * 3)(0, q.stride(1), q.stride(0))
            out_layout = 1
            out = torch.empty((rows, H * hd), dtype=q.dtype, device=q.device)
            mask_ptr, ms, keep = None, None, None
            if rows == 0:
                B = 0
        else:
            B, H, S = (int(s) for s in q.shape[:3])
            rows = B * S
            strides = (ctypes.c_int64 * 3)(q.stride(0), q.stride(1), q.stride(2))
            mask_ptr = None
            ms = None
            keep = None
            if attn_mask is not None:
                if attn_mask.dtype != torch.bool:
                    raise RuntimeError(f"{who}: attn_mask must be a bool tensor")
                keep = attn_mask.contiguous().expand(B, H, S, S)
                mask_ptr = keep.data_ptr()
                ms = (ctypes.c_int64 * 4)(*keep.stride())
            if out_layout == 1:
                out = torch.empty((B, S, H * hd), dtype=q.dtype, device=q.device)
            else:
                out = torch.empty((B, H, S, hd), dtype=q.dtype, device=q.device)
        n_split, ws_bytes = 1, 0
        if B and H and S:
            n = ctypes.c_int32(1)
            nb = ctypes.c_int64(0)
            self._check(self._lib.dotl_attention_split_plan(
                B, H, S, hd, 1 if is_causal else 0, code, 1 if mask_ptr else 0, rows,
                int(impl), int(precision), int(splits), ctypes.byref(n), ctypes.byref(nb)))
            n_split, ws_bytes = int(n.value), int(nb.value)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
        rc = self._lib.dotl_attention_forward(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), code,
            strides, mask_ptr, ms, out.data_ptr(), code,
            out_layout, B, H, S, hd, 1 if is_causal else 0, float(scale), int(impl),
            int(precision), cu_ptr, rows, n_split, ws.data_ptr() if ws is not None else None,
            ws_bytes, self._stream(q.device))
        self._check(rc)
        if rc == DOTL_DECLINED:
            raise RuntimeError(self._err())
        del keep
        return out

    # -- fused FFN block (reference csrc/ffn_block.cuh:270-311) ----------------------

    def fused_ffn_block(self, x, attn_out, norm1_w, norm1_b, ffn_in_w, ffn_in_b, ffn_out_w,
                        ffn_out_b, norm2_w, norm2_b, eps):
        """[x2, normed2] of the fused post-attention block, or [] when the widths
        are not covered (reference csrc/ffn_block.cuh:270-311). fp32 tensors;
        the weights are narrowed to fp16 through the same cache the GEMMs use."""
        import torch

        who = "fused_ffn_block"
        self._require_cuda(who, x, attn_out)
        if tuple(x.shape) != tuple(attn_out.shape):
            raise RuntimeError(f"{who}: x and attn_out must match, got "
                               f"{tuple(x.shape)} and {tuple(attn_out.shape)}")
        if x.dtype != torch.float32 or attn_out.dtype != torch.float32:
            raise RuntimeError(f"{who}: float32 only, got {x.dtype}")
        if ffn_in_w.dim() != 2 or ffn_out_w.dim() != 2:
            raise RuntimeError(f"{who}: ffn weights must be 2-D")
        D = int(x.shape[-1])
        F = int(ffn_in_w.shape[0])
        if (tuple(ffn_in_w.shape) != (F, D) or tuple(ffn_out_w.shape) != (D, F)):
            raise RuntimeError(f"{who}: weight shapes disagree with d_model={D} ffn_dim={F}")
        if D > 128 or F > 512 or D % 8 or F % 8:
            return []
        xc, ac = x.contiguous(), attn_out.contiguous()
        rows = xc.numel() // D
        win, _ = self.weight_half(ffn_in_w, False)
        wout, _ = self.weight_half(ffn_out_w, False)
        params = [t.contiguous().float() for t in (norm1_w, norm1_b, ffn_in_b, ffn_out_b,
                                                    norm2_w, norm2_b)]
        x_out = torch.empty_like(xc)
        normed = torch.empty_like(xc)
        rc = self._check(self._lib.dotl_ffn_block(
            xc.data_ptr(), ac.data_ptr(), params[0].data_ptr(), params[1].data_ptr(),
            win.data_ptr(), params[2].data_ptr(), wout.data_ptr(), params[3].data_ptr(),
            params[4].data_ptr(), params[5].data_ptr(), x_out.data_ptr(), normed.data_ptr(),
            rows, D, F, float(eps), self._stream(x.device)))
        if rc == DOTL_DECLINED:
            return []
        return [x_out, normed]

    # -- knobs (reference csrc/fused_attention.cu:157-366) -------------------------

    def wmma_set_fp16(self, on: bool) -> None:
        self._lib.dotl_wmma_set_fp16(1 if on else 0)

    def wmma_fp16(self) -> bool:
        return bool(self._lib.dotl_wmma_fp16())

    def wmma_set_cp_async(self, mode: int) -> None:
        self._lib.dotl_wmma_set_cp_async(int(mode))

    def attention_set_pipeline(self, waves: int = 0, stages: int = 0) -> None:
        """Force the LDS-DMA attention kernel's waves per workgroup (1, 2, 4, 8)
        and pipeline stages (1-4); 0 restores the automatic choice.
        A measurement knob; not in the reference's surface."""
        self._lib.dotl_attention_set_pipeline(int(waves), int(stages))

    def wmma_cp_async_mode(self) -> int:
        return int(self._lib.dotl_wmma_cp_async_mode())

    # Knobs the reference's scripts flip for A/B runs. They name NVIDIA-kernel
    # variants with no counterpart here; they are accepted and remembered so
    # such scripts run, and change nothing.
    def wmma_set_softmax_mode(self, mode: int) -> None:
        if mode not in (0, 1, 2):
            raise RuntimeError("wmma_set_softmax_mode: mode must be 0, 1 or 2")
        self._wmma_flags["softmax_mode"] = mode

    def wmma_softmax_mode(self) -> int:
        return self._wmma_flags["softmax_mode"]

    def wmma_set_mask_classify(self, on: bool) -> None:
        self._wmma_flags["mask_classify"] = bool(on)

    def wmma_mask_classify_enabled(self) -> bool:
        return self._wmma_flags["mask_classify"]

    def wmma_set_acc_formula(self, on: bool) -> None:
        self._wmma_flags["acc_formula"] = bool(on)

    def wmma_acc_formula_enabled(self) -> bool:
        return self._wmma_flags["acc_formula"]

    def wmma_acc_formula_ok(self) -> List[bool]:
        return [True, True]

    def wmma_set_direct_o(self, on: bool) -> None:
        self._wmma_flags["direct_o"] = bool(on)

    def wmma_direct_o_enabled(self) -> bool:
        return self._wmma_flags["direct_o"]

    def wmma_set_split_kv(self, on: bool) -> None:
        """Let the MFMA kernel split the key range when the grid is small."""
        self._lib.dotl_wmma_set_split_kv(1 if on else 0)

    def wmma_split_kv_enabled(self) -> bool:
        return bool(self._lib.dotl_wmma_split_kv_enabled())

    def wmma_set_split_count(self, n: int) -> None:
        """Force n key splits on calls that leave the choice to the library
        (0 restores the occupancy choice)."""
        self._lib.dotl_wmma_set_split_count(int(n))

    def wmma_split_count(self, B, H, S, head_dim, is_causal) -> int:
        """Key splits an fp16 call of this shape would run (1: none)."""
        return self.attention_split_plan(B, H, S, head_dim, is_causal)[0]

    def wmma_set_causal_reverse(self, on: bool) -> None:
        self._wmma_flags["causal_reverse"] = bool(on)

    def wmma_causal_reverse_enabled(self) -> bool:
        return self._wmma_flags["causal_reverse"]

    def wmma_grid_info(self, B, H, S, head_dim) -> List[int]:
        """{grid blocks, blocks resident at once, BLOCK_M, BLOCK_N} of the MFMA kernel."""
        if head_dim not in (32, 64, 128):
            return [0, 0, 0]
        waves = 1 if S <= 32 else (2 if S <= 64 else 4)
        bm = 32 * waves
        blocks = ((S + bm - 1) // bm) * B * H
        per_cu = 1 if head_dim == 128 else 2
        return [blocks, 256 * 4 * per_cu // waves, bm, 64]

    def layernorm_set_block_threads(self, threads: int) -> None:
        self._layernorm_knobs["block_threads"] = int(threads)

    def layernorm_set_warp_width(self, width: int) -> None:
        self._layernorm_knobs["warp_width"] = int(width)

    def layernorm_warp_width(self) -> int:
        return 8192  # one wavefront per row at every width

    def layernorm_set_warp_rows(self, rows: int) -> None:
        self._layernorm_knobs["warp_rows"] = int(rows)

    def layernorm_warp_rows(self) -> int:
        return 4

    def layernorm_set_fused_reduce(self, enabled: bool) -> None:
        self._layernorm_knobs["fused_reduce"] = bool(enabled)

    def layernorm_fused_reduce_enabled(self) -> bool:
        return True

    def layernorm_block_threads(self, D: int) -> int:
        return 256

    def layernorm_blocks_per_sm(self, D: int) -> int:
        return 8

    # The tile kernels are an NVIDIA programming model; this build has none
    # (reference csrc/tile_attention.cu:1125-1148 is the stub these mirror).
    def tile_workspace_bytes(self, B, H, S, head_dim, is_causal, precision) -> int:
        return 0

    def tile_set_split_kv(self, enabled: bool) -> None:
        self._tile_split_kv = bool(enabled)

    def tile_split_kv_enabled(self) -> bool:
        return self._tile_split_kv


def get_kernels(verbose: bool = False):
    """Load (building once if needed) and return the kernels, or None if unavailable."""
    global _kernels, _load_attempted, _load_error
    if _load_attempted:
        return _kernels
    with _lock:
        if _load_attempted:
            return _kernels
        try:
            import torch

            if not torch.cuda.is_available():
                raise RuntimeError("no HIP device is available (torch.cuda.is_available() is False)")
            if not os.path.exists(_LIB_PATH):
                build(verbose=verbose)
            _kernels = Kernels(load_library())
        except BaseException as exc:  # noqa: BLE001 - reported through load_error()
            _kernels = None
            _load_error = exc
        _load_attempted = True
    return _kernels


def load_error() -> Optional[BaseException]:
    """Whatever went wrong during the last get_kernels() attempt, if anything."""
    return _load_error
