"""The C-ABI library: it loads, exports every symbol include/dotl.h declares, and
its host-side argument checks answer without touching a device."""

import ctypes
import os
import re

import pytest

from conftest import PKG_ROOT, REPO

HEADER = os.path.join(REPO, "include", "dotl.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dotl_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401 - the HIP runtime must be loaded before the library

    import kernel_ext

    path = kernel_ext.library_path()
    if not os.path.exists(path):
        kernel_ext.build()
    return kernel_ext.load_library(path)


def test_header_and_loader_agree():
    import kernel_ext

    assert _declared() == sorted(kernel_ext.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    missing = [s for s in _declared() if not hasattr(lib, s)]
    assert not missing, missing


def test_abi_and_target(lib):
    assert lib.dotl_abi_version() == 3
    assert lib.dotl_target() == b"gfx950"


def test_linear_declines_k_not_multiple_of_8(lib):
    # Returns before any device call: K % 8 != 0 is outside the 16-byte staging.
    rc = lib.dotl_linear(None, 0, None, None, None, None, 0, 4, 4, 12, 0, 0, -1, None)
    assert rc == 1
    assert b"multiple of 8" in lib.dotl_last_error()


def test_linear_rejects_bad_codes(lib):
    assert lib.dotl_linear(None, 7, None, None, None, None, 0, 4, 4, 16, 0, 0, -1, None) == -1
    assert lib.dotl_linear(None, 0, None, None, None, None, 0, 4, 4, 16, 5, 0, -1, None) == -1
    # fp16x3 without the weight residual
    assert lib.dotl_linear(None, 0, None, None, None, None, 0, 4, 4, 16, 0, 1, -1, None) == -1
    # fp16x2 (split x only) takes x as split planes (dtype 2), nothing else
    assert lib.dotl_linear(None, 1, None, None, None, None, 0, 4, 4, 64, 0, 2, -1, None) == -1
    assert b"split fp16 planes" in lib.dotl_last_error()
    assert lib.dotl_linear(None, 2, None, None, None, None, 0, 0, 4, 64, 0, 2, -1, None) == 0
    # the residual epilogue needs its residual
    assert lib.dotl_linear_residual(None, 1, None, None, None, None, None, 4, 4, 64, 0, 0, -1,
                                    None) == -1
    # tile ids beyond the menu
    assert lib.dotl_linear(None, 1, None, None, None, None, 0, 4, 4, 64, 0, 0, 20, None) == -1
    assert b"unknown tile id" in lib.dotl_last_error()
    # empty problems launch nothing and succeed
    assert lib.dotl_linear(None, 0, None, None, None, None, 0, 0, 4, 16, 0, 0, -1, None) == 0


def _attn(lib, **kw):
    args = dict(dtype=1, out_layout=1, B=1, H=1, S=0, hd=64, causal=0, impl=0, prec=0)
    args.update(kw)
    strides = (ctypes.c_int64 * 3)(0, 0, 0)
    return lib.dotl_attention_forward(None, None, None, args["dtype"], strides, None, None,
                                      None, args.get("out_dtype", args["dtype"]),
                                      args["out_layout"], args["B"], args["H"], args["S"],
                                      args["hd"], args["causal"], ctypes.c_double(0.125),
                                      args["impl"], args["prec"], args.get("cu"),
                                      args.get("rows", 0), args.get("splits", 0),
                                      args.get("ws"), args.get("ws_bytes", 0), None)


def _plan(lib, B=1, H=8, S=2048, hd=64, dtype=1, mask=0, rows=None, splits=0, impl=0, prec=0):
    n = ctypes.c_int32(0)
    nb = ctypes.c_int64(0)
    rc = lib.dotl_attention_split_plan(B, H, S, hd, 0, dtype, mask, B * S if rows is None else rows,
                                       impl, prec, splits, ctypes.byref(n), ctypes.byref(nb))
    return rc, n.value, nb.value


def test_split_plan(lib):
    """Split-KV is chosen from occupancy for the fp16 MFMA kernel only, and
    sized as splits x rows x heads x (head_dim fp32 + (max, sum))."""
    lib.dotl_wmma_set_split_kv(1)
    lib.dotl_wmma_set_split_count(0)
    # B=1, H=8, S=2048: 16 query blocks x 8 heads = 128 workgroups -> 4 splits of 8 tiles
    rc, n, nb = _plan(lib)
    assert rc == 0 and n == 4 and nb == 4 * 2048 * 8 * (64 * 4 + 8)
    # a full grid (C4: 4 x 16 heads x 8 blocks of 256 queries) does not split
    assert _plan(lib, B=4, H=16, S=2048, hd=128)[1] == 1
    # short sequences run the one-tile kernel, never split unless forced
    assert _plan(lib, B=1, H=1, S=32)[1] == 1
    # fp32 / bf16 tensors and the exact kernel do not split
    assert _plan(lib, dtype=0)[1] == 1 and _plan(lib, dtype=3)[1] == 1
    assert _plan(lib, impl=1)[1] == 1
    # forcing: capped at one split per 64-key tile, rounded so no split is empty
    assert _plan(lib, S=256, splits=8)[1] == 4
    assert _plan(lib, S=2048, splits=3)[1] == 3
    assert _plan(lib, splits=1)[1:] == (1, 0)
    # the knobs: a forced count, and off
    lib.dotl_wmma_set_split_count(2)
    assert _plan(lib, B=4, H=16, S=2048, hd=128)[1] == 2
    lib.dotl_wmma_set_split_count(0)
    lib.dotl_wmma_set_split_kv(0)
    assert _plan(lib)[1] == 1
    assert _plan(lib, splits=4)[1] == 4       # an explicit count is not a knob's choice
    lib.dotl_wmma_set_split_kv(1)


def test_split_needs_its_workspace(lib):
    # forced splits with no workspace is an error; auto would run unsplit
    assert _attn(lib, B=1, H=8, S=2048, hd=64, splits=4) == -1
    assert b"workspace" in lib.dotl_last_error()
    assert _attn(lib, B=1, H=8, S=2048, hd=64, splits=0) == -1   # then the null tensors
    assert b"null pointer" in lib.dotl_last_error()


def test_attention_vocabulary_checks(lib):
    assert _attn(lib, out_layout=2) == -1
    assert _attn(lib, impl=4) == -1
    assert _attn(lib, prec=5) == -1
    # the tile model has no gfx950 counterpart: unavailable, as the reference's stub
    assert _attn(lib, impl=3) == -3
    assert b"tile" in lib.dotl_last_error()
    # a forced wmma with fp32 arithmetic is a category error
    assert _attn(lib, impl=2, prec=1) == -3
    # scalar (the exact fp32 kernel) has only fp32 arithmetic
    assert _attn(lib, impl=1, prec=3) == -3
    assert b"scalar has no fp16" in lib.dotl_last_error()
    # ... and covers head_dim up to 2048; an empty problem launches nothing
    assert _attn(lib, impl=1, hd=2049) == 1
    assert _attn(lib, impl=1, hd=2048) == 0
    assert _attn(lib, impl=1, hd=3) == 0
    # a forced MFMA kernel declines head dims it has no tile for, and tf32
    # (no tf32 matrix instruction on gfx950) for fp32 tensors
    assert _attn(lib, impl=2, hd=48) == 1
    assert _attn(lib, impl=2, dtype=0, prec=2) == 1
    assert b"tf32" in lib.dotl_last_error()
    # auto takes the exact kernel for those instead
    assert _attn(lib, impl=0, hd=48) == 0
    assert _attn(lib, impl=0, dtype=0, prec=2) == 0
    # an empty problem on the covered path launches nothing
    assert _attn(lib, S=0) == 0
    # packed sequences write the packed layout: out_layout 0 is refused
    cu = (ctypes.c_int32 * 2)(0, 4)
    assert _attn(lib, S=4, out_layout=0, cu=ctypes.cast(cu, ctypes.c_void_p)) == -1


def test_layernorm_checks(lib):
    def ln(rows, D, dtype=0, normed=None, row_index=None, in_rows=0, io=None, io_mode=0):
        return lib.dotl_layernorm(None, None, None, None, None, None, row_index, in_rows, rows, D,
                                  ctypes.c_double(1e-5), dtype,
                                  dtype if normed is None else normed, io, io_mode, None)

    assert ln(4, 0) == -1        # D = 0
    assert ln(0, 64) == 0        # no rows
    assert ln(4, 64, dtype=7) == -1       # unknown dtype
    # fp16 / bf16 inputs take their own dtype as the normed output
    assert ln(0, 64, dtype=1) == 0 and ln(0, 64, dtype=3) == 0
    assert ln(4, 64, dtype=3, normed=1) == -1
    assert b"x's dtype" in lib.dotl_last_error()
    assert ln(4, 64, dtype=1, normed=2) == -1   # split planes only from fp32
    idx = (ctypes.c_int32 * 1)(0)
    assert ln(1, 64, row_index=ctypes.cast(idx, ctypes.c_void_p), in_rows=-1) == -1
    # an io mode needs a slot; modes past 3 do not exist
    assert ln(4, 64, io_mode=1) == -1
    slot = (ctypes.c_int64 * 2)(0, 0)
    assert ln(4, 64, io=ctypes.cast(slot, ctypes.c_void_p), io_mode=4) == -1
    # null tensors that no slot replaces are an error
    assert ln(4, 64, io=ctypes.cast(slot, ctypes.c_void_p), io_mode=1) == -1
    assert b"null pointer" in lib.dotl_last_error()


def test_bind_io_checks(lib):
    assert lib.dotl_bind_io(None, None, None, None) == -1
    assert b"null slot" in lib.dotl_last_error()


def test_linear_layernorm_checks(lib):
    """The GEMM with the row LayerNorm: argument errors, then declines (1) for
    what the kernel does not serve, before any device work."""
    f = lib.dotl_linear_layernorm
    # normed dtype, scattered rows of a narrowed output, tile menu, extents
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 3, None, 4, None, 4, 64,
             64, -1, None) == -1
    assert b"normed output" in lib.dotl_last_error()
    row = ctypes.c_void_p(16)    # never dereferenced: every call below fails its checks first
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 1, row, 8, None, 4, 64, 64,
             -1, None) == -1
    assert b"out_row" in lib.dotl_last_error()
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 0, None, 5, None, 4, 64, 64,
             -1, None) == -1
    assert b"rows" in lib.dotl_last_error()
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 0, None, 4, None, 4, 64, 64,
             15, None) == -1
    assert b"tile" in lib.dotl_last_error()
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 0, None, -1, None, 4, 64,
             64, -1, None) == -1
    # declines: rows wider than a tile, N % 4, K % 64, fp32 x
    for x_dtype, n, k in ((1, 512, 64), (1, 66, 64), (1, 64, 96), (0, 64, 64)):
        assert f(None, x_dtype, None, None, None, None, None, None, 1e-5, None, 0, None, 4, None,
                 4, n, k, -1, None) == 1
    # empty problems succeed without pointers
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 0, None, 0, None, 0, 64, 64,
             -1, None) == 0
    assert f(None, 1, None, None, None, None, None, None, 1e-5, None, 0, None, 4, None, 4, 64, 64,
             -1, None) == -1
    assert b"null pointer" in lib.dotl_last_error()


def test_linear_planes_checks(lib):
    """Split planes given apart: the lo plane and the math are checked before
    the shared linear checks, all before any device work."""
    f = lib.dotl_linear_planes
    assert f(None, None, None, None, None, None, 0, 4, 64, 64, 1, -1, None) == -1
    assert b"lo plane" in lib.dotl_last_error()
    assert f(None, ctypes.c_void_p(8), None, None, None, None, 0, 4, 64, 64, 1, -1, None) == -1
    assert b"aligned" in lib.dotl_last_error()
    lo = ctypes.c_void_p(16)     # never dereferenced: every call below fails its checks first
    assert f(None, lo, None, None, None, None, 0, 4, 64, 64, 0, -1, None) == -1
    assert b"fp16x2 or fp16x3" in lib.dotl_last_error()
    assert f(None, lo, None, None, None, None, 0, 4, 64, 96, 2, -1, None) == 1   # K % 64
    assert f(None, lo, None, None, None, None, 0, 4, 64, 64, 1, -1, None) == -1
    assert b"split weight" in lib.dotl_last_error()
    assert f(None, lo, None, None, None, None, 0, 4, 64, 64, 2, -1, None) == -1
    assert b"null pointer" in lib.dotl_last_error()
    assert f(None, None, None, None, None, None, 0, 0, 64, 64, 2, -1, None) == 0


def test_ffn_layernorm_checks(lib):
    """The fused FFN: argument errors, then declines (1) for what the kernel
    does not serve, before any device work."""
    f = lib.dotl_ffn_layernorm
    n = None

    def call(x_dtype=1, normed_dtype=0, out_row=None, normed_rows=4, M=4, D=256, F=1024,
             zero_padded=0):
        return f(n, x_dtype, n, n, n, n, n, n, n, n, 1e-5, n, normed_dtype, out_row, normed_rows,
                 zero_padded, n, M, D, F, n)

    assert call(normed_dtype=3) == -1
    assert b"normed output" in lib.dotl_last_error()
    row = ctypes.c_void_p(16)    # never dereferenced: every call below fails its checks first
    assert call(normed_dtype=1, out_row=row, normed_rows=8) == -1
    assert b"out_row" in lib.dotl_last_error()
    assert call(normed_rows=5) == -1
    assert b"rows" in lib.dotl_last_error()
    assert call(zero_padded=1) == -1
    assert b"zero_padded" in lib.dotl_last_error()
    assert call(M=-1) == -1
    # declines: fp32 x, d_model other than 256, d_ff not a multiple of 64 or above 2048
    for kw in ({"x_dtype": 0}, {"D": 128}, {"F": 96}, {"F": 4096}, {"F": 0}):
        assert call(**kw) == 1, kw
    assert call(M=0, normed_rows=0) == 0
    assert call() == -1
    assert b"null pointer" in lib.dotl_last_error()


def test_zero_rows_checks(lib):
    assert lib.dotl_zero_rows(None, None, 4, 8, None, None) == -1
    assert b"null pointer" in lib.dotl_last_error()
    assert lib.dotl_zero_rows(None, None, -1, 8, None, None) == -1
    assert lib.dotl_zero_rows(None, None, 0, 8, None, None) == 0


def test_mfma_ceiling_probe_checks(lib):
    sink = ctypes.c_void_p(16)   # never dereferenced: every call below fails its checks first
    assert lib.dotl_mfma_ceiling_probe(1, 1, 1, None, None) == -1
    assert b"null sink" in lib.dotl_last_error()
    assert lib.dotl_mfma_ceiling_probe(0, 1, 1, sink, None) == -1
    assert lib.dotl_mfma_ceiling_probe(1, -1, 1, sink, None) == -1
    assert lib.dotl_mfma_ceiling_probe(1, (1 << 20) + 1, 0, sink, None) == -1
    assert b"workgroups" in lib.dotl_last_error()


def test_ffn_block_checks(lib):
    def ffn(rows, D, F):
        return lib.dotl_ffn_block(*([None] * 12), rows, D, F, ctypes.c_double(1e-5), None)

    # widths past 128, or not multiples of 8: declined, the caller runs the chain
    assert ffn(16, 256, 256) == 1
    assert ffn(16, 128, 640) == 1
    assert ffn(16, 60, 64) == 1
    assert b"not covered" in lib.dotl_last_error()
    # covered widths: an empty problem launches nothing; null tensors are an error
    assert ffn(0, 64, 64) == 0
    assert ffn(16, 48, 48) == -1
    assert ffn(-1, 64, 64) == -1


def test_knobs_roundtrip(lib):
    lib.dotl_wmma_set_fp16(0)
    assert lib.dotl_wmma_fp16() == 0
    lib.dotl_wmma_set_fp16(1)
    assert lib.dotl_wmma_fp16() == 1
    lib.dotl_wmma_set_cp_async(1)
    assert lib.dotl_wmma_cp_async_mode() == 1
    lib.dotl_wmma_set_cp_async(2)


def test_library_is_in_tree_not_site_packages():
    import kernel_ext

    assert os.path.dirname(kernel_ext.library_path()) == PKG_ROOT
