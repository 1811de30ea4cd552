"""dotl_attention_forward_noalloc, through the C ABI, against dotl_attention_forward.

The no-allocation entry point runs the same kernels with the split-KV
partials in the library's fixed per-device array instead of a workspace the
caller allocates. On the same inputs and split count the two entries must
give bit-identical outputs -- the arithmetic is identical, only where the
partials live differs -- on two calls in a row, the second smaller (the
array keeps the first call's contents), and a split request whose partials
do not fit the array is refused with a message, not run.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _args(q, out, B, H, S, hd, causal):
    strides = (ctypes.c_int64 * 3)(q.stride(0), q.stride(1), q.stride(2))
    return strides


def _call(lib, entry, q, k, v, B, H, S, hd, causal, splits, ws=None):
    out = torch.empty((B, S, H * hd), dtype=torch.float16, device=q.device)
    strides = (ctypes.c_int64 * 3)(q.stride(0), q.stride(1), q.stride(2))
    stream = torch.cuda.current_stream().cuda_stream
    common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, strides, None, None, out.data_ptr(),
              1, 1, B, H, S, hd, 1 if causal else 0, ctypes.c_double(hd ** -0.5), 0, 0, None,
              B * S, splits)
    if entry == "noalloc":
        rc = lib.dotl_attention_forward_noalloc(*common, stream)
    else:
        rc = lib.dotl_attention_forward(*common, ws.data_ptr() if ws is not None else None,
                                        ws.numel() if ws is not None else 0, stream)
    return rc, out


def _plan(lib, B, H, S, hd, causal, splits):
    n, nb = ctypes.c_int32(0), ctypes.c_int64(0)
    assert lib.dotl_attention_split_plan(B, H, S, hd, 1 if causal else 0, 1, 0, B * S, 0, 0,
                                         splits, ctypes.byref(n), ctypes.byref(nb)) == 0
    return n.value, nb.value


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_equals_workspace_entry(kernels, order):
    lib = kernels.raw()
    cap = lib.dotl_attention_noalloc_scratch_bytes()
    assert cap == 32 << 20
    cases = [(1, 8, 2048, 64, False, 0), (1, 4, 1024, 128, True, 3)]   # second is smaller
    for B, H, S, hd, causal, splits in cases:
        print(f"[no-alloc] B={B} H={H} S={S} hd={hd} causal={causal} splits={splits}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(S + hd)
        q, k, v = (torch.randn(B, H, S, hd, device="cuda", generator=g).half() for _ in range(3))
        n, nbytes = _plan(lib, B, H, S, hd, causal, splits)
        assert n > 1 and 0 < nbytes <= cap          # the partials really go to the array
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        rc_ws, want = _call(lib, "workspace", q, k, v, B, H, S, hd, causal, n, ws)
        rc_na, got = _call(lib, "noalloc", q, k, v, B, H, S, hd, causal, splits)
        torch.cuda.synchronize()
        assert rc_ws == 0 and rc_na == 0, lib.dotl_last_error()
        assert torch.equal(got, want)
        # and both equal the unsplit kernel to within fp16 output rounding
        _, one = _call(lib, "workspace", q, k, v, B, H, S, hd, causal, 1)
        torch.cuda.synchronize()
        assert (got.float() - one.float()).abs().max().item() < 2e-3


def test_noalloc_refuses_a_split_that_does_not_fit(kernels):
    lib = kernels.raw()
    B, H, S, hd = 4, 16, 2048, 128           # 16 splits would need ~1 GiB of partials
    q = torch.zeros(1, device="cuda", dtype=torch.float16)
    strides = (ctypes.c_int64 * 3)(H * S * hd, S * hd, hd)
    rc = lib.dotl_attention_forward_noalloc(q.data_ptr(), q.data_ptr(), q.data_ptr(), 1, strides,
                                            None, None, q.data_ptr(), 1, 1, B, H, S, hd, 0,
                                            ctypes.c_double(0.1), 0, 0, None, B * S, 16,
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == -1
    assert b"over the" in lib.dotl_last_error()
