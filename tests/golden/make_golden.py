"""Write the golden fixtures under tests/golden/ from the oracle.

The reference holds no golden vectors or fixtures for this path (its
verification scripts compute references live with torch), so these come from
this repository's own oracle, whose every function is pinned in
tests/test_oracle.py. Run from the repository root:

    python tests/golden/make_golden.py            # all fixtures
    python tests/golden/make_golden.py C1 C2      # a subset

Files:
  c1_layer.npz     C1 full output: oracle fp32 and the fp64 brute-force layer
  rows_<C>.npz     C2..C5: 16 sampled (batch, seq) rows of the oracle fp32
                   output, with input checksums that detect generator drift
  ops_kat.npz      tiny per-op known-answer tests from the fp64 brute force
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import torch  # noqa: E402

from oracle import brute  # noqa: E402
from oracle.inputs import CONFIGS, make_case  # noqa: E402
from oracle.layer import reference_layer  # noqa: E402

N_ROWS = 16


def checksums(x, mask, params):
    out = {"x_sum": np.float64(x.astype(np.float64).sum()),
           "x_abs_sum": np.float64(np.abs(x.astype(np.float64)).sum()),
           "x_head": x.reshape(-1)[:64].copy()}
    for name in ("layers.0.attention.q_proj.weight", "layers.0.ffn_out.weight"):
        out["w_sum." + name] = np.float64(params[name].astype(np.float64).sum())
    if mask is not None:
        out["lengths"] = mask.sum(1).astype(np.int64)
    return out


def sample_rows(cfg, mask, seed):
    r = np.random.default_rng(seed)
    B, S = cfg.batch_size, cfg.seq_len
    rows = []
    while len(rows) < N_ROWS:
        b, s = int(r.integers(0, B)), int(r.integers(0, S))
        if (b, s) not in rows:
            rows.append((b, s))
    if mask is not None:  # include a padded row when there is one
        pb = np.nonzero(~mask.all(1))[0]
        if len(pb):
            b = int(pb[0])
            rows[-1] = (b, int(np.nonzero(~mask[b])[0][0]))
    return np.array(rows, dtype=np.int64)


def make_c1():
    cfg = CONFIGS["C1"]
    x, mask, params = make_case(cfg)
    t = time.time()
    out32 = reference_layer(x, mask, params, cfg).numpy()
    out64 = brute.layer(x, mask, params, cfg.num_heads, cfg.causal)
    np.savez_compressed(os.path.join(HERE, "c1_layer.npz"), out32=out32, out64=out64,
                        **checksums(x, mask, params))
    print(f"C1: {time.time() - t:.1f}s  max|fp32 - fp64| = {np.abs(out32 - out64).max():.3e}")


def make_rows(name):
    cfg = CONFIGS[name]
    x, mask, params = make_case(cfg)
    t = time.time()
    out = reference_layer(x, mask, params, cfg).numpy()
    rows = sample_rows(cfg, mask, 7 + cfg.seed_offset)
    vals = np.stack([out[b, s] for b, s in rows])
    np.savez_compressed(os.path.join(HERE, f"rows_{name}.npz"), rows=rows, values=vals,
                        **checksums(x, mask, params))
    print(f"{name}: {time.time() - t:.1f}s  {len(rows)} rows")


def make_kats():
    r = np.random.default_rng(2024)
    ln_x = r.standard_normal((3, 10))
    ln_w = r.standard_normal(10)
    ln_b = r.standard_normal(10)
    lin_x = r.standard_normal((4, 8))
    lin_w = r.standard_normal((6, 8))
    lin_b = r.standard_normal(6)
    g_x = np.linspace(-5, 5, 41)
    q, k, v = (r.standard_normal((1, 2, 9, 4)) for _ in range(3))
    valid = np.array([[1, 1, 1, 0, 1, 1, 0, 1, 1]], dtype=bool)
    np.savez_compressed(
        os.path.join(HERE, "ops_kat.npz"),
        ln_x=ln_x, ln_w=ln_w, ln_b=ln_b, ln_out=brute.layer_norm(ln_x, ln_w, ln_b),
        lin_x=lin_x, lin_w=lin_w, lin_b=lin_b, lin_out=brute.linear(lin_x, lin_w, lin_b),
        gelu_x=g_x, gelu_out=brute.gelu(g_x),
        att_q=q, att_k=k, att_v=v, att_valid=valid,
        att_out=brute.attention(q, k, v, None, False),
        att_out_causal=brute.attention(q, k, v, None, True),
        att_out_masked=brute.attention(q, k, v, valid, False),
    )
    print("ops_kat written")


def main(argv):
    torch.set_num_threads(os.cpu_count() or 1)
    which = argv or ["KAT", "C1", "C2", "C3", "C4", "C5"]
    for name in which:
        if name == "KAT":
            make_kats()
        elif name == "C1":
            make_c1()
        else:
            make_rows(name)


if __name__ == "__main__":
    main(sys.argv[1:])
