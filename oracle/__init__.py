"""CPU oracle for the single-transformer-layer forward pass.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (the
`distraction-optimizedtransformerlayer_amd/` source root: `kernel_ext.py`,
`optimized/`, `csrc/`) may import, call or link anything here. Only `tests/`,
`__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg use it, and only
as the checker or as the timed CPU baseline, never as the thing measured.

Modules:

  inputs   portable seeded generator for the five BASELINE configs (numpy PCG64)
  layer    fp32/fp64 torch-CPU restatement of BaselineTransformer(num_layers=1)
           (torch_transformer_benchmark.py:70-133, 222-272)
  brute    fp64 numpy restatements of each op, written as explicit loops or
           closed forms, used to pin `layer` on tiny shapes
  compare  the harness's element rule (torch_transformer_benchmark.py:557-624)

Every function is pinned by a test in tests/test_oracle.py against closed
forms, brute force or invariants; none is "parity unpinned".
"""
