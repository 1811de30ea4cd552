"""Runtime knobs for the optimized model, read at call time.

Same names, values and meaning as the reference's optimized/config.py, so a
script that flips `optimized.config.X` between runs keeps working. Always go
through the module (`config.CUDA_GRAPH = "off"`): a `from ... import` binds
the value, not the setting. The thresholds below were re-derived for MI355X
(256 CUs, 288 GB HBM3E) rather than carried over from the reference's card.

Seven knobs are new in this build:
  QKV_PRECISION  arithmetic of the fused QKV projection (auto, fp16x2, fp16x3, fp16)
  GELU_FP16      whether linear_gelu stores its output as fp16 for ffn_out
  ROW_PACKING    whether a padded batch runs on its valid rows only
  RESIDUAL_EPILOGUE  whether out_proj and ffn_out add the residual stream
  LN_EPILOGUE    whether they also apply the following LayerNorm (narrow rows)
  FFN_LN         whether the whole FFN (+ residual, + LayerNorm) runs as one kernel
"""

# Attention backend. One legal value: the custom kernels, never a prebuilt
# attention (reference optimized/config.py:15-26).
ATTENTION_BACKEND = "custom"

# WHICH attention kernel. "auto" = the first that covers the shape; "wmma"
# forces the MFMA kernel (the name is kept for command-line compatibility);
# "scalar" and "tile" name reference kernels this build does not have and
# are reported as uncovered.
ATTENTION_IMPL = "auto"
_IMPL_CODE = {"auto": 0, "scalar": 1, "wmma": 2, "tile": 3}

# The arithmetic attention contracts q/k/v in. "auto" resolves to fp16 on
# the MFMA kernel.
ATTENTION_PRECISION = "auto"
_PRECISION_CODE = {"auto": 0, "fp32": 1, "tf32": 2, "fp16": 3, "bf16": 4}

# Attention writes [B, S, H*head_dim], the layout out_proj reads.
_OUT_LAYOUT_BSHD = 1

# FFN first Linear fused with its GELU. "auto": fp16 operands; "tf32": the
# split fp16x3 arithmetic (fp32-class products; the slot the reference used
# for tf32); "off": F.linear + F.gelu.
LINEAR_GELU = "auto"

# Accepted for command-line compatibility; gfx950 staging has no cp.async.
CP_ASYNC = "auto"
_CP_ASYNC_CODE = {"off": 0, "sync": 1, "auto": 2}

# The model's entry LayerNorm on the custom kernel ("off": F.layer_norm).
LAYERNORM = "auto"

# The activation-free projections (QKV, out_proj, ffn_out) on the custom
# GEMM. "auto": fp16 operands; "tf32": split fp16x3; "off": F.linear.
LINEAR_BIAS = "auto"

# Above this many rows "auto" declines to F.linear. The MFMA GEMM has no
# measured crossover against the library GEMM at any row count the configs
# reach, so the bound only marks the int32 grid limit of the launch.
_LINEAR_BIAS_MAX_ROWS = 1 << 31

# Arithmetic of the fused QKV projection:
#   "auto" (default): "fp16x2" when some query row attends to fewer than
#          _QKV_SPLIT_MIN_KEYS keys (a causal mask, a short sequence, a short
#          valid length), else "fp16";
#   "fp16x2": the LayerNorm output as split fp16 hi+lo planes (~22 bits), the
#          weight in fp16: two MFMA passes;
#   "fp16x3": the weight split too: three passes, fp32-class products;
#   "fp16":   one pass on fp16 operands.
#
# This is where the accuracy budget is spent. The layer's error is a sum of
# fp16 operand roundings, and the projection's roundings perturb the
# attention SCORES; how much that moves the output depends on how many keys
# a query row spreads its weight over. Measured on MI355X against the fp32
# oracle, worst element with fp16x2 / fp16 QKV:
#   C5 (1-16 keys a row): 1.90e-3 / 2.07e-3 with 2 failing elements;
#   C3 (causal, row i sees i + 1 keys): 1.18e-3 / 1.67e-3;
#   C2 (>= 256 keys a row): 0.98e-3 / 1.03e-3; C4 (2048 keys): 1.89e-3 / 1.77e-3
#   (at C4 the worst element comes from ffn_in's fp16 operands, not QKV).
# So the split planes are spent where rows see few keys and the one-pass
# projection (half the MFMA work, the 256x256 tiles) runs elsewhere.
QKV_PRECISION = "auto"
_QKV_SPLIT_MIN_KEYS = 128
# Under "auto", an unpadded causal batch with sequences longer than
# _QKV_SPLIT_MIN_KEYS keeps the split planes only for the rows that attend to
# fewer keys -- each sequence's first _QKV_SPLIT_MIN_KEYS rows, whose queries
# see only keys from the same prefix -- and projects the rest in one fp16
# pass, as the configs whose rows all see >= 128 keys do. C3 (one causal
# sequence of 4096): the prefix is 3% of the rows.
_QKV_CAUSAL_PREFIX = True
# linear_bias `math` when the projection's input is not split planes (an
# fp32 or fp16 x): the split arithmetic for either split setting.
_QKV_MATH_CODE = {"fp16x3": 0, "fp16x2": 0, "fp16": -1}

# Hand attention its q/k/v in fp16 (the QKV GEMM rounds once in its
# epilogue instead of attention rounding while staging: bit-identical).
QKV_FP16 = "auto"
# No lower bound: on MI355X the fp16 read path costs the consumer nothing
# (the MFMA operands are fp16 either way), so halving the bytes never loses.
_QKV_FP16_MIN_ROWS = 0

# Store a LayerNorm's output as fp16 where the GEMM consuming it narrows to
# fp16 anyway (norm2 -> linear_gelu, and norm1 -> QKV when QKV_PRECISION is
# "fp16"). The residual stream and the final norm are never narrowed.
NORMED_FP16 = "auto"
_NORMED_FP16_MAX_K = 1 << 30

# Store GELU's output as fp16 for ffn_out, whose fp16 operand path narrows it
# with the same RNE: a moved rounding, bit-identical, half the traffic of the
# layer's widest intermediate.
GELU_FP16 = "auto"

# Fused post-attention block (add+LN, Linear+GELU, Linear, add+LN in one
# kernel, kernel_ext.fused_ffn_block) on the unpadded path: "auto" up to
# d_model _FFN_BLOCK_MAX_D (the reference's gate), "force" at any width the
# kernel covers (d_model and d_ff up to 128), "off" never. The kernel's
# outputs equal the unfused chain's, so this is a speed choice only.
FFN_BLOCK = "auto"
_FFN_BLOCK_MAX_D = 64

# math ids for linear_bias / linear_gelu: -1 auto (fp16), 0 the split fp16x3.
_GEMM_MATH_CODE = {"auto": -1, "tf32": 0}

# hipGraph capture (torch.cuda.CUDAGraph is hipGraph on ROCm).
#   "off" never; "auto" captures shapes up to _GRAPH_MAX_ACTIVATION elements
#   and keeps a graph only when its measured replay beats the eager forward
#   on the same input; "always" keeps every graph that replays correctly.
CUDA_GRAPH = "auto"

# Largest activation (B*S*D elements) "auto" tries to capture. Replays read
# the caller's input and write its output through an I/O slot, so a graph
# costs no copies at any size; the cap bounds the private pool a capture
# pins (the intermediates of one forward: ~1.5 GB at 41 M elements).
_GRAPH_MAX_ACTIVATION = 1 << 26

# "auto" keeps a graph only if its replay is at least this much faster than
# the eager forward (a smaller gain is within the timing noise).
_GRAPH_MIN_GAIN = 0.01

# A captured pool larger than this share of the card is released.
_GRAPH_POOL_SAFETY_FRACTION = 0.25

# Captured graphs held at once (each owns a private pool).
_GRAPH_MAX_ENTRIES = 4

# Eager forwards run on the capture stream before capture, so lazily built
# caches (the fused QKV weight, the fp16 weight copies) are allocated
# outside the graph's pool.
_GRAPH_WARMUP_ITERS = 2

# Refuse to capture with less than this much device memory free.
_GRAPH_MIN_FREE_BYTES = 512 << 20

# Padded batches: "auto" runs the layer on the valid rows only (gathered by
# the first LayerNorm, attention over packed sequences, scattered back by the
# final add+LayerNorm with zero padded rows); "off" runs all B*S rows and
# zeroes the padded ones with masked_fill, as the reference does. Same
# outputs either way (bit-identical on prefix masks); see optimized/packing.py.
ROW_PACKING = "auto"

# Residual adds in the GEMM epilogue: "auto" makes out_proj write x + attn
# and ffn_out write h1 + ffn (the same fp32 sums, bit-identical outputs), so
# the LayerNorms after them read one tensor and write only the normalised
# one; "off" keeps the reference's add+LayerNorm kernels. "auto" applies
# from d_model _RESIDUAL_EPILOGUE_MIN_D. Since tiles wholly inside the output
# load the residual and store in straight lines it pays at every config;
# same-box A/B (layer µs, min 1024 / 0, i.e. off / on below C3): C1 36.6 /
# 35.4, C2 96.0 / 93.6, C3 268.6 / 268.7, C5 574 / 544.
RESIDUAL_EPILOGUE = "auto"
_RESIDUAL_EPILOGUE_MIN_D = 0

# The LayerNorm after out_proj and after ffn_out in the same GEMM's epilogue
# (with the residual epilogue on): "auto" where one workgroup's tile spans a
# whole row (d_model <= _LN_EPILOGUE_MAX_D, a multiple of 4): the epilogue
# normalises each row with the LayerNorm kernels' arithmetic (bit-identical
# outputs) and the LayerNorm launches and their reads of the residual
# stream go away; "off" keeps the separate LayerNorms.
LN_EPILOGUE = "auto"
_LN_EPILOGUE_MAX_D = 256
# ... and from this many rows: the one tile built with it (128x256, one
# workgroup a CU) needs a few hundred tiles. Same-box A/B (layer µs, on /
# off): C5 (85 104 rows) 518 / 530; C1 (128 rows, one tile) 54.6 / 35.4,
# and with a 64x256 tile (two workgroups, bit-identical) still 39.1 / 34.5.
_LN_EPILOGUE_MIN_ROWS = 32768

# The FFN as one kernel (ffn_in, GELU, ffn_out, the residual add and the
# following LayerNorm; dotl_ffn_layernorm): "auto" where the LayerNorm
# epilogue above applies to ffn_out, d_model is 256 and d_ff a multiple of
# 64 up to 2048 (C5). The hidden activations then stay in LDS, a step of 64
# at a time, instead of making a round trip through HBM; outputs are
# bit-identical to the two GEMMs. "off" runs the two GEMMs.
FFN_LN = "auto"

# Arithmetic of a model with more than one block. Each block's fp16 operand
# roundings add to the residual stream the next block reads, so the error at
# the output grows with depth. "auto": in a multi-block forward, LINEAR_BIAS
# and LINEAR_GELU set to "auto" run as "tf32" (the split fp16x3, fp32-class
# GEMMs), which keeps a stack inside the 2e-3 / 2% element rule; measured on
# the padded mass-batch shape (d_model 256, 3000 sequences) at 4 blocks the
# worst element goes from 3.1e-3 (74 failing elements) to 1.8e-3 (none).
# "off": every block uses the single-block arithmetic.
STACK_PRECISION = "auto"

# Run a batch that does not fit in device memory as batch chunks: the chunk
# count is planned from the layer's per-token working set
# (model.forward_bytes_per_token) against _MICROBATCH_BUDGET_FRACTION of the
# free device memory, and doubled after each out-of-memory error down to
# _MICROBATCH_MIN_ROWS sequences a chunk.
MICROBATCH_FALLBACK = True
_MICROBATCH_MIN_ROWS = 1
_MICROBATCH_BUDGET_FRACTION = 0.85
