/*
 * dotl.h -- C ABI of libdotl_hip.so, the MI355X (gfx950) kernels behind the
 * single-transformer-layer forward pass.
 *
 * This is the drop-in boundary for the reference's pybind module
 * `transformer_kernels` (reference csrc/fused_attention.cu:118-376). Every
 * entry point below replaces one pybind entry; the Python shim
 * (kernel_ext.py in the package source root) rebuilds the reference's
 * torch-level signatures on top of these, so optimized/kernels.py calls the
 * same names with the same arguments.
 *
 * Conventions
 *   - Plain device pointers, int64 sizes and strides in ELEMENTS, a dtype
 *     code, and the HIP stream to launch on (hipStream_t passed as void*;
 *     NULL is the default stream). Nothing here allocates device memory:
 *     outputs and workspace are the caller's, so every entry point is legal
 *     inside hipGraph stream capture.
 *   - Return value: DOTL_OK (0) after launching, DOTL_DECLINED (1) when the
 *     case is outside what the kernels cover and nothing was launched (the
 *     caller picks a fallback, as the reference's undefined-tensor / empty-list
 *     returns do), and a negative DOTL_E_* code on error, with a message in
 *     dotl_last_error() (thread-local, valid until the next call on the same
 *     thread). Negative codes correspond to the reference's TORCH_CHECK raises.
 *   - Launches are asynchronous on `stream`; hipGetLastError is checked after
 *     every launch.
 *   - Load the library only after the process's HIP runtime is up (import
 *     torch first): it binds to the libamdhip64 already loaded.
 */
#ifndef DOTL_H
#define DOTL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DOTL_ABI_VERSION 3

#define DOTL_OK 0
#define DOTL_DECLINED 1
#define DOTL_E_INVALID (-1)   /* bad argument: the reference's TORCH_CHECK raise */
#define DOTL_E_LAUNCH (-2)    /* hipGetLastError reported a failure */
#define DOTL_E_UNSUPPORTED (-3) /* a forced impl/precision that does not exist */

/* dtype codes */
#define DOTL_F32 0
#define DOTL_F16 1
#define DOTL_F16X2 2 /* split fp16 planes [2][n]: hi = fp16(v), then
                        lo = fp16((v - hi) * 2^12); v ~= hi + lo * 2^-12 */
#define DOTL_BF16 3  /* bfloat16 */

/* linear activation codes */
#define DOTL_ACT_NONE 0
#define DOTL_ACT_GELU 1 /* exact erf GELU, F.gelu(approximate="none") */

/* linear math codes (the reference's `math` argument: -1 auto, 0 tf32,
 * reference csrc/linear_gelu.cuh:598-719) */
#define DOTL_MATH_FP16 0   /* fp16 operands, fp32 accumulate: one MFMA pass */
#define DOTL_MATH_FP16X3 1 /* split fp16 hi+lo operands, three MFMA passes:
                              fp32-class products (the reference's tf32 slot) */
#define DOTL_MATH_FP16X2 2 /* x as split fp16 hi+lo planes, W in fp16: two
                              passes, hi(x)*W + 2^-12 lo(x)*W */

/* Thread-local message for the last negative return; "" if none. */
const char* dotl_last_error(void);

/* DOTL_ABI_VERSION of the loaded library. */
int dotl_abi_version(void);

/* Name of the device the library was built for ("gfx950"). */
const char* dotl_target(void);

/* y[i] = x[i] for i < n (float32). Replaces smoke_test_identity
 * (reference csrc/fused_attention.cu:96-114). */
int dotl_smoke_test_identity(const float* x, float* y, int64_t n, void* stream);

/* Writes the accumulator (row, col) that each (lane, register) of one
 * v_mfma_f32_32x32x16_f16 and one v_mfma_f32_16x16x32_f16 holds, as
 * out[0 .. 64*16) = row*32+col for 32x32, then out[1024 .. 1024+64*4) =
 * row*16+col for 16x16 (int32 device buffer, 1280 elements). The MFMA
 * counterpart of the reference's accumulator probe (acc_row_probe_kernel,
 * reference csrc/attention_wmma.cuh:798-828), run as a test, not at start-up. */
int dotl_mfma_layout_probe(int32_t* out, void* stream);

/* Sustained matrix-core rate, no reference counterpart (a measurement aid
 * for the roofline): `workgroups` workgroups of 4 wavefronts, each wave
 * `iters` rounds of 16 v_mfma_f32_32x32x16_f16 (32768 flops each) on
 * register operands, random values when random_operands != 0 (as a GEMM's
 * fragments are: the clock then drops under the matrix cores' power draw)
 * else constants. Flops = workgroups * 4 * iters * 16 * 32768; the caller
 * times the launch on `stream`. `sink` (one float, device) is never written
 * in practice. */
int dotl_mfma_ceiling_probe(int64_t workgroups, int32_t iters, int32_t random_operands, float* sink,
                            void* stream);

/*
 * LayerNorm over the last dimension, optionally fused with a residual add.
 * Replaces fused_add_layernorm / fused_layernorm
 * (reference csrc/add_layernorm.cuh:491-692).
 *
 *   x, sub      [rows, D] contiguous, dtype `dtype` (DOTL_F32, DOTL_F16 or
 *               DOTL_BF16, the reference's float/Half/BFloat16 dispatch,
 *               csrc/add_layernorm.cuh:555-557). sub == NULL: plain LN.
 *   weight,bias [D], x's dtype
 *   x_new       [rows, D] output of x's dtype, x + sub rounded to that dtype
 *               (the value the statistics are taken of), or x alone when
 *               sub == NULL; may be NULL to skip the store
 *   normed      [rows, D] output, LayerNorm(x + sub) * weight + bias, of
 *               dtype normed_dtype: x's dtype; or, for a float32 x only,
 *               DOTL_F16 (RNE narrowing) or DOTL_F16X2 ([2][rows][D] split
 *               planes for the split-arithmetic GEMMs)
 *   row_index   optional (NULL) int32 [rows]: output row t reads input row
 *               row_index[t] of x and sub ([in_rows, D] each), and an entry
 *               outside [0, in_rows) writes zeros to every output of row t.
 *               Without it, x and sub are [rows, D] and in_rows is ignored.
 *               Packs the valid rows of a padded batch (gather) and returns
 *               them to the padded layout with zeroed padding (scatter) --
 *               the reference zeroes padded rows with masked_fill (reference
 *               optimized/layers.py:247-252, optimized/model.py:141-142); no
 *               reference counterpart of its own.
 *   io, io_mode graph I/O slot, no reference counterpart: with bit 0 of
 *               io_mode the kernel reads its x pointer from io[0] at run
 *               time (x may then be NULL), with bit 1 its normed pointer from
 *               io[1]. A captured graph then serves any input and output
 *               buffer, rebound by dotl_bind_io before each replay, without
 *               copies. io_mode 0: io unused (may be NULL).
 *   Statistics: fp32, mean then the centred sum of squares (biased variance),
 *   eps inside the square root.
 *   D in [1, 8192]; rows >= 0.
 */
int dotl_layernorm(const void* x, const void* sub, const void* weight, const void* bias,
                   void* x_new, void* normed, const int32_t* row_index, int64_t in_rows,
                   int64_t rows, int64_t D, double eps, int dtype, int normed_dtype,
                   const int64_t* io, int io_mode, void* stream);

/*
 * slot[0] = in, slot[1] = out, written by a one-wave kernel on `stream`, so
 * the write is ordered before the graph replay launched after it. slot is a
 * device int64 [2] that a captured graph's kernels read (dotl_layernorm's
 * io). No reference counterpart: the reference copies each input into the
 * captured graph's static buffer and clones its output
 * (reference optimized/graphs.py:49-73).
 */
int dotl_bind_io(int64_t* slot, const void* in, void* out, void* stream);

/*
 * Weight preparation for dotl_linear: w_hi = fp16(w) (RNE) and, when w_lo is
 * not NULL, w_lo = fp16((w - w_hi) * 2^12), the scaled residual the
 * DOTL_MATH_FP16X3 path consumes. n elements, float32 in.
 * No reference counterpart of its own: the reference narrows W inside the
 * GEMM's staging (reference csrc/linear_gelu.cuh:186-462); here the narrowing
 * is done once per weight version and cached by the caller.
 */
int dotl_weight_split(const float* w, void* w_hi, void* w_lo, int64_t n, void* stream);

/*
 * out[M, N] = act(x[M, K] @ W[N, K]^T + bias[N]) on MFMA.
 * Replaces linear_bias / linear_gelu (reference csrc/linear_gelu.cuh:598-756).
 *
 *   x         [M, K] contiguous, x_dtype DOTL_F32 (narrowed with RNE when
 *             staged), DOTL_F16, DOTL_F16X2 ([2][M][K] hi/lo planes), or
 *             DOTL_BF16 (with a bf16 W, one pass on v_mfma_f32_32x32x16_bf16,
 *             K % 64 == 0; the reference's BFloat16 dispatch,
 *             csrc/linear_gelu.cuh:598-719): a 16-bit model's own weights
 *   w_hi      [N, K] fp16 from dotl_weight_split (or a model's fp16 weight as
 *             it is), bf16 for a DOTL_BF16 x
 *   w_lo      [N, K] fp16 scaled residual; required for DOTL_MATH_FP16X3
 *   bias      [N] float32 (required; the reference's kernels always add one)
 *   out       [M, N], out_dtype DOTL_F32, DOTL_F16 (RNE; not with a bf16 x) or
 *             DOTL_BF16 (RNE; bf16 x only)
 *   act       DOTL_ACT_NONE / DOTL_ACT_GELU, applied in fp32 before the store
 *   math      DOTL_MATH_FP16, DOTL_MATH_FP16X3 (an fp16 x is exact in
 *             fp16, so with it the split path runs two passes: x*hi + x*lo;
 *             a DOTL_F16X2 x runs three: + lo(x)*hi(W)) or DOTL_MATH_FP16X2
 *             (DOTL_F16X2 x only; w_lo unused)
 *   tile      -1 auto; otherwise a tile id (0: 128x128, 1: 256x128 [one
 *             pass], 2: 64x64, 3: 256x256 [one pass], 4: 128x64; 5-8: 128x128,
 *             256x128 [one pass], 128x64, 64x64 with shallower pipelines that
 *             fit two workgroups per CU; 9-13: 256x256 [one pass], 128x128,
 *             256x128 [one pass], 128x128 [one pass, two stages], 128x64 with
 *             128-byte K rows; 14: 192x128 with 128-byte K rows [one or two
 *             passes]; 15-17: 8 waves a workgroup, two per SIMD, [one pass]:
 *             256x256 with 128-byte K rows, 256x256 with 64-byte K rows,
 *             256x128 with 128-byte K rows; 18: 128x256, 8 waves [one pass];
 *             19: 192x128, 8 waves [two passes]); 100 + id (id <= 4) forces
 *             the register-staged kernel (for measurement)
 *   fp16 / split-fp16 x with K % 64 == 0 runs the LDS-DMA pipelined kernel;
 *   anything else the register-staged one. Declines when K % 8 != 0, or a
 *   DOTL_F16X2 x with K % 64 != 0.
 */
int dotl_linear(const void* x, int x_dtype, const void* w_hi, const void* w_lo,
                const float* bias, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                int act, int math, int tile, void* stream);

/*
 * out[M, N] = residual[M, N] + act(x @ W^T + bias): dotl_linear with the
 * residual add the following add+LayerNorm would do (reference
 * csrc/add_layernorm.cuh:149-165, x_new = x + sub) moved into the GEMM's
 * epilogue, the same fp32 sum. The layer uses it for out_proj (+ x) and
 * ffn_out (+ h1); the LayerNorm after it then reads one tensor instead of
 * two and writes none back. No counterpart entry in the reference, whose
 * linear_bias (csrc/linear_gelu.cuh:598-719) the other arguments follow.
 * fp32 out only; residual 16-byte aligned. Declines (DOTL_DECLINED) where
 * the pipelined kernel does not run (fp32 x, K % 64 != 0): the caller adds
 * the residual itself.
 */
int dotl_linear_residual(const void* x, int x_dtype, const void* w_hi, const void* w_lo,
                         const float* bias, const float* residual, float* out, int64_t M,
                         int64_t N, int64_t K, int act, int math, int tile, void* stream);

/*
 * dotl_linear on split fp16 planes (x_dtype DOTL_F16X2) whose lo plane does
 * not directly follow the hi plane: x_hi and x_lo each fp16 [M, K]
 * (contiguous, 16-byte aligned), e.g. a block of rows of a [2][rows][K]
 * LayerNorm output; no activation; math DOTL_MATH_FP16X2 or
 * DOTL_MATH_FP16X3. Otherwise as dotl_linear (reference linear_bias,
 * csrc/linear_gelu.cuh:598-719, whose input here is the split form). No
 * counterpart entry in the reference: the layer projects one causal
 * prefix's rows this way, in place, into the QKV output.
 */
int dotl_linear_planes(const void* x_hi, const void* x_lo, const void* w_hi, const void* w_lo,
                       const float* bias, void* out, int out_dtype, int64_t M, int64_t N,
                       int64_t K, int math, int tile, void* stream);

/*
 * h = residual + x @ W^T + bias (fp32 [M, N]) and normed = LayerNorm(h) *
 * ln_weight + ln_bias in one kernel: linear_bias followed by the reference's
 * fused_add_layernorm (csrc/linear_gelu.cuh:598-719, then
 * csrc/add_layernorm.cuh:491-692: x_new = x + sub, normed with the biased
 * variance and fp32 statistics), for rows of up to 256 columns, which one
 * workgroup's tile spans. The LayerNorm is the LayerNorm kernels' own
 * arithmetic, so both outputs equal dotl_linear_residual + dotl_layernorm
 * bit for bit. No counterpart entry in the reference.
 *   x            fp16 [M, K], K a positive multiple of 64 (one fp16 pass)
 *   w_hi         fp16 [N, K] (dotl_weight_split); bias fp32 [N]
 *   residual     optional (NULL) fp32 [M, N]
 *   out          optional (NULL: h is not stored) fp32 [M, N]
 *   normed       [normed_rows, N] in normed_dtype: DOTL_F32, DOTL_F16 (RNE)
 *                or DOTL_F16X2 (split planes [2][normed_rows][N]); row r of
 *                h goes to row out_row[r] (fp32 only) or, with out_row NULL,
 *                to row r (normed_rows == M). Rows out_row does not name are
 *                left untouched.
 *   io           optional (NULL) graph I/O slot: normed is read from io[1]
 *                when the kernel runs (see dotl_bind_io)
 *   tile         -1 or 18 (128x256, the one tile built with this epilogue)
 * Declines (DOTL_DECLINED) for other operand types and for N > 256 or
 * N % 4 != 0: the caller runs dotl_linear_residual and dotl_layernorm.
 * Every tensor 16-byte aligned.
 */
int dotl_linear_layernorm(const void* x, int x_dtype, const void* w_hi, const float* bias,
                          const float* residual, float* out, const float* ln_weight,
                          const float* ln_bias, double eps, void* normed, int normed_dtype,
                          const int32_t* out_row, int64_t normed_rows, const int64_t* io,
                          int64_t M, int64_t N, int64_t K, int tile, void* stream);

/*
 * The position-wise FFN with the residual add and the row LayerNorm in one
 * kernel, for d_model 256:
 *   h = GELU(x W1^T + b1) in fp16, y = residual + h W2^T + b2,
 *   normed = LayerNorm(y) * ln_weight + ln_bias.
 * Replaces linear_gelu, then linear_bias and fused_add_layernorm
 * (csrc/linear_gelu.cuh:598-756, csrc/add_layernorm.cuh:491-692, as
 * optimized/layers.py chains them); equals dotl_linear (GELU, fp16 out)
 * followed by dotl_linear_layernorm bit for bit, without writing h to
 * memory. No counterpart entry in the reference.
 *   x            fp16 [M, D], D == 256
 *   w1_hi        fp16 [F, D], w2_hi fp16 [D, F] (dotl_weight_split);
 *                F a positive multiple of 64 up to 2048
 *   b1           fp32 [F]; b2 fp32 [D]
 *   residual     optional (NULL) fp32 [M, D]
 *   out          optional (NULL: y is not stored) fp32 [M, D]
 *   normed, normed_dtype, out_row, normed_rows, io: as dotl_linear_layernorm
 *   zero_padded  with out_row (strictly increasing): the rows of normed that
 *                out_row does not name are written with zeros too (what
 *                dotl_zero_rows would do after it); 0 leaves them untouched
 * Declines (DOTL_DECLINED) for other shapes and operand types: the caller
 * runs the two GEMMs. Every tensor 16-byte aligned.
 */
int dotl_ffn_layernorm(const void* x, int x_dtype, const void* w1_hi, const float* b1,
                       const void* w2_hi, const float* b2, const float* residual, float* out,
                       const float* ln_weight, const float* ln_bias, double eps, void* normed,
                       int normed_dtype, const int32_t* out_row, int64_t normed_rows,
                       int zero_padded, const int64_t* io, int64_t M, int64_t D, int64_t F,
                       void* stream);

/*
 * Zero row r of out (fp32 [rows, width]) wherever row_map[r] < 0: the padded
 * rows of a padded batch's output, whose valid rows dotl_linear_layernorm
 * scattered there (row_map is the padded -> packed map, -1 for padding; the
 * reference zeroes them with masked_fill, optimized/model.py:141-142). With
 * io, out is read from io[1] when the kernel runs (a graph I/O slot).
 */
int dotl_zero_rows(float* out, const int32_t* row_map, int64_t rows, int64_t width,
                   const int64_t* io, void* stream);

/*
 * Fused scaled-dot-product attention, flash style on MFMA.
 * Replaces fused_attention_forward
 * (reference csrc/attention_dispatch.cuh:332-519).
 *
 *   q, k, v      logical [B, H, S, head_dim], dtype DOTL_F16, DOTL_BF16 or
 *                DOTL_F32 (narrowed with RNE when staged), head_dim stride
 *                1, and the (batch, head, seq) strides given once in
 *                qkv_strides[3] (in elements) for all three -- the strided
 *                views of a fused [B, S, 3, H, hd] projection pass through
 *                without copies.
 *   mask         optional (NULL) bool bytes, true = may attend, addressed as
 *                mask[b*ms[0] + h*ms[1] + i*ms[2] + j*ms[3]] (expanded
 *                [B,H,S,S] strides; stride 0 on broadcast dims)
 *   out          out_layout 0: [B, H, S, head_dim]; 1: [B, S, H*head_dim];
 *                dtype out_dtype (DOTL_F16 or DOTL_F32; DOTL_BF16 exactly
 *                when q/k/v are bf16)
 *   is_causal    key j > query i is excluded (combinable with mask)
 *   impl         0 auto, 1 scalar, 2 wmma (here: the MFMA kernel), 3 tile
 *   precision    0 auto, 1 fp32, 2 tf32, 3 fp16, 4 bf16 (bf16 tensors
 *                contract in bf16 on the MFMA kernel)
 *   cu_seqlens   optional (NULL) int32 [B + 1], non-decreasing, cu[0] = 0:
 *                packed sequences. Sequence b is rows [cu[b], cu[b+1]) of
 *                q/k/v (row stride qkv_strides[2], head stride
 *                qkv_strides[1]; qkv_strides[0] unused) and of out, which is
 *                then [rows, H*head_dim] (out_layout must be 1, mask NULL).
 *                Contract: S >= every sequence's length (the grid is sized
 *                from S; rows of a longer sequence past S are not written),
 *                and rows == cu[B]. This is the padded batch with its
 *                padding removed: no reference counterpart of its own (the
 *                reference masks padded keys,
 *                reference csrc/attention_dispatch.cuh:404-450).
 *   rows         with cu_seqlens, the packed row count cu[B] (q's first
 *                dimension); ignored otherwise
 *   splits       key-range splits (split-KV, the LDS-DMA kernel for fp16
 *                q/k/v only; other kernels ignore it): 0 the library's
 *                choice (dotl_wmma_set_split_count / dotl_wmma_set_split_kv,
 *                else from occupancy), 1 none, n > 1 that many (at most one
 *                per 64-key tile). Replaces the reference's split-KV path
 *                (reference csrc/attention_wmma.cuh:706-759, 1783-1826).
 *   workspace    device memory for the split partials, workspace_bytes long
 *                (16-byte aligned): dotl_attention_split_plan says how many
 *                bytes. Too small (or NULL) with splits = 0: the call runs
 *                unsplit; with splits > 1: DOTL_E_INVALID.
 *   A query row with no allowed key produces 0.
 *   Returns DOTL_DECLINED when no kernel covers (dtype, head_dim); the caller
 *   raises, as the reference does.
 */
int dotl_attention_forward(const void* q, const void* k, const void* v, int dtype,
                           const int64_t* qkv_strides, const uint8_t* mask,
                           const int64_t* mask_strides, void* out, int out_dtype,
                           int out_layout, int B, int H, int S, int head_dim,
                           int is_causal, double scale, int impl, int precision,
                           const int32_t* cu_seqlens, int64_t rows, int splits,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * dotl_attention_forward that allocates nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under
 * hipGraph stream capture, serving loops or harnesses that forbid hipMalloc).
 * Same arguments and results as dotl_attention_forward minus the workspace:
 * the split-KV partials live in a fixed array of this library, one per GPU,
 * of dotl_attention_noalloc_scratch_bytes() bytes (32 MiB), held until the
 * process ends; its address is resolved on the first call on each device
 * (make that first call outside stream capture). splits = 0 runs the largest
 * split count up to the library's choice that fits the array; an explicit
 * splits > 1 that does not fit returns DOTL_E_INVALID. Nothing in the array
 * needs to start at zero (every partial the combine reads is written first
 * by the same call). Calls that overlap on one GPU (concurrent streams)
 * race on the array: serialise them.
 */
int dotl_attention_forward_noalloc(const void* q, const void* k, const void* v, int dtype,
                                   const int64_t* qkv_strides, const uint8_t* mask,
                                   const int64_t* mask_strides, void* out, int out_dtype,
                                   int out_layout, int B, int H, int S, int head_dim,
                                   int is_causal, double scale, int impl, int precision,
                                   const int32_t* cu_seqlens, int64_t rows, int splits,
                                   void* stream);

/* Bytes of the per-GPU scratch array dotl_attention_forward_noalloc uses. */
int64_t dotl_attention_noalloc_scratch_bytes(void);

/*
 * The split count dotl_attention_forward would resolve `splits` (0, 1 or n)
 * to for these arguments, and the workspace bytes it then needs (0 when it
 * would not split). rows: B * S, or the packed row count. No device access.
 * The counterpart of the reference's wmma_split_count
 * (reference csrc/fused_attention.cu, csrc/attention_wmma.cuh:706-759).
 */
int dotl_attention_split_plan(int B, int H, int S, int head_dim, int is_causal, int dtype,
                              int has_mask, int64_t rows, int impl, int precision, int splits,
                              int* splits_out, int64_t* workspace_bytes_out);

/*
 * Fused post-attention block. Replaces fused_ffn_block (reference
 * csrc/ffn_block.cuh:270-311):
 *   x1 = x + attn_out;            n1 = LayerNorm(x1; norm1_w, norm1_b)
 *   h  = GELU(n1 W_in^T + b_in);  x_out = x1 + h W_out^T + b_out
 *   normed_out = LayerNorm(x_out; norm2_w, norm2_b)
 * x, attn_out, x_out, normed_out fp32 [rows, D]; W_in [F, D] and W_out
 * [D, F] given as fp16 (the fp16-operand GEMMs' narrowing of the fp32
 * weights, RNE); biases and LayerNorm parameters fp32. The arithmetic is the
 * unfused chain's (fp16 operands, fp32 accumulation, h rounded to fp16), so
 * the outputs equal that chain's bit for bit.
 * Covers D up to 128 and F up to 512, multiples of 8 (the reference
 * instantiates D == F in {16, 32, 48, 64, 128}; F up to 512 adds the 4x FFN
 * of d_model 128); other widths return DOTL_DECLINED and the caller runs the
 * unfused chain, as the reference's empty-list decline.
 * Tensors 16-byte aligned.
 */
int dotl_ffn_block(const float* x, const float* attn_out, const float* norm1_w,
                   const float* norm1_b, const void* ffn_in_w_half, const float* ffn_in_b,
                   const void* ffn_out_w_half, const float* ffn_out_b, const float* norm2_w,
                   const float* norm2_b, float* x_out, float* normed_out, int64_t rows,
                   int64_t D, int64_t F, double eps, void* stream);

/* Writes where each lane's 16 bytes of one global_load_lds_dwordx4 land in
 * LDS: src is 256 int32 (64 lanes x 4), out 512 int32 (a zeroed 2 KiB LDS
 * region after the load, read back). Expected: lane l at bytes [16 l, 16 l + 16).
 * A test, not a start-up step. */
int dotl_lds_dma_probe(const int32_t* src, int32_t* out, void* stream);

/* Process-wide knobs with the reference's names
 * (reference csrc/fused_attention.cu:234-339). wmma_set_fp16 selects the
 * arithmetic "auto" attention precision resolves to: fp16 (1) or the split
 * fp16x3 path (0). cp_async selects how fp16 K/V tiles reach LDS, as the
 * reference's cp.async staging knob does: 0 register-staged (load to VGPRs,
 * then write LDS), 1 or 2 (default) asynchronous LDS-DMA through a
 * multi-stage pipeline. */
void dotl_wmma_set_fp16(int on);
int dotl_wmma_fp16(void);
void dotl_wmma_set_cp_async(int mode);
int dotl_wmma_cp_async_mode(void);
/* Split-KV knobs (reference wmma_set_split_kv / wmma_set_split_count): on
 * (default) lets splits = 0 split from occupancy; a count n > 0 forces n
 * splits for splits = 0 calls, 0 restores the occupancy choice. */
void dotl_wmma_set_split_kv(int on);
int dotl_wmma_split_kv_enabled(void);
void dotl_wmma_set_split_count(int n);

/* Measurement knob of the LDS-DMA attention kernel, no reference
 * counterpart: force its wavefronts per workgroup (1, 2, 4 or 8; 0 = by
 * sequence length and head_dim) and pipeline stages (1 to 4; 0 = by
 * head_dim, length and waves).
 * Process-wide, like the knobs above. */
void dotl_attention_set_pipeline(int waves, int stages);

#ifdef __cplusplus
}
#endif

#endif /* DOTL_H */
