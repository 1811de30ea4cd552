// The position-wise feed-forward block with the residual add and the row
// LayerNorm, for d_model 256, in one kernel:
//   h      = GELU(x W1^T + b1)            (fp16, held in LDS a step at a time)
//   y      = r + h W2^T + b2              (fp32, stored when C is given)
//   normed = LayerNorm(y) * ln_w + ln_b   (at row out_row[m], or m)
// Replaces linear_gelu followed by linear_bias and the add+LayerNorm
// (reference csrc/linear_gelu.cuh:598-756, csrc/add_layernorm.cuh:491-692,
// as optimized/layers.py chains them), and equals this library's chain of
// the two GEMMs (dotl_linear with GELU and an fp16 output, then
// dotl_linear_layernorm) bit for bit: both products run the same 32x32x16
// MFMAs over the same operands in the same k order, the GELU and its fp16
// rounding are the same functions, and the epilogue is the GEMM's own.
//
// MI355X design: d_ff is streamed in steps of 64. A workgroup (8 waves)
// owns 128 rows; each step it forms its rows' 128 x 64 block of h from x
// (held in registers as MFMA fragments for the whole launch: 32 rows a
// wave) and a 64-row slice of W1, puts the GELU'd fp16 block in LDS, and
// multiplies it into the 128 x 256 fp32 accumulators with W2's matching
// 64-column slice. Both weight slices (64 KiB a step) arrive by LDS-DMA,
// double-buffered; the 1 MiB of fp16 weights stays in each XCD's L2, so
// HBM sees x, the residual and the output once -- the unfused chain also
// writes and re-reads h, 2 x 2 x d_ff bytes a row (C5: 349 MB).
#include "gemm_dma_impl.h"

namespace dotl {
namespace gemm_dma {
namespace {

constexpr int kD = 256;      // d_model: one LayerNorm row a wave instruction
constexpr int kBM = 128;     // rows a workgroup
constexpr int kFC = 64;      // d_ff columns a step (the second product's K tile)
constexpr int kWaves = 8;
constexpr int kMaxF = 2048;  // b1 is staged whole in LDS
// A stage: W2's 64-column slice (kD rows of 64 halves), then W1's 64-row
// slice as four 64-wide k blocks (4 x 64 rows of 64 halves). Rows are 128
// bytes with the GEMM's chunk swizzle.
constexpr int kW1Row = kD;
constexpr int kStage = (kD + 4 * kFC) * 64;   // halves: 64 KiB

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

template <int LN>
__global__ __launch_bounds__(kWaves * 64) void ffn_ln_kernel(
    const _Float16* __restrict__ X, const _Float16* __restrict__ W1,
    const float* __restrict__ b1, const _Float16* __restrict__ W2,
    const float* __restrict__ b2, const float* __restrict__ R, void* __restrict__ C, int64_t M,
    int64_t F, LnEpi ln, int zero_padded) {
    // The second product is the 128x256 tile of the GEMM (8 waves, 2 x 4,
    // each a 64 x 64 block): its fragment reader, MFMA and accumulators.
    using G = DmaGemm<kBM, kD, 64, 2, 0, DOTL_ACT_NONE, DOTL_F32, kWaves>;
    using L = typename G::L;
    __shared__ __attribute__((aligned(1024))) _Float16 st0[kStage];
    __shared__ __attribute__((aligned(1024))) _Float16 st1[kStage];
    __shared__ __attribute__((aligned(1024))) _Float16 hbuf[kBM * kFC];
    __shared__ __attribute__((aligned(16))) float sbias[kD];
    __shared__ __attribute__((aligned(16))) float sb1[kMaxF];

    G g;
    g.M = M;
    g.N = kD;
    g.K = F;
    g.lane = threadIdx.x & 63;
    g.wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    g.wm = g.wave / G::WGN;
    g.wn = g.wave % G::WGN;
    g.lr = g.lane & 31;
    g.lg = g.lane >> 5;
    g.m0 = static_cast<int64_t>(blockIdx.x) * kBM;
    g.n0 = 0;
    g.nk = F / kFC;
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j) g.acc[i][j] = floatx16{};

    for (int c = threadIdx.x; c < kD; c += kWaves * 64) sbias[c] = b2[c];
    for (int c = threadIdx.x; c < F; c += kWaves * 64) sb1[c] = b1[c];

    // The first product: wave w forms h rows 32 (w / 2) .. + 32, columns
    // 32 (w % 2) .. + 32 of the step's 64, from x fragments loaded once
    // (row clamped to the last valid one: rows past M are never stored).
    const int hr = g.wave >> 1, hc = g.wave & 1;
    half8 xf[kD / 16];
    {
        int64_t xrow = g.m0 + 32 * hr + g.lr;
        xrow = xrow < M ? xrow : M - 1;
        const _Float16* xp = X + xrow * kD + 8 * g.lg;
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) xf[s] = *reinterpret_cast<const half8*>(xp + 16 * s);
    }

    // This wave's four DMA instructions per slice: stage rows rd * 64 +
    // wave * 8 + lane / 8 (W2 row n; W1 k block rd, d_ff row wave * 8 +
    // lane / 8), physical chunk lane % 8 holding logical chunk pc ^ swz.
    unsigned off2[4], off1[4];
    {
        const int sub = g.lane >> 3, pc = g.lane & 7;
#pragma unroll
        for (int rd = 0; rd < 4; ++rd) {
            const int r = rd * 64 + g.wave * 8 + sub;
            const int lc = pc ^ L::swz(r);
            off2[rd] = static_cast<unsigned>((r * F + lc * 8) * 2);
            off1[rd] = static_cast<unsigned>(((g.wave * 8 + sub) * kD + rd * 64 + lc * 8) * 2);
        }
    }
    auto issue = [&](_Float16* stage, int64_t c) {
#pragma unroll
        for (int rd = 0; rd < 4; ++rd)
            dma16_off(W2 + c * kFC, off2[rd], stage + (rd * 64 + g.wave * 8) * 64);
#pragma unroll
        for (int rd = 0; rd < 4; ++rd)
            dma16_off(W1 + c * kFC * kD, off1[rd], stage + (kW1Row + rd * 64 + g.wave * 8) * 64);
    };

    // zero_padded: the rows of the (fp32) normed output that out_row skips
    // -- those after each of this workgroup's rows up to the next named one,
    // and, in workgroup 0, those before the first -- written with zeros, one
    // 1 KiB row a wave instruction, during the first step: the stores then
    // drain under its products (the next step's wait covers them), where at
    // the end of the launch they measured as slow as a separate pass. The
    // rows are disjoint from every named row. Lane u holds out_row of this
    // wave's u-th row (u <= 16; loaded before the first DMA, so its wait
    // does not take the DMAs with it).
    const bool zeroing = zero_padded && ln.out_row != nullptr;
    constexpr int kRowsPerWave = kBM / kWaves;
    const int64_t zlo = g.m0 + kRowsPerWave * g.wave;
    int zr = 0;
    if (zeroing && g.lane <= kRowsPerWave) {
        const int64_t m = zlo + g.lane;
        zr = ln.out_row[m < M ? m : M - 1];
    }
    auto zero_padded_rows = [&]() {
        float* nout = static_cast<float*>(ln.io != nullptr ? reinterpret_cast<void*>(ln.io[1])
                                                           : ln.normed);
        const int64_t rows = ln.plane / kD;
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        auto zero = [&](int64_t lo, int64_t hi) {
            hi = hi < rows ? hi : rows;
            for (int64_t r = lo; r < hi; ++r)
                *reinterpret_cast<float4*>(nout + r * kD + 4 * g.lane) = z;
        };
        static_for<0, kRowsPerWave>([&](auto uu) {
            constexpr int u = decltype(uu)::value;
            const int64_t m = zlo + u;
            if (m < M) {
                const int64_t next = m + 1 < M ? __builtin_amdgcn_readlane(zr, u + 1) : rows;
                zero(static_cast<int64_t>(__builtin_amdgcn_readlane(zr, u)) + 1, next);
            }
        });
        if (blockIdx.x == 0 && g.wave == 0) zero(0, __builtin_amdgcn_readlane(zr, 0));
    };

    const int tr = 32 * hr + g.lr;   // this lane's h row (tile-local)
    auto step = [&](auto sc, int64_t c, auto zc) {
        constexpr int S = decltype(sc)::value;
        constexpr bool ZERO = decltype(zc)::value;   // the first step: zeroing too
        _Float16* cur = S == 0 ? st0 : st1;
        _Float16* nxt = S == 0 ? st1 : st0;
        // (a) every wave's slices of step c have landed, and every wave is
        // done with step c - 1 (h block and the other stage free)
        wait_vmcnt<0>();
        stage_barrier();
        if constexpr (ZERO) {
            if (zeroing) zero_padded_rows();
        }
        if (c + 1 < g.nk) issue(nxt, c + 1);
        // h block: 16 MFMAs over d_model, k in order (the GEMM's sequence)
        floatx16 h = floatx16{};
        static_for<0, kD / 16>([&](auto ss) {
            constexpr int s = decltype(ss)::value;
            const half8 b = g.frag(cur + (kW1Row + (s / 4) * 64) * 64, 32 * hc + g.lr, s % 4);
            h = G::mma(b, xf[s], h);
        });
        // bias, GELU, fp16: the GEMM epilogue's operations, into LDS in the
        // swizzled A-operand layout
        const float* bb = sb1 + c * kFC + 32 * hc + 4 * g.lg;
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            const float4 bv = *reinterpret_cast<const float4*>(bb + 8 * grp);
            const float bvs[4] = {bv.x, bv.y, bv.z, bv.w};
            half4_t o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float a = h[4 * grp + e];
                a += bvs[e];
                o[e] = static_cast<_Float16>(gelu_erf<false>(a));
            }
            *reinterpret_cast<half4_t*>(hbuf + tr * 64 + ((4 * hc + grp) ^ L::swz(tr)) * 8 +
                                        4 * g.lg) = o;
        }
        // (b) the h block is complete
        stage_barrier();
        static_for<0, kFC / 16>([&](auto kk) {
            constexpr int ks = decltype(kk)::value;
            half8 a[G::TM], b[G::TN];
#pragma unroll
            for (int i = 0; i < G::TM; ++i) a[i] = g.frag(hbuf, g.wm * G::WM + i * 32 + g.lr, ks);
#pragma unroll
            for (int j = 0; j < G::TN; ++j) b[j] = g.frag(cur, g.wn * G::WN + j * 32 + g.lr, ks);
#pragma unroll
            for (int i = 0; i < G::TM; ++i)
#pragma unroll
                for (int j = 0; j < G::TN; ++j) g.acc[i][j] = G::mma(b[j], a[i], g.acc[i][j]);
        });
    };

    // The first step is peeled off the loop: the zeroing's values are dead
    // before the loop (left live across it they cost 14 VGPRs and ~8 us at
    // C5 even with zeroing off).
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    issue(st0, 0);
    step(I0{}, 0, std::true_type{});
    int64_t c = 1;
    for (; c + 2 <= g.nk; c += 2) {
        step(I1{}, c, std::false_type{});
        step(I0{}, c + 1, std::false_type{});
    }
    if (c < g.nk) step(I1{}, c, std::false_type{});

    auto stage_rt = [&](int b) -> _Float16* { return b == 0 ? st0 : st1; };
    store_tile<kBM, kD, 2, DOTL_ACT_NONE, DOTL_F32, kWaves, LN, kStage>(g, stage_rt, sbias, R, C,
                                                                        M, kD, ln);
}

template <int LN>
void launch(const _Float16* X, const _Float16* W1, const float* b1, const _Float16* W2,
            const float* b2, const float* R, void* C, int64_t M, int64_t F, const LnEpi& ln,
            int zero_padded, hipStream_t stream) {
    hipLaunchKernelGGL((ffn_ln_kernel<LN>), dim3(static_cast<unsigned>((M + kBM - 1) / kBM)),
                       dim3(kWaves * 64), 0, stream, X, W1, b1, W2, b2, R, C, M, F, ln,
                       zero_padded);
}

}  // namespace
}  // namespace gemm_dma
}  // namespace dotl

extern "C" int dotl_ffn_layernorm(const void* x, int x_dtype, const void* w1_hi, const float* b1,
                                  const void* w2_hi, const float* b2, const float* residual,
                                  float* out, const float* ln_weight, const float* ln_bias,
                                  double eps, void* normed, int normed_dtype,
                                  const int32_t* out_row, int64_t normed_rows,
                                  int zero_padded, const int64_t* io, int64_t M, int64_t D,
                                  int64_t F, void* stream) {
    using namespace dotl;
    using namespace dotl::gemm_dma;
    clear_error();
    const char* who = "ffn_layernorm";
    DOTL_REQUIRE(M >= 0 && D >= 0 && F >= 0 && normed_rows >= 0, "%s: negative extent", who);
    DOTL_REQUIRE(normed_dtype == DOTL_F32 || normed_dtype == DOTL_F16 ||
                     normed_dtype == DOTL_F16X2,
                 "%s: the normed output is float32, float16 or split float16", who);
    DOTL_REQUIRE(out_row != nullptr || normed_rows == M,
                 "%s: without out_row the normed output has the input's %lld rows", who,
                 static_cast<long long>(M));
    DOTL_REQUIRE(out_row == nullptr || normed_dtype == DOTL_F32,
                 "%s: scattered rows (out_row) take a float32 normed output", who);
    DOTL_REQUIRE(zero_padded == 0 || out_row != nullptr,
                 "%s: zero_padded applies to scattered rows (out_row)", who);
    if (x_dtype != DOTL_F16 || D != kD || F % kFC != 0 || F == 0 || F > kMaxF ||
        M * D * 2 >= (int64_t{1} << 32)) {
        set_error(std::string(who) + ": served for a float16 x, d_model 256 and d_ff a positive "
                  "multiple of 64 up to 2048; run the two GEMMs");
        return DOTL_DECLINED;
    }
    if (M == 0) return DOTL_OK;
    DOTL_REQUIRE(x && w1_hi && b1 && w2_hi && b2 && ln_weight && ln_bias && (normed || io),
                 "%s: null pointer", who);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w1_hi) |
                            reinterpret_cast<uintptr_t>(w2_hi) |
                            reinterpret_cast<uintptr_t>(residual) |
                            reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(ln_weight) |
                            reinterpret_cast<uintptr_t>(ln_bias) |
                            reinterpret_cast<uintptr_t>(normed);
    DOTL_REQUIRE(align % 16 == 0, "%s: every tensor must be 16-byte aligned", who);
    const LnEpi ln{ln_weight, ln_bias, static_cast<float>(eps), normed, normed_rows * D, out_row,
                   io};
    const auto* xh = static_cast<const _Float16*>(x);
    const auto* w1 = static_cast<const _Float16*>(w1_hi);
    const auto* w2 = static_cast<const _Float16*>(w2_hi);
    const hipStream_t s = as_stream(stream);
    const bool wc = out != nullptr;
    switch (normed_dtype) {
        case DOTL_F32:
            wc ? launch<DOTL_F32 + 4>(xh, w1, b1, w2, b2, residual, out, M, F, ln, zero_padded, s)
               : launch<DOTL_F32>(xh, w1, b1, w2, b2, residual, out, M, F, ln, zero_padded, s);
            break;
        case DOTL_F16:
            wc ? launch<DOTL_F16 + 4>(xh, w1, b1, w2, b2, residual, out, M, F, ln, zero_padded, s)
               : launch<DOTL_F16>(xh, w1, b1, w2, b2, residual, out, M, F, ln, zero_padded, s);
            break;
        default:
            wc ? launch<DOTL_F16X2 + 4>(xh, w1, b1, w2, b2, residual, out, M, F, ln, zero_padded, s)
               : launch<DOTL_F16X2>(xh, w1, b1, w2, b2, residual, out, M, F, ln, zero_padded, s);
            break;
    }
    return check_launch(who);
}
