// Fused post-attention block for narrow layers (reference csrc/ffn_block.cuh,
// fused_ffn_block :270-311):
//
//   x1 = x + attn_out              n1 = LayerNorm(x1; norm1)
//   h  = GELU(n1 W_in^T + b_in)    y  = h W_out^T + b_out
//   x2 = x1 + y                    n2 = LayerNorm(x2; norm2)      -> (x2, n2)
//
// for d_model up to 128 and d_ff up to 512 (multiples of 8; the reference's
// fused block stops at 128 for both, this one also covers a 4x FFN on
// d_model 128, the C1 layer, whose unfused chain is four launch-bound
// kernels). x1, n1, h and y never reach HBM: per row the block reads x and
// attn_out and writes x2 and n2. LDS at d_model 128, d_ff 512: x1 34 KiB,
// n1 17, h 67, parameters 5.
//
// The arithmetic is the unfused chain's, operation for operation, so fusing
// is a pure speed choice with the same bits: the LayerNorms follow the
// layernorm.hip vector kernel's summation order, the GEMMs are the fp16
// operand v_mfma_f32_32x32x16_f16 chains over K in increasing order with the
// bias added to the accumulator, GELU is gelu_erf and h is rounded to fp16 as
// linear_gelu stores it for ffn_out.
//
// MI355X layout: one workgroup of 4 waves (8 for d_ff above 128) per 64
// rows. A LayerNorm row of D <= 128 floats is 32 float4 chunks, so a wave
// normalises two rows per step (one per 32-lane half) and all its row
// pairs' reductions run in lockstep. The GEMMs are 32x32 tiles issued as W x A^T (each accumulator a
// C^T tile: a lane owns 4 consecutive columns of one row), A from LDS, the
// fp16 weights (<= 32 KiB each) straight from L2.
#include "dotl_common.h"

namespace dotl {

namespace {

constexpr int kRows = 64;     // rows per workgroup

struct FfnArgs {
    const float* x;
    const float* attn;
    const float* w1;
    const float* b1;
    const _Float16* win;   // [F, D]
    const float* bin;
    const _Float16* wout;  // [D, F]
    const float* bout;
    const float* w2;
    const float* b2;
    float* x_out;
    float* n_out;
    int64_t rows;
    int D, F;
    float eps;
};

// Mean and 1/std of NB row pairs (lane half = pair member, lane % 32 = float4
// chunk, zeros past the row), reduced over 32-lane butterflies in lockstep.
// The layernorm.hip vector kernel's operation order: its 64-lane butterfly
// adds an upper half of zeros first, which changes no value.
template <int NB>
__device__ __forceinline__ void ln_pairs(const float4 (&v)[NB], float eps, float inv_d,
                                         float (&mean_est)[NB], float (&delta)[NB],
                                         float (&rstd)[NB], bool (&has)[NB]) {
    float s[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) s[i] = (v[i].x + v[i].y) + (v[i].z + v[i].w);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1)
#pragma unroll
        for (int i = 0; i < NB; ++i) s[i] += __shfl_xor(s[i], off, kWave);
    float sd[NB], sd2[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        mean_est[i] = s[i] * inv_d;
        sd[i] = 0.f;
        sd2[i] = 0.f;
        if (has[i]) {
            const float d0 = v[i].x - mean_est[i], d1 = v[i].y - mean_est[i];
            const float d2 = v[i].z - mean_est[i], d3 = v[i].w - mean_est[i];
            sd[i] = (d0 + d1) + (d2 + d3);
            sd2[i] = ln_sq4(d0, d1, d2, d3);
        }
    }
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1)
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            sd[i] += __shfl_xor(sd[i], off, kWave);
            sd2[i] += __shfl_xor(sd2[i], off, kWave);
        }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        delta[i] = sd[i] * inv_d;
        rstd[i] = 1.0f / sqrtf(ln_var(sd2[i], delta[i], inv_d) + eps);
    }
}

__device__ __forceinline__ float4 ln_apply(float4 v, float m, float dl, float r, float4 w,
                                           float4 b) {
    return make_float4(ln_out(v.x, m, dl, r, w.x, b.x), ln_out(v.y, m, dl, r, w.y, b.y),
                       ln_out(v.z, m, dl, r, w.z, b.z), ln_out(v.w, m, dl, r, w.w, b.w));
}

// The W fragments of one 32x32 output tile's column block nt: W [N][K] fp16
// in global memory (rows >= N and k >= K read as zero), 16-deep k steps.
template <int KS>
__device__ __forceinline__ void load_wtile(half8 (&wf)[KS], const _Float16* w, int n_rows,
                                           int k_len, int nt, int lane) {
    const int lr = lane & 31, lg = lane >> 5;
    // unconditional loads from clamped indices (a branch per fragment made
    // the compiler wait on each load in turn); mma_wtile zeroes the
    // out-of-range ones where it uses them, so nothing here waits
    const int n = nt * 32 + lr;
    const int nc = n < n_rows ? n : n_rows - 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int k = ks * 16 + lg * 8;
        const int kc = k < k_len ? k : k_len - 8;
        wf[ks] = *reinterpret_cast<const half8*>(w + static_cast<int64_t>(nc) * k_len + kc);
    }
}

// A W^T for one 32x32 tile from fragments already loaded: A [64][KS*16] fp16
// in LDS (pitch PA), row block mt. K in increasing order, one accumulator
// chain (the unfused GEMM's order). Lane l holds row l % 32 of the tile and
// columns 8 g + 4 (l / 32) + e in register 4 g + e.
// W rows >= n_rows and k >= k_len count as zero (the fragments hold clamped
// loads there).
template <int KS>
__device__ __forceinline__ floatx16 mma_wtile(const half8 (&wf)[KS], const _Float16* a_lds,
                                              int pa, int mt, int nt, int n_rows, int k_len,
                                              int lane) {
    const int lr = lane & 31, lg = lane >> 5;
    const bool n_ok = nt * 32 + lr < n_rows;
    floatx16 acc{};
    const _Float16* arow = a_lds + (mt * 32 + lr) * pa + lg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const half8 af = *reinterpret_cast<const half8*>(arow + ks * 16);
        const half8 b = (n_ok && ks * 16 + lg * 8 < k_len) ? wf[ks] : half8{};
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, af, acc, 0, 0, 0);
    }
    return acc;
}

// NW waves a workgroup (4, or 8 for d_ff above 128). Each wave's weight
// fragments are loaded before they are needed, all of a GEMM's at once: the
// ffn_in ones at kernel start, under the first LayerNorm, the ffn_out ones
// as soon as the ffn_in MFMAs are issued. The MFMA work per tile is a few
// hundred cycles and an L2 round trip a few thousand; loaded tile by tile
// (as a wave walked its tiles), a 128 x 512 block took ~40 us for 128 rows.
template <int DP, int FP, int NW>
__global__ __launch_bounds__(NW * 64) void ffn_block_kernel(FfnArgs a) {
    constexpr int PX = DP + 4;    // fp32 row pitch (floats)
    constexpr int PN = DP + 8;    // fp16 pitches (halves)
    constexpr int PH = FP + 8;
    constexpr int NP = kRows / (2 * NW);            // row pairs per wave
    constexpr int T1 = 2 * (FP / 32);               // ffn_in tiles
    constexpr int T2 = 2 * (DP / 32);               // ffn_out tiles
    constexpr int TW1 = (T1 + NW - 1) / NW;         // per wave
    constexpr int TW2 = (T2 + NW - 1) / NW;
    constexpr int KS1 = DP / 16, KS2 = FP / 16;
    __shared__ __attribute__((aligned(16))) float sX[kRows * PX];       // x1, then x2
    __shared__ __attribute__((aligned(16))) _Float16 sN[kRows * PN];    // n1
    __shared__ __attribute__((aligned(16))) _Float16 sH[kRows * PH];    // h
    __shared__ __attribute__((aligned(16))) float sP[6 * DP + FP];      // LN params, biases
    float* p_w1 = sP;
    float* p_b1 = sP + DP;
    float* p_w2 = sP + 2 * DP;
    float* p_b2 = sP + 3 * DP;
    float* p_bout = sP + 4 * DP;
    float* p_bin = sP + 5 * DP;

    const int D = a.D, F = a.F;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hf = lane >> 5, lh = lane & 31;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRows;
    const float inv_d = 1.0f / static_cast<float>(D);
    const bool lane_in_row = 4 * lh < D;   // D is a multiple of 8

    // This wave's ffn_in weight fragments, in flight from the start.
    half8 wf1[TW1][KS1];
#pragma unroll
    for (int i = 0; i < TW1; ++i) {
        const int t = wave + i * NW;
        if (t < T1) load_wtile<KS1>(wf1[i], a.win, F, D, t >> 1, lane);
    }

    // Row pair i of this wave: local rows wave * 2 NP + 2 i + hf.
    auto local_row = [&](int i) { return wave * (2 * NP) + 2 * i + hf; };

    // ---- x1 = x + attn_out; n1 = LN(x1) ------------------------------------------
    // The row loads are unconditional, from addresses clamped into the
    // tensors (rows >= 1 here), and the unused values zeroed after: behind a
    // per-row branch the compiler issued them one row pair at a time, each
    // waited out before the next was sent.
    float4 v[NP];
    bool has[NP];
    float4 xv[NP], av[NP];
    const int col4 = 4 * (lane_in_row ? lh : 0);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int64_t row = row0 + local_row(i);
        has[i] = lane_in_row && row < a.rows;
        const int64_t rc = row < a.rows ? row : a.rows - 1;
        xv[i] = *reinterpret_cast<const float4*>(a.x + rc * D + col4);
        av[i] = *reinterpret_cast<const float4*>(a.attn + rc * D + col4);
    }
    // Parameters to LDS, loads unconditional (clamped index) for the same reason.
    for (int i = threadIdx.x; i < DP; i += NW * 64) {
        const bool ok = i < D;
        const int ic = ok ? i : 0;
        const float w1 = a.w1[ic], b1 = a.b1[ic], w2 = a.w2[ic], b2 = a.b2[ic], bo = a.bout[ic];
        p_w1[i] = ok ? w1 : 0.f;
        p_b1[i] = ok ? b1 : 0.f;
        p_w2[i] = ok ? w2 : 0.f;
        p_b2[i] = ok ? b2 : 0.f;
        p_bout[i] = ok ? bo : 0.f;
    }
    for (int i = threadIdx.x; i < FP; i += NW * 64) {
        const float bi = a.bin[i < F ? i : 0];
        p_bin[i] = i < F ? bi : 0.f;
    }

#pragma unroll
    for (int i = 0; i < NP; ++i) {
        v[i] = make_float4(xv[i].x + av[i].x, xv[i].y + av[i].y, xv[i].z + av[i].z,
                           xv[i].w + av[i].w);
        if (!has[i]) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();   // parameters staged
    {
        float m[NP], dl[NP], r[NP];
        ln_pairs<NP>(v, a.eps, inv_d, m, dl, r, has);
        const float4 ww = *reinterpret_cast<const float4*>(p_w1 + 4 * (lh % (DP / 4)));
        const float4 bb = *reinterpret_cast<const float4*>(p_b1 + 4 * (lh % (DP / 4)));
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int lr = local_row(i);
            if (4 * lh < DP) {
                half4 hv = half4{};
                if (has[i]) {
                    const float4 o = ln_apply(v[i], m[i], dl[i], r[i], ww, bb);
                    hv[0] = to_half(o.x); hv[1] = to_half(o.y);
                    hv[2] = to_half(o.z); hv[3] = to_half(o.w);
                }
                *reinterpret_cast<half4*>(sN + lr * PN + 4 * lh) = hv;
                *reinterpret_cast<float4*>(sX + lr * PX + 4 * lh) = v[i];
            }
        }
    }
    __syncthreads();

    // ---- h = GELU(n1 W_in^T + b_in), fp16 -----------------------------------------
    floatx16 acc1[TW1];
#pragma unroll
    for (int i = 0; i < TW1; ++i) {
        const int t = wave + i * NW;
        if (t < T1) acc1[i] = mma_wtile<KS1>(wf1[i], sN, PN, t & 1, t >> 1, F, D, lane);
    }
    // The ffn_out fragments, issued under the GELU work below.
    half8 wf2[TW2][KS2];
#pragma unroll
    for (int i = 0; i < TW2; ++i) {
        const int t = wave + i * NW;
        if (t < T2) load_wtile<KS2>(wf2[i], a.wout, D, F, t >> 1, lane);
    }
#pragma unroll
    for (int i = 0; i < TW1; ++i) {
        const int t = wave + i * NW;
        if (t >= T1) continue;
        const int mt = t & 1, nt = t >> 1;
        const int lr = mt * 32 + (lane & 31);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = nt * 32 + 8 * g + 4 * (lane >> 5);
            half4 hv;
#pragma unroll
            for (int e = 0; e < 4; ++e) hv[e] = to_half(gelu_erf<false>(acc1[i][4 * g + e] + p_bin[c + e]));
            *reinterpret_cast<half4*>(sH + lr * PH + c) = hv;
        }
    }
    __syncthreads();

    // ---- x2 = x1 + (h W_out^T + b_out), in place ----------------------------------
#pragma unroll
    for (int i = 0; i < TW2; ++i) {
        const int t = wave + i * NW;
        if (t >= T2) continue;
        const int mt = t & 1, nt = t >> 1;
        const floatx16 acc = mma_wtile<KS2>(wf2[i], sH, PH, mt, nt, D, F, lane);
        const int lr = mt * 32 + (lane & 31);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = nt * 32 + 8 * g + 4 * (lane >> 5);
            float4* px = reinterpret_cast<float4*>(sX + lr * PX + c);
            float4 x1 = *px;
            x1.x = x1.x + (acc[4 * g + 0] + p_bout[c + 0]);
            x1.y = x1.y + (acc[4 * g + 1] + p_bout[c + 1]);
            x1.z = x1.z + (acc[4 * g + 2] + p_bout[c + 2]);
            x1.w = x1.w + (acc[4 * g + 3] + p_bout[c + 3]);
            *px = x1;
        }
    }
    __syncthreads();

    // ---- n2 = LN(x2); write x2 and n2 ------------------------------------------------
    {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (has[i]) v[i] = *reinterpret_cast<const float4*>(sX + local_row(i) * PX + 4 * lh);
        }
        float m[NP], dl[NP], r[NP];
        ln_pairs<NP>(v, a.eps, inv_d, m, dl, r, has);
        const float4 ww = *reinterpret_cast<const float4*>(p_w2 + 4 * (lh % (DP / 4)));
        const float4 bb = *reinterpret_cast<const float4*>(p_b2 + 4 * (lh % (DP / 4)));
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            if (!has[i]) continue;
            const int64_t row = row0 + local_row(i);
            *reinterpret_cast<float4*>(a.x_out + row * D + 4 * lh) = v[i];
            *reinterpret_cast<float4*>(a.n_out + row * D + 4 * lh) =
                ln_apply(v[i], m[i], dl[i], r[i], ww, bb);
        }
    }
}

template <int DP, int FP>
void launch_ffn(const FfnArgs& a, hipStream_t stream) {
    constexpr int NW = FP > 128 ? 8 : 4;
    const int64_t blocks = (a.rows + kRows - 1) / kRows;
    hipLaunchKernelGGL((ffn_block_kernel<DP, FP, NW>), dim3(static_cast<unsigned>(blocks)),
                       dim3(NW * 64), 0, stream, a);
}

template <int DP>
bool launch_fp(const FfnArgs& a, int fp, hipStream_t stream) {
    switch (fp) {
        case 32: launch_ffn<DP, 32>(a, stream); return true;
        case 64: launch_ffn<DP, 64>(a, stream); return true;
        case 96: launch_ffn<DP, 96>(a, stream); return true;
        case 128: launch_ffn<DP, 128>(a, stream); return true;
        case 256: launch_ffn<DP, 256>(a, stream); return true;
        case 512: launch_ffn<DP, 512>(a, stream); return true;
    }
    return false;
}

}  // namespace
}  // namespace dotl

extern "C" int dotl_ffn_block(const float* x, const float* attn_out, const float* norm1_w,
                              const float* norm1_b, const void* ffn_in_w_half,
                              const float* ffn_in_b, const void* ffn_out_w_half,
                              const float* ffn_out_b, const float* norm2_w,
                              const float* norm2_b, float* x_out, float* normed_out,
                              int64_t rows, int64_t D, int64_t F, double eps, void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(rows >= 0 && D >= 1 && F >= 1, "fused_ffn_block: bad extents");
    if (D > 128 || F > 512 || D % 8 != 0 || F % 8 != 0) {
        char buf[200];
        std::snprintf(buf, sizeof(buf),
                      "fused_ffn_block: d_model=%lld, ffn_dim=%lld not covered: the fused block "
                      "takes d_model up to 128 and ffn_dim up to 512, multiples of 8; run the "
                      "unfused chain",
                      static_cast<long long>(D), static_cast<long long>(F));
        set_error(buf);
        return DOTL_DECLINED;
    }
    if (rows == 0) return DOTL_OK;
    DOTL_REQUIRE(x && attn_out && norm1_w && norm1_b && ffn_in_w_half && ffn_in_b &&
                     ffn_out_w_half && ffn_out_b && norm2_w && norm2_b && x_out && normed_out,
                 "fused_ffn_block: null pointer");
    const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(attn_out) |
                         reinterpret_cast<uintptr_t>(x_out) |
                         reinterpret_cast<uintptr_t>(normed_out) |
                         reinterpret_cast<uintptr_t>(ffn_in_w_half) |
                         reinterpret_cast<uintptr_t>(ffn_out_w_half);
    DOTL_REQUIRE(al % 16 == 0, "fused_ffn_block: tensors must be 16-byte aligned");
    DOTL_REQUIRE(rows <= (static_cast<int64_t>(0x7fffffff) * kRows),
                 "fused_ffn_block: too many rows");
    FfnArgs a{x, attn_out, norm1_w, norm1_b, static_cast<const _Float16*>(ffn_in_w_half),
              ffn_in_b, static_cast<const _Float16*>(ffn_out_w_half), ffn_out_b, norm2_w,
              norm2_b, x_out, normed_out, rows, static_cast<int>(D), static_cast<int>(F),
              static_cast<float>(eps)};
    const int dp = static_cast<int>((D + 31) / 32 * 32);
    int fp = static_cast<int>((F + 31) / 32 * 32);
    if (fp > 128) fp = fp <= 256 ? 256 : 512;
    const hipStream_t st = as_stream(stream);
    bool ok = false;
    switch (dp) {
        case 32: ok = launch_fp<32>(a, fp, st); break;
        case 64: ok = launch_fp<64>(a, fp, st); break;
        case 96: ok = launch_fp<96>(a, fp, st); break;
        case 128: ok = launch_fp<128>(a, fp, st); break;
    }
    if (!ok) {
        set_error("fused_ffn_block: no instance for this width");
        return DOTL_E_INVALID;
    }
    return check_launch("fused_ffn_block");
}
