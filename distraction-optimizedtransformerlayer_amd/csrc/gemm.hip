// out = act(x @ W^T + bias) on gfx950 MFMA.
//
// Replaces linear_bias / linear_gelu (reference csrc/linear_gelu.cuh:186-756):
// same operation, same operand layouts (x [M, K] row-major, W [N, K] in
// nn.Linear layout, fp32 bias), same fp16-operand / fp32-accumulate
// arithmetic for the default math, the exact-erf GELU in the epilogue.
//
// MI355X design:
//   * both operands are K-contiguous ("NT" GEMM), which is what MFMA wants:
//     lane l of v_mfma_f32_32x32x16_f16 supplies 8 consecutive K elements of
//     one A row and of one W row, so LDS tiles are plain row-major
//     [rows][BK] and every fragment is one 16-byte LDS read;
//   * 256 threads = 4 wavefronts in a 2 x 2 grid, each wavefront owning a
//     (BM/2) x (BN/2) block of 32x32 accumulator tiles;
//   * a two-stage pipeline: while the MFMAs read K tile kt from one LDS
//     stage, tile kt+1 (already in registers) is written to the other stage
//     and tile kt+2 is in flight from HBM/L2 -- one barrier per K step;
//   * a tile menu from 64x64 to 256x256 (the 256x256 tile holds a 128x128
//     accumulator block per wavefront: 256 accumulator registers), picked
//     per shape so the grid covers the 256 CUs;
//   * LDS rows are padded by 16 bytes so the 32 rows a fragment read touches
//     fall on distinct bank groups;
//   * W arrives pre-narrowed (dotl_weight_split, once per weight version);
//     x may be fp32 (narrowed with RNE while staging, exactly the rounding
//     the reference's Fp16Math applies) or fp16;
//   * DOTL_MATH_FP16X3: x and W are split into hi + 2^-12 * lo fp16 pairs and
//     the product is hi*hi + 2^-12 (hi*lo + lo*hi), with the two sums in
//     separate fp32 accumulators. Three MFMA passes buy ~22-bit operands:
//     fp32-class products on the fp16 matrix cores. It is what the
//     projection feeding attention's scores uses (the accuracy budget is
//     spent there; see the precision notes in the package's kernels.py).
//   * the output tile is written from the accumulators: lane l holds one
//     column and 16 rows of each 32x32 tile, so each store instruction
//     writes two 128-byte row segments.
#include "dotl_common.h"

namespace dotl {

int pick_dma_tile(int64_t M, int64_t N, int64_t K, int passes);
bool launch_gemm_dma(const _Float16* A, const _Float16* Alo, const _Float16* W,
                     const _Float16* Wlo, const float* bias, const float* R, void* C, int64_t M,
                     int64_t N, int64_t K, int mode, int act, int out_dtype, int tile,
                     hipStream_t stream);
bool launch_gemm_dma_ln(const _Float16* A, const _Float16* W, const float* bias, const float* R,
                        float* C, int64_t M, int64_t N, int64_t K, const float* ln_w,
                        const float* ln_b, float eps, void* normed, int normed_dtype,
                        int64_t plane, const int32_t* out_row, const int64_t* io, int tile,
                        hipStream_t stream);

namespace {

constexpr int kThreads = 256;
constexpr int kPad = 8;  // halves of padding per LDS row (16 bytes)

template <int BM, int BN, int BK>
struct TileShape {
    static constexpr int WM = BM / 2;       // rows per wavefront
    static constexpr int WN = BN / 2;       // cols per wavefront
    static constexpr int TM = WM / 32;      // 32x32 tiles per wavefront, M
    static constexpr int TN = WN / 32;      // 32x32 tiles per wavefront, N
    static constexpr int KS = BK / 16;      // MFMA k-steps per tile
    static constexpr int LDK = BK + kPad;   // LDS row pitch in halves
};

// Global -> register staging of one [ROWS, BK] fp16 tile: chunks of 8 halves.
template <int ROWS, int BK>
struct HalfTile {
    static constexpr int kChunks = ROWS * BK / 8;
    static constexpr int kPer = (kChunks + kThreads - 1) / kThreads;
    half8 r[kPer];

    __device__ __forceinline__ void load(const _Float16* __restrict__ src, int64_t ld,
                                         int64_t row0, int64_t nrows, int64_t k0, int64_t K) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + i * kThreads;
            const int row = c / (BK / 8);
            const int col = (c % (BK / 8)) * 8;
            half8 v = {};
            if (c < kChunks && row0 + row < nrows && k0 + col < K) {
                v = *reinterpret_cast<const half8*>(src + (row0 + row) * ld + k0 + col);
            }
            r[i] = v;
        }
    }
    __device__ __forceinline__ void store(_Float16* lds) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + i * kThreads;
            if (c < kChunks) {
                const int row = c / (BK / 8);
                const int col = (c % (BK / 8)) * 8;
                *reinterpret_cast<half8*>(lds + row * (BK + kPad) + col) = r[i];
            }
        }
    }
};

// Global -> register staging of one [ROWS, BK] fp32 tile, narrowed (and
// optionally split) when written to LDS. Chunks of 4 floats.
template <int ROWS, int BK>
struct FloatTile {
    static constexpr int kChunks = ROWS * BK / 4;
    static constexpr int kPer = (kChunks + kThreads - 1) / kThreads;
    float4 r[kPer];

    __device__ __forceinline__ void load(const float* __restrict__ src, int64_t ld,
                                         int64_t row0, int64_t nrows, int64_t k0, int64_t K) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + i * kThreads;
            const int row = c / (BK / 4);
            const int col = (c % (BK / 4)) * 4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c < kChunks && row0 + row < nrows && k0 + col < K) {
                v = *reinterpret_cast<const float4*>(src + (row0 + row) * ld + k0 + col);
            }
            r[i] = v;
        }
    }
    __device__ __forceinline__ void store(_Float16* lds) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + i * kThreads;
            if (c < kChunks) {
                const int row = c / (BK / 4);
                const int col = (c % (BK / 4)) * 4;
                half4 h;
                h[0] = to_half(r[i].x); h[1] = to_half(r[i].y);
                h[2] = to_half(r[i].z); h[3] = to_half(r[i].w);
                *reinterpret_cast<half4*>(lds + row * (BK + kPad) + col) = h;
            }
        }
    }
    __device__ __forceinline__ void store_split(_Float16* lds_hi, _Float16* lds_lo) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + i * kThreads;
            if (c < kChunks) {
                const int row = c / (BK / 4);
                const int col = (c % (BK / 4)) * 4;
                half4 h, l;
                h[0] = to_half(r[i].x); l[0] = split_lo(r[i].x, h[0]);
                h[1] = to_half(r[i].y); l[1] = split_lo(r[i].y, h[1]);
                h[2] = to_half(r[i].z); l[2] = split_lo(r[i].z, h[2]);
                h[3] = to_half(r[i].w); l[3] = split_lo(r[i].w, h[3]);
                *reinterpret_cast<half4*>(lds_hi + row * (BK + kPad) + col) = h;
                *reinterpret_cast<half4*>(lds_lo + row * (BK + kPad) + col) = l;
            }
        }
    }
};

// Workgroup -> output tile. Workgroups are dispatched round-robin over the
// 8 XCDs, each with its own L2, so the linear id is first regrouped so that
// every XCD walks a contiguous stretch of the tile order; that order then
// visits kGroupM row-tiles per column sweep, so the A rows and W columns a
// stretch touches stay L2-resident while they are reused.
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

__device__ __forceinline__ void tile_of(int64_t id, int64_t nm, int64_t nn, int64_t& mt,
                                        int64_t& nt) {
    const int64_t total = nm * nn;
    const int64_t per = total / kXcds;
    if (id < per * kXcds) id = (id % kXcds) * per + id / kXcds;
    const int64_t in_group = kGroupM * nn;
    const int64_t group = id / in_group;
    const int64_t first_m = group * kGroupM;
    const int64_t gsize = min(static_cast<int64_t>(kGroupM), nm - first_m);
    const int64_t r = id - group * in_group;
    mt = first_m + r % gsize;
    nt = r / gsize;
}

// LDS footprint of one pipeline stage, in halves: A [BM][LDK], W [BN][LDK],
// and for the split path lo(W) [BN][LDK] and, with an fp32 A, lo(A) [BM][LDK].
template <int BM, int BN, int BK, bool A_F32, bool SPLIT>
struct StageLayout {
    static constexpr int LDK = BK + kPad;
    static constexpr int A = 0;
    static constexpr int W = A + BM * LDK;
    static constexpr int WLO = W + BN * LDK;
    static constexpr int ALO = WLO + (SPLIT ? BN * LDK : 0);
    static constexpr int SIZE = ALO + ((SPLIT && A_F32) ? BM * LDK : 0);
    static constexpr size_t BYTES = 2u * SIZE * sizeof(_Float16);  // two stages
};

template <int BM, int BN, int BK, bool A_F32, bool SPLIT, int ACT, bool OUT_F16>
__global__ __launch_bounds__(kThreads) void gemm_kernel(
    const void* __restrict__ A_, const _Float16* __restrict__ Whi,
    const _Float16* __restrict__ Wlo, const float* __restrict__ bias,
    void* __restrict__ C_, int64_t M, int64_t N, int64_t K) {
    using TS = TileShape<BM, BN, BK>;
    using SL = StageLayout<BM, BN, BK, A_F32, SPLIT>;
    constexpr int LDK = TS::LDK;

    // Two pipeline stages: while the MFMAs read stage kt&1, the next K tile
    // (already in registers) is written to the other stage, and the tile after
    // that is in flight from HBM/L2. One barrier per K step.
    extern __shared__ __attribute__((aligned(16))) _Float16 smem[];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1;  // wave row in the 2x2 grid
    const int wn = wave & 1;
    const int lr = lane & 31;  // fragment row/col supplied by this lane
    const int lg = lane >> 5;  // which 8-wide K slice of the 16

    int64_t mt, nt;
    tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, mt, nt);
    const int64_t m0 = mt * BM;
    const int64_t n0 = nt * BN;

    floatx16 acc[TS::TM][TS::TN];
    floatx16 acc2[SPLIT ? TS::TM : 1][SPLIT ? TS::TN : 1];
#pragma unroll
    for (int i = 0; i < TS::TM; ++i)
#pragma unroll
        for (int j = 0; j < TS::TN; ++j) {
            acc[i][j] = floatx16{};
            if constexpr (SPLIT) acc2[i][j] = floatx16{};
        }

    using ATile = typename std::conditional<A_F32, FloatTile<BM, BK>, HalfTile<BM, BK>>::type;
    ATile ta;
    HalfTile<BN, BK> tw;
    HalfTile<SPLIT ? BN : 8, SPLIT ? BK : 8> twlo;

    auto fetch = [&](int64_t k0) {
        if constexpr (A_F32) {
            ta.load(static_cast<const float*>(A_), K, m0, M, k0, K);
        } else {
            ta.load(static_cast<const _Float16*>(A_), K, m0, M, k0, K);
        }
        tw.load(Whi, K, n0, N, k0, K);
        if constexpr (SPLIT) twlo.load(Wlo, K, n0, N, k0, K);
    };
    auto commit = [&](_Float16* st) {
        if constexpr (SPLIT && A_F32) {
            ta.store_split(st + SL::A, st + SL::ALO);
        } else {
            ta.store(st + SL::A);
        }
        tw.store(st + SL::W);
        if constexpr (SPLIT) twlo.store(st + SL::WLO);
    };

    // Bias columns for the epilogue, fetched before the K loop.
    float bvals[TS::TN];
#pragma unroll
    for (int j = 0; j < TS::TN; ++j) {
        const int64_t col = n0 + wn * TS::WN + j * 32 + lr;
        bvals[j] = col < N ? bias[col] : 0.f;
    }

    const int64_t nk = (K + BK - 1) / BK;
    fetch(0);
    commit(smem);
    if (nk > 1) fetch(BK);
    __syncthreads();

    for (int64_t kt = 0; kt < nk; ++kt) {
        _Float16* cur = smem + (kt & 1) * SL::SIZE;
        if (kt + 1 < nk) commit(smem + ((kt + 1) & 1) * SL::SIZE);
        if (kt + 2 < nk) fetch((kt + 2) * BK);

        const _Float16* sA = cur + SL::A;
        const _Float16* sW = cur + SL::W;
#pragma unroll
        for (int ks = 0; ks < TS::KS; ++ks) {
            const int kc = ks * 16 + lg * 8;
            half8 a[TS::TM], b[TS::TN];
#pragma unroll
            for (int i = 0; i < TS::TM; ++i)
                a[i] = *reinterpret_cast<const half8*>(sA + (wm * TS::WM + i * 32 + lr) * LDK + kc);
#pragma unroll
            for (int j = 0; j < TS::TN; ++j)
                b[j] = *reinterpret_cast<const half8*>(sW + (wn * TS::WN + j * 32 + lr) * LDK + kc);
#pragma unroll
            for (int i = 0; i < TS::TM; ++i)
#pragma unroll
                for (int j = 0; j < TS::TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            if constexpr (SPLIT) {
                // 2^-12-scaled residual products: hi(x) * lo(W), and for an
                // fp32 x also lo(x) * hi(W). An fp16 x has no residual.
                const _Float16* sWlo = cur + SL::WLO;
                half8 bl[TS::TN];
#pragma unroll
                for (int j = 0; j < TS::TN; ++j)
                    bl[j] = *reinterpret_cast<const half8*>(sWlo + (wn * TS::WN + j * 32 + lr) * LDK + kc);
#pragma unroll
                for (int i = 0; i < TS::TM; ++i)
#pragma unroll
                    for (int j = 0; j < TS::TN; ++j)
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl[j], acc2[i][j], 0, 0, 0);
                if constexpr (A_F32) {
                    const _Float16* sAlo = cur + SL::ALO;
                    half8 al[TS::TM];
#pragma unroll
                    for (int i = 0; i < TS::TM; ++i)
                        al[i] = *reinterpret_cast<const half8*>(sAlo + (wm * TS::WM + i * 32 + lr) * LDK + kc);
#pragma unroll
                    for (int i = 0; i < TS::TM; ++i)
#pragma unroll
                        for (int j = 0; j < TS::TN; ++j)
                            acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], acc2[i][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    // Epilogue. Accumulator register r of a 32x32 tile at lane l holds
    // row 8*(r/4) + 4*(l/32) + (r%4), column l%32.
#pragma unroll
    for (int j = 0; j < TS::TN; ++j) {
        const int64_t col = n0 + wn * TS::WN + j * 32 + lr;
        if (col >= N) continue;
        const float bcol = bvals[j];
#pragma unroll
        for (int i = 0; i < TS::TM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * TS::WM + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                if (row < M) {
                    float v = acc[i][j][r];
                    if constexpr (SPLIT) v += acc2[i][j][r] * kLoUnscale;
                    v += bcol;
                    if constexpr (ACT == DOTL_ACT_GELU) v = gelu_erf<false>(v);
                    if constexpr (OUT_F16) {
                        static_cast<_Float16*>(C_)[row * N + col] = to_half(v);
                    } else {
                        static_cast<float*>(C_)[row * N + col] = v;
                    }
                }
            }
        }
    }
}

__global__ void weight_split_kernel(const float* __restrict__ w, _Float16* __restrict__ hi,
                                    _Float16* __restrict__ lo, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) {
        const _Float16 h = to_half(w[i]);
        hi[i] = h;
        if (lo) lo[i] = split_lo(w[i], h);
    }
}

struct GemmArgs {
    const void* A;
    const _Float16* Whi;
    const _Float16* Wlo;
    const float* bias;
    void* C;
    int64_t M, N, K;
    hipStream_t stream;
};

template <int BM, int BN, int BK, bool A_F32, bool SPLIT, int ACT, bool OUT_F16>
void launch(const GemmArgs& g) {
    using SL = StageLayout<BM, BN, BK, A_F32, SPLIT>;
    auto kern = gemm_kernel<BM, BN, BK, A_F32, SPLIT, ACT, OUT_F16>;
    // Above 64 KiB of dynamic LDS the kernel must opt in; done once per
    // instantiation, on the first (eager, never captured) call.
    static const bool attr_ok = [&] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(SL::BYTES)) == hipSuccess;
    }();
    (void)attr_ok;
    const dim3 grid(static_cast<unsigned>(((g.N + BN - 1) / BN) * ((g.M + BM - 1) / BM)));
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), SL::BYTES, g.stream, g.A, g.Whi, g.Wlo, g.bias,
                       g.C, g.M, g.N, g.K);
}

// Tile menu (ids are the C ABI's `tile` argument). 2 x 2 wavefronts each.
//   0: 128 x 128   1: 256 x 128   2: 64 x 64   3: 256 x 256   4: 128 x 64
template <bool A_F32, bool SPLIT, int ACT, bool OUT_F16>
bool launch_tile(const GemmArgs& g, int tile) {
    switch (tile) {
        case 0: launch<128, 128, 64, A_F32, SPLIT, ACT, OUT_F16>(g); return true;
        case 2: launch<64, 64, 64, A_F32, SPLIT, ACT, OUT_F16>(g); return true;
        case 4: launch<128, 64, 64, A_F32, SPLIT, ACT, OUT_F16>(g); return true;
        case 1:
            if constexpr (!SPLIT) { launch<256, 128, 64, A_F32, SPLIT, ACT, OUT_F16>(g); return true; }
            return false;
        case 3:
            if constexpr (!SPLIT && !A_F32) { launch<256, 256, 64, A_F32, SPLIT, ACT, OUT_F16>(g); return true; }
            return false;
    }
    return false;
}

template <bool A_F32, bool SPLIT>
bool launch_epilogue(const GemmArgs& g, int tile, int act, bool out_f16) {
    if (act == DOTL_ACT_GELU) {
        return out_f16 ? launch_tile<A_F32, SPLIT, DOTL_ACT_GELU, true>(g, tile)
                       : launch_tile<A_F32, SPLIT, DOTL_ACT_GELU, false>(g, tile);
    }
    return out_f16 ? launch_tile<A_F32, SPLIT, DOTL_ACT_NONE, true>(g, tile)
                   : launch_tile<A_F32, SPLIT, DOTL_ACT_NONE, false>(g, tile);
}

// Tile choice for 256 CUs: the largest tile the operand types allow that
// still gives about one workgroup per CU; below that, the smallest.
int pick_tile(int64_t M, int64_t N, bool a_f32, bool split) {
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    const int64_t fill = 240;
    if (!split && !a_f32 && tiles(256, 256) >= fill) return 3;
    if (!split && tiles(256, 128) >= fill) return 1;
    if (tiles(128, 128) >= fill) return 0;
    if (tiles(128, 64) >= fill) return 4;
    return 2;
}

}  // namespace
}  // namespace dotl

extern "C" int dotl_weight_split(const float* w, void* w_hi, void* w_lo, int64_t n,
                                 void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(n >= 0, "weight_split: negative size");
    if (n == 0) return DOTL_OK;
    DOTL_REQUIRE(w && w_hi, "weight_split: null pointer");
    const int64_t blocks = (n + 255) / 256;
    DOTL_REQUIRE(blocks <= 0x7fffffff, "weight_split: too many elements");
    hipLaunchKernelGGL(weight_split_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       as_stream(stream), w, static_cast<_Float16*>(w_hi),
                       static_cast<_Float16*>(w_lo), n);
    return check_launch("weight_split");
}

namespace dotl {
namespace {

// x_lo: the lo plane of a split x (DOTL_F16X2) where it does not follow the
// hi plane directly (null: at x + M * K).
int linear_impl(const void* x, int x_dtype, const void* w_hi, const void* w_lo,
                const float* bias, const float* residual, void* out, int out_dtype, int64_t M,
                int64_t N, int64_t K, int act, int math, int tile, void* stream,
                const void* x_lo = nullptr) {
    clear_error();
    const char* who = act == DOTL_ACT_GELU ? "linear_gelu" : "linear_bias";
    DOTL_REQUIRE(x_dtype == DOTL_F32 || x_dtype == DOTL_F16 || x_dtype == DOTL_F16X2 ||
                     x_dtype == DOTL_BF16,
                 "%s: x must be float32, float16, bfloat16 or split float16", who);
    DOTL_REQUIRE(out_dtype == DOTL_F32 || out_dtype == DOTL_F16 || out_dtype == DOTL_BF16,
                 "%s: out must be float32, float16 or bfloat16", who);
    DOTL_REQUIRE((x_dtype == DOTL_BF16) == (out_dtype == DOTL_BF16) || out_dtype == DOTL_F32,
                 "%s: a bfloat16 x writes float32 or bfloat16, other x float32 or float16", who);
    DOTL_REQUIRE(x_dtype != DOTL_BF16 || math == DOTL_MATH_FP16,
                 "%s: a bfloat16 x (with a bfloat16 W) runs one pass (math %d)", who,
                 DOTL_MATH_FP16);
    DOTL_REQUIRE(act == DOTL_ACT_NONE || act == DOTL_ACT_GELU, "%s: unknown activation %d", who, act);
    DOTL_REQUIRE(math == DOTL_MATH_FP16 || math == DOTL_MATH_FP16X3 || math == DOTL_MATH_FP16X2,
                 "%s: unknown math %d", who, math);
    DOTL_REQUIRE(math != DOTL_MATH_FP16X2 || x_dtype == DOTL_F16X2,
                 "%s: the fp16x2 math takes x as split fp16 planes", who);
    DOTL_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative extent", who);
    if (K % 8 != 0 || K == 0) {
        set_error(std::string(who) + ": K must be a positive multiple of 8 for 16-byte staging");
        return DOTL_DECLINED;
    }
    if (x_dtype == DOTL_F16X2 && K % 64 != 0) {
        set_error(std::string(who) + ": a split-fp16 x needs K % 64 == 0");
        return DOTL_DECLINED;
    }
    DOTL_REQUIRE(math != DOTL_MATH_FP16X3 || w_lo != nullptr,
                 "%s: the fp16x3 math needs the split weight residual", who);
    DOTL_REQUIRE(((M + 63) / 64) * ((N + 63) / 64) <= 0x7fffffff, "%s: too large", who);
    DOTL_REQUIRE(tile == -1 || (tile >= 0 && tile <= 19) || (tile >= 100 && tile <= 104),
                 "%s: unknown tile id %d", who, tile);
    if (M == 0 || N == 0) return DOTL_OK;
    DOTL_REQUIRE(x && w_hi && bias && out, "%s: null pointer", who);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_hi) |
                            reinterpret_cast<uintptr_t>(w_lo);
    DOTL_REQUIRE(align % 16 == 0, "%s: x and W must be 16-byte aligned", who);
    const bool of16 = out_dtype == DOTL_F16;
    const bool split = math == DOTL_MATH_FP16X3;
    const bool bf16 = x_dtype == DOTL_BF16;

    // LDS-DMA pipelined kernel: fp16 operands, K a multiple of 64, each
    // operand under 4 GiB (its per-lane DMA offsets are 32-bit).
    const bool force_staged = tile >= 100;
    const bool dma_fits = M * K * 2 < (int64_t{1} << 32) && N * K * 2 < (int64_t{1} << 32);
    if (!force_staged && x_dtype != DOTL_F32 && K % 64 == 0 && dma_fits) {
        const _Float16* xh = static_cast<const _Float16*>(x);
        const _Float16* xl =
            x_dtype != DOTL_F16X2 ? nullptr
                                  : (x_lo != nullptr ? static_cast<const _Float16*>(x_lo) : xh + M * K);
        // split modes: bit 0 lo(W), bit 1 lo(x)
        const int mode = bf16 ? 4
                         : (math == DOTL_MATH_FP16X2 ? 2
                            : (!split ? 0 : (x_dtype == DOTL_F16X2 ? 3 : 1)));
        const int passes = 1 + (mode & 1) + ((mode >> 1) & 1);
        const int t = tile < 0 ? pick_dma_tile(M, N, K, passes) : tile;
        if (launch_gemm_dma(xh, xl, static_cast<const _Float16*>(w_hi),
                            static_cast<const _Float16*>(w_lo), bias, residual, out, M, N, K,
                            mode, act, out_dtype, t, as_stream(stream))) {
            return check_launch(who);
        }
        DOTL_REQUIRE(x_dtype != DOTL_F16X2, "%s: tile id %d is not built for split passes", who, tile);
    }
    DOTL_REQUIRE(x_dtype != DOTL_F16X2,
                 "%s: split-fp16 x is served by the pipelined kernel only (K %% 64 == 0, operands "
                 "under 4 GiB)", who);
    if (bf16) {
        set_error(std::string(who) + ": bfloat16 operands are served by the pipelined kernel "
                  "only (K % 64 == 0, operands under 4 GiB)");
        return DOTL_DECLINED;
    }
    if (residual != nullptr) {
        set_error(std::string(who) + ": the residual epilogue is served by the pipelined kernel "
                  "only (fp16 or split x, K % 64 == 0); add the residual separately");
        return DOTL_DECLINED;
    }

    GemmArgs g{x, static_cast<const _Float16*>(w_hi), static_cast<const _Float16*>(w_lo), bias,
               out, M, N, K, as_stream(stream)};
    const bool a_f32 = x_dtype == DOTL_F32;
    const int t = (tile < 0 || tile % 100 > 4) ? pick_tile(M, N, a_f32, split) : (tile % 100);
    bool ok;
    if (split) {
        ok = a_f32 ? launch_epilogue<true, true>(g, t, act, of16)
                   : launch_epilogue<false, true>(g, t, act, of16);
    } else {
        ok = a_f32 ? launch_epilogue<true, false>(g, t, act, of16)
                   : launch_epilogue<false, false>(g, t, act, of16);
    }
    DOTL_REQUIRE(ok, "%s: tile id %d is not built for these operand types", who, tile);
    return check_launch(who);
}

}  // namespace
}  // namespace dotl

extern "C" int dotl_linear(const void* x, int x_dtype, const void* w_hi, const void* w_lo,
                           const float* bias, void* out, int out_dtype, int64_t M, int64_t N,
                           int64_t K, int act, int math, int tile, void* stream) {
    return dotl::linear_impl(x, x_dtype, w_hi, w_lo, bias, nullptr, out, out_dtype, M, N, K, act,
                             math, tile, stream);
}

extern "C" int dotl_linear_planes(const void* x_hi, const void* x_lo, const void* w_hi,
                                  const void* w_lo, const float* bias, void* out, int out_dtype,
                                  int64_t M, int64_t N, int64_t K, int math, int tile,
                                  void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(M == 0 || N == 0 || x_lo != nullptr, "linear_bias: null lo plane");
    DOTL_REQUIRE(reinterpret_cast<uintptr_t>(x_lo) % 16 == 0,
                 "linear_bias: the lo plane must be 16-byte aligned");
    DOTL_REQUIRE(math == DOTL_MATH_FP16X2 || math == DOTL_MATH_FP16X3,
                 "linear_bias: split planes take the fp16x2 or fp16x3 math");
    return linear_impl(x_hi, DOTL_F16X2, w_hi, w_lo, bias, nullptr, out, out_dtype, M, N, K,
                       DOTL_ACT_NONE, math, tile, stream, x_lo);
}

extern "C" int dotl_linear_residual(const void* x, int x_dtype, const void* w_hi,
                                    const void* w_lo, const float* bias, const float* residual,
                                    float* out, int64_t M, int64_t N, int64_t K, int act, int math,
                                    int tile, void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(M == 0 || N == 0 || residual != nullptr, "linear_bias: null residual");
    DOTL_REQUIRE(reinterpret_cast<uintptr_t>(residual) % 16 == 0,
                 "linear_bias: the residual must be 16-byte aligned");
    return linear_impl(x, x_dtype, w_hi, w_lo, bias, residual, out, DOTL_F32, M, N, K, act, math,
                       tile, stream);
}

extern "C" int dotl_linear_layernorm(const void* x, int x_dtype, const void* w_hi,
                                     const float* bias, const float* residual, float* out,
                                     const float* ln_weight, const float* ln_bias, double eps,
                                     void* normed, int normed_dtype, const int32_t* out_row,
                                     int64_t normed_rows, const int64_t* io, int64_t M, int64_t N,
                                     int64_t K, int tile, void* stream) {
    using namespace dotl;
    clear_error();
    const char* who = "linear_layernorm";
    DOTL_REQUIRE(M >= 0 && N >= 0 && K >= 0 && normed_rows >= 0, "%s: negative extent", who);
    DOTL_REQUIRE(normed_dtype == DOTL_F32 || normed_dtype == DOTL_F16 ||
                     normed_dtype == DOTL_F16X2,
                 "%s: the normed output is float32, float16 or split float16", who);
    DOTL_REQUIRE(out_row != nullptr || normed_rows == M,
                 "%s: without out_row the normed output has the product's %lld rows", who,
                 static_cast<long long>(M));
    DOTL_REQUIRE(out_row == nullptr || normed_dtype == DOTL_F32,
                 "%s: scattered rows (out_row) take a float32 normed output", who);
    DOTL_REQUIRE(tile == -1 || tile == 18, "%s: tile %d (18, 128x256, takes a row LayerNorm)",
                 who, tile);
    if (x_dtype != DOTL_F16 || N > 256 || N % 4 != 0 || K % 64 != 0 || K == 0 ||
        M * K * 2 >= (int64_t{1} << 32) || N * K * 2 >= (int64_t{1} << 32)) {
        set_error(std::string(who) + ": served for a float16 x, N a multiple of 4 up to 256, "
                  "K a positive multiple of 64 and operands under 4 GiB; run the GEMM and the "
                  "LayerNorm separately");
        return DOTL_DECLINED;
    }
    if (M == 0 || N == 0) return DOTL_OK;
    DOTL_REQUIRE(x && w_hi && bias && ln_weight && ln_bias && (normed || io), "%s: null pointer",
                 who);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_hi) |
                            reinterpret_cast<uintptr_t>(residual) |
                            reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(ln_weight) |
                            reinterpret_cast<uintptr_t>(ln_bias) |
                            reinterpret_cast<uintptr_t>(normed);
    DOTL_REQUIRE(align % 16 == 0, "%s: every tensor must be 16-byte aligned", who);
    const int t = 18;   // 128x256: a row per wave instruction
    const bool ok = launch_gemm_dma_ln(static_cast<const _Float16*>(x),
                                       static_cast<const _Float16*>(w_hi), bias, residual, out, M,
                                       N, K, ln_weight, ln_bias, static_cast<float>(eps), normed,
                                       normed_dtype, normed_rows * N, out_row, io, t,
                                       as_stream(stream));
    DOTL_REQUIRE(ok, "%s: tile %d is not built with the LayerNorm epilogue", who, t);
    return check_launch(who);
}
