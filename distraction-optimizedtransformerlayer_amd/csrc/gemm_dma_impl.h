#pragma once
// out = act(x @ W^T + bias) on gfx950 MFMA, operands streamed HBM -> LDS by
// the LDS-DMA loads (global_load_lds_dwordx4), NS pipeline stages deep.
//
// The fast path behind dotl_linear for fp16 operands (x fp16, or x as split
// fp16 hi/lo planes) with K a multiple of 64; gemm.hip's register-staged
// kernel serves everything else (fp32 x, ragged K).
//
// MI355X design:
//   * no staging registers: each lane's 16-byte load lands directly in LDS
//     (the wave's 64 lanes fill one contiguous 1 KiB run, lane l at +16 l),
//     so the pipeline can be 2-8 stages deep (up to 144 KiB of the CU's
//     160 KiB LDS) without spending VGPRs. Measured on MI355X with the C4
//     QKV product's address stream alone (1.5 GB of L2 -> LDS): 128-byte K
//     rows (BK = 64, each 8 lanes one whole cache line) stream it in 74 us
//     with one 64 KiB stage in flight a workgroup and two workgroups a CU,
//     70 us with two stages in flight; 64-byte rows (BK = 32) take 114 us,
//     each line being fetched twice. One workgroup a CU with one stage in
//     flight (the 256x256 tile's 2 x 64 KiB) takes 125 us: the stage's
//     round trip, ~1.3 us, is what the tile's MFMAs must cover;
//   * the MFMA ceiling with data: 32x32x16 f16 products on random operands
//     pull the clock down to ~1.7 GHz (2.2 GHz on constant ones), ~1.5
//     PFLOP/s sustained, so ~60% of the 2.5 PFLOP/s datasheet figure is the
//     practical roof of every kernel here;
//   * each stage is its own __shared__ array and the K loop is unrolled by
//     NS, so every LDS read names a stage the in-flight DMA provably does not
//     write: the compiler then adds no conservative vmcnt(0) before the reads;
//     the kernel waits itself, for exactly the loads of the tile it is about
//     to read (vmcnt = loads of the younger tiles still allowed in flight);
//   * LDS rows are BK*2 bytes with the 16-byte chunks XOR-swizzled: a
//     ds_read_b128 serves 16 lanes per pass over the 64 four-byte banks, and
//     the 16 rows a fragment read touches then sit on 16 distinct 16-byte
//     bank groups (chunk ^ (row / rows-per-256B) % chunks-per-row),
//     conflict-free without padding (which would break the DMA's contiguous
//     lane layout; measured with SQ_LDS_BANK_CONFLICT on an LDS-only loop:
//     zero, against 2-way for a 128-byte sweep and 4-way unswizzled). The
//     swizzle is applied on the global side: each DMA lane writes a fixed
//     physical chunk and loads the logical chunk that maps there;
//   * rows past M (or N) are clamped to the last valid row -- those outputs
//     are never stored -- so every DMA is in bounds and branch-free; K must
//     be a multiple of 64 (no K tail);
//   * MODE 4 streams bf16 x and W (v_mfma_f32_32x32x16_bf16), one pass;
//   * MODE (bit 0: split W, bit 1: split x) sets the passes: 0 x*W; 1
//     x*W + 2^-12 x*lo(W) (x exact in fp16); 2 hi(x)*W + 2^-12 lo(x)*W (x
//     given as fp16 hi/lo planes, W in fp16); 3 all three products: the
//     lo terms in a second fp32 accumulator;
//   * 2 x 2 (or 2 x 4) wavefronts, each a (BM/2) x (BN/WGN) block of 32x32
//     accumulators, issued as W x A^T so every accumulator holds a C^T
//     tile: each lane owns runs of 4 consecutive output columns of one row.
//     The epilogue transposes the tile through the (then free) stage
//     buffers so that bias, GELU, residual loads and output stores run on
//     row-contiguous 16-byte chunks. Its cost matters: with one workgroup
//     per CU nothing overlaps it, and at the configs' short K (256-512) it
//     was costing more than the MFMAs.
#include <type_traits>

#include "dotl_dma.h"
#include "gemm_dma.h"

// Kernels and launchers with external linkage in dotl::gemm_dma: each mode's
// translation unit instantiates only its own (DOTL_GEMM_DMA_INSTANTIATE).
namespace dotl {
namespace gemm_dma {


constexpr int kThreads = 256;
constexpr int kXcds = 8;
// Share of the last k step's MFMAs a tile defers past the next barrier, in
// eighths (DmaGemm::compute). Same-box A/B on MI355X, none / half / all
// (bit-identical outputs): C4 QKV 188 / 180 / 174 us, ffn_in 263 / 257 /
// 255, ffn_out + residual 240 / 238 / 236, C3 split QKV 64 / 61 / 61, C5
// ffn_in 118 / 114 / 110.
constexpr int kDeferEighths = 8;
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

// NWV wavefronts a workgroup: 4 (2 x 2, one per SIMD) or 8 (2 x 4, two per
// SIMD, so one wave's MFMAs run while its partner waits on LDS or the DMA).
template <int BM, int BN, int BK, int MODE, int NWV = 4>
struct DmaLayout {
    // rows of BK halves in one stage: A, W, then lo(W) (MODE & 1), lo(A) (MODE & 2)
    static constexpr bool SW = (MODE & 1) != 0;
    static constexpr bool SA = (MODE & 2) != 0;
    static constexpr int CPR = BK / 8;               // 16-byte chunks per row
    static constexpr int ROWS_PER_DMA = 64 / CPR;    // rows one wave instruction fills
    static constexpr int ROWS_PER_ROUND = NWV * ROWS_PER_DMA;
    static constexpr int SWZ_DIV = 256 / (BK * 2);   // rows per 256-byte bank sweep
    static constexpr int A_ROW = 0;
    static constexpr int W_ROW = BM;
    static constexpr int WLO_ROW = BM + BN;
    static constexpr int ALO_ROW = WLO_ROW + (SW ? BN : 0);
    static constexpr int ROWS = ALO_ROW + (SA ? BM : 0);
    static constexpr int HALVES = ROWS * BK;
    static constexpr int LOADS = ROWS / ROWS_PER_ROUND;   // DMA instructions per wave per stage
    static_assert(BM % ROWS_PER_ROUND == 0 && BN % ROWS_PER_ROUND == 0, "rows per round");
    __device__ __forceinline__ static int swz(int row) { return (row / SWZ_DIV) % CPR; }
};

template <int BM, int BN, int BK, int NS, int MODE, int ACT, int OUTT, int NWV = 4>
struct DmaGemm {
    using L = DmaLayout<BM, BN, BK, MODE, NWV>;
    static constexpr int WGN = NWV / 2;          // waves across N (2 or 4); 2 across M
    static constexpr bool SPLIT = (MODE & 3) != 0;
    // MODE 4: bf16 operands (the LDS stages hold 16-bit values either way), one pass
    static constexpr bool BF16 = MODE == 4;
    static constexpr int WM = BM / 2, WN = BN / WGN;
    static constexpr int TM = WM / 32, TN = WN / 32;

    const _Float16* __restrict__ A;
    const _Float16* __restrict__ Alo;
    const _Float16* __restrict__ W;
    const _Float16* __restrict__ Wlo;
    int64_t M, N, K, m0, n0, nk;
    int wave, lane, wm, wn, lr, lg;
    floatx16 acc[TM][TN];
    floatx16 acc2[SPLIT ? TM : 1][SPLIT ? TN : 1];

    // A stage's DMA instructions (this wave's), in order: the rounds of A,
    // W, lo(W) (MODE & 1), lo(A) (MODE & 2). Each lane's byte offset
    // into its operand at k = 0 is computed once (row clamped to the last
    // valid one, logical chunk from the swizzle); a stage then only adds the
    // wave-uniform k offset to the operand's base, in scalar registers.
    static constexpr int RA = BM / L::ROWS_PER_ROUND, RW = BN / L::ROWS_PER_ROUND;
    static constexpr int NDMA = L::LOADS;
    static constexpr int KS = BK / 16;
    static constexpr int NWLO = L::SW ? RW : 0;
    static constexpr int op_of(int d) {
        return d < RA ? 0 : (d < RA + RW ? 1 : (d < RA + RW + NWLO ? 2 : 3));
    }
    static constexpr int round_of(int d) {
        return d < RA ? d : (d < RA + RW ? d - RA : (d < RA + RW + NWLO ? d - RA - RW : d - RA - RW - NWLO));
    }
    static constexpr int region_row(int op) {
        return op == 0 ? L::A_ROW : (op == 1 ? L::W_ROW : (op == 2 ? L::WLO_ROW : L::ALO_ROW));
    }
    unsigned doff[NDMA];

    __device__ __forceinline__ void init_offsets() {
        const int sub = lane / L::CPR;      // row within this wave's instruction
        const int pc = lane % L::CPR;       // physical chunk this lane fills
        static_for<0, NDMA>([&](auto dd) {
            constexpr int D = decltype(dd)::value;
            constexpr int op = op_of(D);
            constexpr bool is_a = op == 0 || op == 3;
            const int r = round_of(D) * L::ROWS_PER_ROUND + wave * L::ROWS_PER_DMA + sub;
            const int lc = pc ^ L::swz(r);  // logical chunk it holds
            const int64_t nrows = is_a ? M : N;
            int64_t gr = (is_a ? m0 : n0) + r;
            gr = gr < nrows ? gr : nrows - 1;
            doff[D] = static_cast<unsigned>((gr * K + lc * 8) * 2);
        });
    }

    template <int D>
    __device__ __forceinline__ void issue_one(_Float16* stage, int64_t kt) const {
        constexpr int op = op_of(D);
        const _Float16* src = op == 0 ? A : (op == 1 ? W : (op == 2 ? Wlo : Alo));
        constexpr int row = region_row(op) + round_of(D) * L::ROWS_PER_ROUND;
        dma16_off(src + kt * BK, doff[D], stage + (row + wave * L::ROWS_PER_DMA) * BK);
    }

    // DMAs [LO, HI) of tile kt into `stage`.
    template <int LO, int HI>
    __device__ __forceinline__ void issue_range(_Float16* stage, int64_t kt) const {
        static_for<LO, HI>([&](auto dd) { issue_one<decltype(dd)::value>(stage, kt); });
    }

    // One 32x32x16 product on the operand type the mode streams.
    __device__ __forceinline__ static floatx16 mma(half8 b, half8 a, floatx16 c) {
        if constexpr (BF16) {
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b),
                                                           __builtin_bit_cast(bf16x8, a), c, 0,
                                                           0, 0);
        } else {
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c, 0, 0, 0);
        }
    }

    // Fragment of row `row` (tile-local), 16-wide k step `ks`: the 8 halves of
    // lane group lg, at the swizzled chunk.
    __device__ __forceinline__ half8 frag(const _Float16* region, int row, int ks) const {
        const int pc = (ks * 2 + lg) ^ L::swz(row);
        return *reinterpret_cast<const half8*>(region + row * BK + pc * 8);
    }

    // Multiply the tile in `stage`; if `more`, issue tile kt_next into
    // `next` meanwhile. Three schedules, all measured on MI355X:
    //   * with two stages the next tile's DMAs all go out during the first
    //     two 16-deep k steps' worth of MFMAs, one after an MFMA (the
    //     vector-memory issue stalls while the CU's load queue is full;
    //     behind an MFMA the stall is hidden), so the stage's round trip
    //     (~1.3 us for 64 KiB, one stage in flight a CU) runs under the
    //     tile's remaining MFMAs. Spread evenly over the tile, the last slice
    //     was issued at its end and the barrier waited out its full latency;
    //   * the fragments of k step ks + 1 are read from LDS before the MFMAs
    //     of step ks are issued, so their latency too runs under MFMAs;
    //   * DEFER of the last k step's PER MFMAs (one per accumulator) are
    //     issued after the next tile's barrier, from fragments already in
    //     registers: they keep the matrix core busy while that tile's first
    //     fragment reads are in flight, a latency every wave otherwise waited
    //     out with the core idle at each tile boundary (the ones not deferred
    //     would cover the waves' skew in reaching the barrier instead; all
    //     deferred measured best).
    static constexpr int PER = TM * TN;
    static constexpr int DEFER = PER * kDeferEighths / 8;
    static_assert(KS % 2 == 0, "the deferred fragments sit in register set 1");
    half8 fa[2][TM], fb[2][TN];

    // The deferred MFMAs of the previous tile (all of them when it is the last).
    template <int LO, int HI>
    __device__ __forceinline__ void deferred_mma() {
        static_for<LO, HI>([&](auto mm) {
            constexpr int m = PER - DEFER + decltype(mm)::value;
            constexpr int i = m / TN, j = m % TN;
            acc[i][j] = mma(fb[1][j], fa[1][i], acc[i][j]);
        });
    }
    __device__ __forceinline__ void finish() { deferred_mma<0, DEFER>(); }

    __device__ __forceinline__ void compute(const _Float16* stage, _Float16* next, int64_t kt_next,
                                            bool more, bool pend) {
        // MFMA rounds the DMAs are spread over: the first two k steps' worth
        // with two stages (the next barrier waits for them; on MI355X two
        // beat one by 1-4% and all four lose 3-5%); with more stages each
        // tile has NS - 2 further tiles' MFMAs to land, and an even spread
        // over the whole tile issues more gently.
        constexpr int ISSUE = (NS == 2 ? (KS < 2 ? KS : 2) : KS) * PER;
        constexpr int NF = TM + TN;                     // fragment reads a k step
        constexpr int ROUNDS = PER > NF ? PER : NF;
        auto dma_slot = [&](auto rr) {
            constexpr int r = decltype(rr)::value;      // MFMA round within the tile
            if constexpr (r < ISSUE) {
                if (more) issue_range<r * NDMA / ISSUE, (r + 1) * NDMA / ISSUE>(next, kt_next);
            }
        };
        // Phase 0: the previous tile's deferred MFMAs, this tile's first
        // fragment reads, the first DMA slices.
        static_for<0, (DEFER > NF ? DEFER : NF)>([&](auto mm) {
            constexpr int m = decltype(mm)::value;
            if constexpr (m < DEFER) {
                if (pend) deferred_mma<m, m + 1>();
                dma_slot(std::integral_constant<int, m>{});
            }
            if constexpr (m < NF) {
                if constexpr (m < TM)
                    fa[0][m] = frag(stage + L::A_ROW * BK, wm * WM + m * 32 + lr, 0);
                else
                    fb[0][m - TM] = frag(stage + L::W_ROW * BK, wn * WN + (m - TM) * 32 + lr, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        static_for<0, KS>([&](auto kk) {
            constexpr int ks = decltype(kk)::value;
            constexpr int cur = ks & 1;
            half8 (&a)[TM] = fa[cur];
            half8 (&b)[TN] = fb[cur];
            // MFMAs of this step: all of them, or the last step's undeferred.
            constexpr int NM = ks + 1 < KS ? PER : PER - DEFER;
            // Round m: MFMA m of this step, fragment read m of the next step,
            // DMA slice m. The scheduling barrier after each round keeps the
            // compiler from regrouping them: left free it sank the reads of
            // step ks + 1 below the MFMAs of step ks (less register pressure),
            // and every step then began by waiting out a full LDS read
            // latency with the matrix core idle -- the loop ran at ~55% of
            // the MFMA rate with no global traffic at all.
            static_for<0, (NM > NF ? NM : NF)>([&](auto mm) {
                constexpr int m = decltype(mm)::value;
                if constexpr (m < NM) {
                    constexpr int i = m / TN, j = m % TN;
                    acc[i][j] = mma(b[j], a[i], acc[i][j]);
                    dma_slot(std::integral_constant<int, DEFER + ks * PER + m>{});
                }
                if constexpr (ks + 1 < KS && m < NF) {
                    if constexpr (m < TM)
                        fa[cur ^ 1][m] = frag(stage + L::A_ROW * BK, wm * WM + m * 32 + lr, ks + 1);
                    else
                        fb[cur ^ 1][m - TM] =
                            frag(stage + L::W_ROW * BK, wn * WN + (m - TM) * 32 + lr, ks + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
            if constexpr (L::SW) {
                half8 bl[TN];
#pragma unroll
                for (int j = 0; j < TN; ++j) bl[j] = frag(stage + L::WLO_ROW * BK, wn * WN + j * 32 + lr, ks);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bl[j], a[i], acc2[i][j], 0, 0, 0);
            }
            if constexpr (L::SA) {
                half8 al[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i) al[i] = frag(stage + L::ALO_ROW * BK, wm * WM + i * 32 + lr, ks);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[j], al[i], acc2[i][j], 0, 0, 0);
            }
        });
    }

    // Wait until tile kt's DMAs (this wave's) have landed. Younger tiles
    // already issued: min(NS - 2, nk - 1 - kt); each is L::LOADS instructions.
    template <int Y>
    __device__ __forceinline__ void wait_younger(int64_t younger) const {
        if constexpr (Y == 0) {
            wait_vmcnt<0>();
        } else {
            if (younger >= Y) { wait_vmcnt<Y * L::LOADS>(); return; }
            wait_younger<Y - 1>(younger);
        }
    }
    __device__ __forceinline__ void wait_tile(int64_t kt) const {
        wait_younger<NS - 2>(nk - 1 - kt);
    }
};

// The tile's epilogue, shared by the pipelined GEMM and the fused FFN
// kernel: bias, activation, residual and the row LayerNorm applied to the
// accumulators of G (a DmaGemm), and the stores. stage_buf(b) returns LDS
// stage buffer b (0 <= b < NS) of SZ halves each, free once the K loop ends.
template <int BM, int BN, int NS, int ACT, int OUTT, int NWV, int LN, int SZ, class G, class BufFn>
__device__ __forceinline__ void store_tile(G& g, BufFn stage_buf, const float* sbias,
                                           const float* __restrict__ R, void* __restrict__ C,
                                           int64_t M, int64_t N, const LnEpi& ln) {
    // Epilogue. The MFMAs were issued as W x A^T, so each 32x32 accumulator
    // holds a tile of C^T: lane l owns C row (l % 32) of the tile, and
    // registers 4g .. 4g+3 hold the four consecutive C columns
    // 8g + 4 (l / 32) + 0..3. Stored from there, one wave instruction would
    // touch 32 rows in 16- or 32-byte pieces (and so would the residual's
    // loads): on MI355X an fp32 output then cost more than the MFMAs of a
    // short-K tile (C4 ffn_in shape: 345 us fp32 out, 272 fp16). So the
    // tile goes through LDS, which the finished K loop leaves free: each
    // wave writes its raw accumulators into the stage buffers, then every
    // thread takes row-contiguous 16-byte chunks -- a wave instruction
    // covers 1 KiB of one row -- adds bias, activation and residual in fp32
    // (the same operations in the same order as per element before), and
    // stores. A 256 x 256 fp32 tile takes two rounds of the 2 x 64 KiB
    // stages. The 16-byte chunks are XOR-swizzled by row (chunk ^ row % 16)
    // so that both the column writes (16 rows a pass) and the row reads are
    // free of bank conflicts.
    using TO = typename std::conditional<
        OUTT == DOTL_F32, float,
        typename std::conditional<OUTT == DOTL_BF16, __bf16, _Float16>::type>::type;
    const bool vec_ok = (N & 3) == 0;
    // The direct epilogue (each lane stores its own runs of 4 columns) for a
    // GELU with a 16-bit output: there the staged one measured no better
    // (C4 ffn_in shape on the 8-wave tile, both with the full-tile paths
    // below: 266-271 us direct, 272-274 staged; C5's equal) and worse on
    // the 4-wave ones, whose waves have no partner to overlap the transpose.
    constexpr bool STAGED = LN >= 0 || !(ACT == DOTL_ACT_GELU && OUTT != DOTL_F32);
    static_assert(LN < 0 || (ACT == DOTL_ACT_NONE && OUTT == DOTL_F32 && BN == 256),
                  "the LayerNorm epilogue: fp32 rows a wave instruction wide");
    if constexpr (!STAGED) {
        // A tile wholly inside C stores without per-row or per-column tests
        // (the same reason as the staged rounds below).
        auto direct = [&](auto fullc) {
            constexpr bool FULL = decltype(fullc)::value;
#pragma unroll
            for (int i = 0; i < G::TM; ++i) {
                const int64_t row = g.m0 + g.wm * G::WM + i * 32 + g.lr;
                if (!FULL && row >= M) continue;
#pragma unroll
                for (int j = 0; j < G::TN; ++j) {
#pragma unroll
                    for (int grp = 0; grp < 4; ++grp) {
                        const int cl = g.wn * G::WN + j * 32 + 8 * grp + 4 * g.lg;  // tile-local column
                        const int64_t col = g.n0 + cl;
                        float v[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float a = g.acc[i][j][4 * grp + e];
                            if constexpr (G::SPLIT) a += g.acc2[i][j][4 * grp + e] * kLoUnscale;
                            a += sbias[cl + e];
                            if constexpr (ACT == DOTL_ACT_GELU) a = gelu_erf<NWV == 8>(a);
                            v[e] = a;
                        }
                        TO* crow = static_cast<TO*>(C) + row * N;
                        if (FULL || (vec_ok && col + 4 <= N)) {
                            store4f(crow + col, make_float4(v[0], v[1], v[2], v[3]));
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (col + e < N) crow[col + e] = from_f32<TO>(v[e]);
                        }
                    }
                }
            }
        };
        if (vec_ok && g.m0 + BM <= M && g.n0 + BN <= N)
            direct(std::integral_constant<bool, true>{});
        else
            direct(std::integral_constant<bool, false>{});
        return;
    } else {
    constexpr int BUF_BYTES = SZ * 2;
    constexpr int ROW_BYTES = BN * 4;
    constexpr int RPB = (BUF_BYTES / ROW_BYTES) / 32 * 32;   // tile rows a stage buffer holds
    constexpr int CPR = BN / 4;                              // 16-byte chunks a row
    static_assert(RPB >= 32, "a stage buffer must hold 32 fp32 tile rows");
    static_assert(CPR >= 16 && (64 % CPR == 0 || CPR % 64 == 0), "row chunks");
    constexpr int RR = RPB * NS;                            // tile rows a round holds
    constexpr int ROUNDS = (BM + RR - 1) / RR;
    constexpr int THREADS = NWV * 64;
    auto buf = [&](int b) -> float* { return reinterpret_cast<float*>(stage_buf(b)); };
    // The LayerNorm epilogue: a wave instruction covers one row (64 lanes x
    // 4 columns), so each lane's columns are the same in every row; their
    // weights are loaded once.
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 lnw = z4, lnb = z4;
    void* normed = nullptr;
    if constexpr (LN >= 0) {
        normed = ln.io != nullptr ? reinterpret_cast<void*>(ln.io[1]) : ln.normed;
        const int64_t lcol = g.n0 + (threadIdx.x & 63) * 4;
        if (lcol < N) {
            lnw = *reinterpret_cast<const float4*>(ln.w + lcol);
            lnb = *reinterpret_cast<const float4*>(ln.b + lcol);
        }
    }
    stage_barrier();   // every wave is done reading the stages
    // A tile wholly inside C (every tile but the right and bottom edges)
    // takes a copy of the rounds with no per-row or per-column tests: its
    // residual loads and stores are then single 16-byte accesses in a
    // straight line, so the compiler can count them and wait only for what
    // each chunk needs instead of draining every store before the next.
    auto rounds = [&](auto kindc) {
        // 2: the tile lies wholly inside C; 1: an edge tile of a C whose rows
        // are whole 16-byte chunks (N % 4 == 0); 0: any other edge tile
        constexpr int KIND = decltype(kindc)::value;
        constexpr bool FULL = KIND == 2;
        constexpr bool VEC = KIND >= 1;
        static_for<0, ROUNDS>([&](auto qq) {
            constexpr int q = decltype(qq)::value;
            constexpr int r_lo = q * RR;
            constexpr int r_hi = (q + 1) * RR < BM ? (q + 1) * RR : BM;
            constexpr int CHUNKS = (r_hi - r_lo) * CPR;
            static_assert(CHUNKS % THREADS == 0, "round chunks");
            constexpr int PER_T = CHUNKS / THREADS;
            // The round's residual, loaded first: its HBM latency then runs
            // under the LDS writes and the barrier instead of stalling the
            // store loop once per batch.
            float4 res[OUTT == DOTL_F32 ? PER_T : 1];
            // and, for a LayerNorm epilogue that scatters its rows, their
            // output rows (one per wave instruction: lanes share the row)
            int32_t orow[LN >= 0 ? PER_T : 1];
            if constexpr (LN >= 0) {
                if (ln.out_row != nullptr) {
#pragma unroll
                    for (int u = 0; u < PER_T; ++u) {
                        const int64_t row = g.m0 + r_lo + (threadIdx.x + u * THREADS) / CPR;
                        orow[u] = ln.out_row[row < M ? row : M - 1];
                    }
                }
            }
            if constexpr (OUTT == DOTL_F32) {
                if (R != nullptr) {
#pragma unroll
                    for (int u = 0; u < PER_T; ++u) {
                        const int c = threadIdx.x + u * THREADS;
                        const int64_t row = g.m0 + r_lo + c / CPR;
                        const int64_t col = g.n0 + (c % CPR) * 4;
                        if constexpr (VEC) {
                            // unconditional: an edge tile's rows past M and
                            // chunks past N read the last row / chunk (those
                            // outputs are never stored), so the loads go out
                            // back to back instead of each behind a branch
                            const int64_t rr = FULL ? row : (row < M ? row : M - 1);
                            const int64_t cc4 = FULL ? col : (col < N - 4 ? col : N - 4);
                            res[u] = *reinterpret_cast<const float4*>(R + rr * N + cc4);
                            continue;
                        }
                        const float* rrow = R + row * N + col;
                        res[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                        if (row < M) {
                            if (vec_ok && col + 4 <= N) {
                                res[u] = *reinterpret_cast<const float4*>(rrow);
                            } else {
                                if (col + 0 < N) res[u].x = rrow[0];
                                if (col + 1 < N) res[u].y = rrow[1];
                                if (col + 2 < N) res[u].z = rrow[2];
                                if (col + 3 < N) res[u].w = rrow[3];
                            }
                        }
                    }
                }
            }
            if constexpr (q > 0) stage_barrier();   // the previous round's reads are done
            // write: this wave's 32-row groups that fall in the round
#pragma unroll
            for (int i = 0; i < G::TM; ++i) {
                const int gb = g.wm * G::WM + i * 32;   // wave-uniform
                if (gb < r_lo || gb >= r_hi) continue;
                const int b = (gb - r_lo) / RPB;
                const int rb = (gb - r_lo) % RPB + g.lr;
                float* base = buf(b) + rb * BN;
#pragma unroll
                for (int j = 0; j < G::TN; ++j) {
#pragma unroll
                    for (int grp = 0; grp < 4; ++grp) {
                        const int chunk = (g.wn * G::WN + j * 32 + 8 * grp) / 4 + g.lg;
                        float4 v;
                        v.x = g.acc[i][j][4 * grp + 0];
                        v.y = g.acc[i][j][4 * grp + 1];
                        v.z = g.acc[i][j][4 * grp + 2];
                        v.w = g.acc[i][j][4 * grp + 3];
                        if constexpr (G::SPLIT) {
                            v.x += g.acc2[i][j][4 * grp + 0] * kLoUnscale;
                            v.y += g.acc2[i][j][4 * grp + 1] * kLoUnscale;
                            v.z += g.acc2[i][j][4 * grp + 2] * kLoUnscale;
                            v.w += g.acc2[i][j][4 * grp + 3] * kLoUnscale;
                        }
                        *reinterpret_cast<float4*>(base + ((chunk ^ (rb & 15)) * 4)) = v;
                    }
                }
            }
            stage_barrier();
            // read + store: row-contiguous chunks of rows [r_lo, r_hi). Chunk
            // u of this thread: its row, its column, and act(acc + bias)
            // (+ residual) from the stage buffer.
            auto value = [&](int u, int64_t& row, int64_t& col) -> float4 {
                const int c = threadIdx.x + u * THREADS;
                const int rl = c / CPR;                 // row within the round
                const int cc = c % CPR;                 // logical chunk
                const int b = rl / RPB;
                const int rb = rl % RPB;
                row = g.m0 + r_lo + rl;
                const int cl = cc * 4;                  // tile-local column
                col = g.n0 + cl;
                const float4 a4 =
                    *reinterpret_cast<const float4*>(buf(b) + rb * BN + ((cc ^ (rb & 15)) * 4));
                float v[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float a = v[e] + sbias[cl + e];
                    if constexpr (ACT == DOTL_ACT_GELU) a = gelu_erf<NWV == 8>(a);
                    v[e] = a;
                }
                if constexpr (OUTT == DOTL_F32) {
                    // residual stream: out = R + act(x W^T + b), the add the
                    // following LayerNorm would otherwise do (same fp32 sum)
                    if (R != nullptr) {
                        v[0] = res[u].x + v[0]; v[1] = res[u].y + v[1];
                        v[2] = res[u].z + v[2]; v[3] = res[u].w + v[3];
                    }
                }
                return make_float4(v[0], v[1], v[2], v[3]);
            };
            if constexpr (LN >= 0) {
                // Each row's LayerNorm, in the LayerNorm kernels' exact
                // arithmetic for a row of <= 256 columns held one float4 a
                // lane (zeros past N): the same sums in the same order, so
                // the normed values are theirs bit for bit. A wave
                // instruction covers one row; the thread's rows go through
                // each step LG at a time, their butterflies interleaved and on
                // permlane / swizzle / DPP exchanges (one row at a time on
                // ds_bpermute, every step waited out an LDS round trip; all of
                // a round's rows at once spilled). Rows past M are reduced too
                // (wave-uniform) and not stored.
                static_assert(CPR == 64, "one row a wave instruction");
                constexpr int LG = PER_T < 4 ? PER_T : 4;
                static_assert(PER_T % LG == 0, "row groups");
                const float inv_d = 1.0f / static_cast<float>(N);
                static_for<0, PER_T / LG>([&](auto gg) {
                    constexpr int U0 = decltype(gg)::value * LG;
                    float4 xv[LG];
                    float mean_est[LG], sd[LG], sd2[LG];
                    int64_t rows_[LG];
                    int64_t col = 0;
#pragma unroll
                    for (int k = 0; k < LG; ++k) {
                        const float4 v4 = value(U0 + k, rows_[k], col);
                        xv[k] = col < N ? v4 : z4;   // N % 4 == 0: whole chunks
                        mean_est[k] = 0.f;
                        mean_est[k] += (xv[k].x + xv[k].y) + (xv[k].z + xv[k].w);
                    }
                    const bool in = col < N;         // this lane's column, every row
                    wave_sum_n(mean_est);
#pragma unroll
                    for (int k = 0; k < LG; ++k) {
                        mean_est[k] *= inv_d;
                        sd[k] = 0.f;
                        sd2[k] = 0.f;
                        if (in) {
                            const float d0 = xv[k].x - mean_est[k], d1 = xv[k].y - mean_est[k];
                            const float d2 = xv[k].z - mean_est[k], d3 = xv[k].w - mean_est[k];
                            sd[k] += (d0 + d1) + (d2 + d3);
                            sd2[k] += ln_sq4(d0, d1, d2, d3);
                        }
                    }
                    {
                        // sd and sd2 reduced together, as the LayerNorm kernels do
                        float both[2 * LG];
#pragma unroll
                        for (int k = 0; k < LG; ++k) { both[2 * k] = sd[k]; both[2 * k + 1] = sd2[k]; }
                        wave_sum_n(both);
#pragma unroll
                        for (int k = 0; k < LG; ++k) { sd[k] = both[2 * k]; sd2[k] = both[2 * k + 1]; }
                    }
#pragma unroll
                    for (int k = 0; k < LG; ++k) {
                        const int64_t row = rows_[k];
                        if (!FULL && row >= M) continue;   // wave-uniform
                        const float delta = sd[k] * inv_d;
                        const float var = ln_var(sd2[k], delta, inv_d);
                        const float rstd = 1.0f / sqrtf(var + ln.eps);
                        if (in) {
                            if constexpr ((LN & 4) != 0)
                                store4f(static_cast<float*>(C) + row * N + col, xv[k]);
                            float4 o;
                            o.x = ln_out(xv[k].x, mean_est[k], delta, rstd, lnw.x, lnb.x);
                            o.y = ln_out(xv[k].y, mean_est[k], delta, rstd, lnw.y, lnb.y);
                            o.z = ln_out(xv[k].z, mean_est[k], delta, rstd, lnw.z, lnb.z);
                            o.w = ln_out(xv[k].w, mean_est[k], delta, rstd, lnw.w, lnb.w);
                            const int64_t nrow = ln.out_row != nullptr ? orow[U0 + k] : row;
                            store_normed4<(LN & 3)>(normed, ln.plane, nrow * N + col, o);
                        }
                    }
                });
            } else {
#pragma unroll
                for (int u = 0; u < PER_T; ++u) {
                    int64_t row, col;
                    // the row test first: a row past M reads nothing
                    const int c = threadIdx.x + u * THREADS;
                    if (!FULL && g.m0 + r_lo + c / CPR >= M) continue;
                    const float4 v4 = value(u, row, col);
                    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
                    TO* crow = static_cast<TO*>(C) + row * N;
                    if (FULL || (VEC && col + 4 <= N)) {
                        store4f(crow + col, v4);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) crow[col + e] = from_f32<TO>(v[e]);
                    }
                }
            }
        });
    };
    if (vec_ok && g.m0 + BM <= M && g.n0 + BN <= N)
        rounds(std::integral_constant<int, 2>{});
    else if (vec_ok)
        rounds(std::integral_constant<int, 1>{});
    else
        rounds(std::integral_constant<int, 0>{});
    }
}

// LN >= 0: the row LayerNorm epilogue (LnEpi; LN & 3 the normed dtype code,
// LN & 4 set when C is stored as well).
template <int BM, int BN, int BK, int NS, int MODE, int ACT, int OUTT, int NWV = 4, int LN = -1>
__global__ __launch_bounds__(NWV * 64) void gemm_dma_kernel(
    const _Float16* __restrict__ A, const _Float16* __restrict__ Alo,
    const _Float16* __restrict__ W, const _Float16* __restrict__ Wlo,
    const float* __restrict__ bias, const float* __restrict__ R, void* __restrict__ C, int64_t M,
    int64_t N, int64_t K, LnEpi ln) {
    using G = DmaGemm<BM, BN, BK, NS, MODE, ACT, OUTT, NWV>;
    using L = typename G::L;
    static_assert(NS >= 2 && NS <= 8, "2 to 8 stages");
    static_assert((NS - 2) * L::LOADS < 64, "vmcnt is 6 bits");
    constexpr int SZ = L::HALVES;

    // One __shared__ array per stage (see the header comment).
    __shared__ __attribute__((aligned(1024))) _Float16 st0[SZ];
    __shared__ __attribute__((aligned(1024))) _Float16 st1[SZ];
    __shared__ __attribute__((aligned(1024))) _Float16 st2[NS > 2 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 st3[NS > 3 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 st4[NS > 4 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 st5[NS > 5 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 st6[NS > 6 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 st7[NS > 7 ? SZ : 8];

    G g;
    g.A = A; g.Alo = Alo; g.W = W; g.Wlo = Wlo;
    g.M = M; g.N = N; g.K = K;
    g.lane = threadIdx.x & 63;
    g.wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    g.wm = g.wave / G::WGN;
    g.wn = g.wave % G::WGN;
    g.lr = g.lane & 31;
    g.lg = g.lane >> 5;
    int64_t mt, nt;
    tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, mt, nt);
    g.m0 = mt * BM;
    g.n0 = nt * BN;
    g.nk = K / BK;
    g.init_offsets();
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
            g.acc[i][j] = floatx16{};
            if constexpr (G::SPLIT) g.acc2[i][j] = floatx16{};
        }

    auto stage = [&](auto s) -> _Float16* {
        constexpr int S = decltype(s)::value;
        if constexpr (S == 0) return st0;
        else if constexpr (S == 1) return st1;
        else if constexpr (S == 2) return st2;
        else if constexpr (S == 3) return st3;
        else if constexpr (S == 4) return st4;
        else if constexpr (S == 5) return st5;
        else if constexpr (S == 6) return st6;
        else return st7;
    };

    // The tile's bias columns, staged in LDS before the K loop (the loop's
    // barriers publish them): read in the epilogue from LDS, they do not wait
    // behind the epilogue's own global stores the way a global load would.
    __shared__ __attribute__((aligned(16))) float sbias[BN];
    for (int c = threadIdx.x; c < BN; c += NWV * 64) {
        const int64_t col = g.n0 + c;
        sbias[c] = col < N ? bias[col] : 0.f;
    }

    // Prologue: tiles 0 .. NS-2 in flight.
    auto prologue = [&](auto s) {
        constexpr int S = decltype(s)::value;
        if constexpr (S < NS - 1) {
            if (S < g.nk) g.template issue_range<0, G::NDMA>(stage(s), S);
        }
    };
    prologue(std::integral_constant<int, 0>{});
    prologue(std::integral_constant<int, 1>{});
    prologue(std::integral_constant<int, 2>{});
    prologue(std::integral_constant<int, 3>{});
    prologue(std::integral_constant<int, 4>{});
    prologue(std::integral_constant<int, 5>{});
    prologue(std::integral_constant<int, 6>{});

    // One step: wait for tile kt (in stage S), barrier (everyone's DMAs for kt
    // landed, everyone done reading the stage tile kt + NS - 1 will reuse),
    // multiply tile kt while issuing tile kt + NS - 1 into stage
    // (S + NS - 1) % NS.
    auto step = [&](auto s, int64_t kt) {
        constexpr int S = decltype(s)::value;
        if constexpr (S < NS) {
            constexpr int NEXT = (S + NS - 1) % NS;
            g.wait_tile(kt);
            stage_barrier();
            g.compute(stage(s), stage(std::integral_constant<int, NEXT>{}), kt + NS - 1,
                      kt + NS - 1 < g.nk, kt > 0);
        }
    };

    int64_t kt = 0;
    for (; kt + NS <= g.nk; kt += NS) {
        step(std::integral_constant<int, 0>{}, kt);
        step(std::integral_constant<int, 1>{}, kt + 1);
        step(std::integral_constant<int, 2>{}, kt + 2);
        step(std::integral_constant<int, 3>{}, kt + 3);
        step(std::integral_constant<int, 4>{}, kt + 4);
        step(std::integral_constant<int, 5>{}, kt + 5);
        step(std::integral_constant<int, 6>{}, kt + 6);
        step(std::integral_constant<int, 7>{}, kt + 7);
    }
    // Remainder: fewer than NS tiles, in stages 0, 1, ...
    if (kt < g.nk) step(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < g.nk) step(std::integral_constant<int, 1>{}, kt + 1);
    if (kt + 2 < g.nk) step(std::integral_constant<int, 2>{}, kt + 2);
    if (kt + 3 < g.nk) step(std::integral_constant<int, 3>{}, kt + 3);
    if (kt + 4 < g.nk) step(std::integral_constant<int, 4>{}, kt + 4);
    if (kt + 5 < g.nk) step(std::integral_constant<int, 5>{}, kt + 5);
    if (kt + 6 < g.nk) step(std::integral_constant<int, 6>{}, kt + 6);
    g.finish();   // the last tile's deferred MFMAs

    auto stage_rt = [&](int b) -> _Float16* {
        _Float16* p = st0;
        if (b == 1) p = st1;
        if constexpr (NS > 2) if (b == 2) p = st2;
        if constexpr (NS > 3) if (b == 3) p = st3;
        if constexpr (NS > 4) if (b == 4) p = st4;
        if constexpr (NS > 5) if (b == 5) p = st5;
        if constexpr (NS > 6) if (b == 6) p = st6;
        if constexpr (NS > 7) if (b == 7) p = st7;
        return p;
    };
    store_tile<BM, BN, NS, ACT, OUTT, NWV, LN, SZ>(g, stage_rt, sbias, R, C, M, N, ln);
}

template <int BM, int BN, int BK, int NS, int MODE, int ACT, int OUTT, int NWV = 4, int LN = -1>
void launch_dma(const DmaArgs& a, const LnEpi& ln = LnEpi{}) {
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, BK, NS, MODE, ACT, OUTT, NWV, LN>),
                       dim3(static_cast<unsigned>(tiles)), dim3(NWV * 64), 0, a.stream, a.A,
                       a.Alo, a.W, a.Wlo, a.bias, a.R, a.C, a.M, a.N, a.K, ln);
}

// Tile ids (dotl_linear's `tile`): 0 128x128, 1 256x128, 2 64x64, 3 256x256,
// 4 128x64. K tiles of 32; stage counts fill <= 144 KiB of LDS.
template <int MODE, int ACT, int OUTT>
bool dispatch_tile(const DmaArgs& a, int tile) {
    // Stage depths are chosen by operand planes a stage holds: 2 + split ones.
    constexpr int PASSES = 1 + (MODE & 1) + ((MODE >> 1) & 1);
    switch (tile) {
        case 0:   // stage: 256 / 384 / 512 rows x 64 B = 16 / 24 / 32 KiB
            if constexpr (PASSES == 1) launch_dma<128, 128, 32, 8, MODE, ACT, OUTT>(a);
            else if constexpr (PASSES == 2) launch_dma<128, 128, 32, 6, MODE, ACT, OUTT>(a);
            else launch_dma<128, 128, 32, 4, MODE, ACT, OUTT>(a);
            return true;
        case 1:   // 384 rows: 24 KiB
            if constexpr (PASSES == 1) { launch_dma<256, 128, 32, 6, MODE, ACT, OUTT>(a); return true; }
            return false;
        case 2:   // 128 / 192 / 256 rows
            if constexpr (PASSES == 1) launch_dma<64, 64, 32, 8, MODE, ACT, OUTT>(a);
            else launch_dma<64, 64, 32, 8, MODE, ACT, OUTT>(a);
            return true;
        case 3:   // 512 rows: 32 KiB
            if constexpr (PASSES == 1) { launch_dma<256, 256, 32, 4, MODE, ACT, OUTT>(a); return true; }
            return false;
        case 4:   // 192 / 320 / 384 rows
            if constexpr (PASSES == 1) launch_dma<128, 64, 32, 8, MODE, ACT, OUTT>(a);
            else if constexpr (PASSES == 2) launch_dma<128, 64, 32, 7, MODE, ACT, OUTT>(a);
            else launch_dma<128, 64, 32, 6, MODE, ACT, OUTT>(a);
            return true;
        // Shallow pipelines whose LDS (<= 72 KiB) lets two workgroups share a
        // CU, i.e. two waves per SIMD, the co-resident one hiding latency.
        case 5:
            if constexpr (PASSES == 1) launch_dma<128, 128, 32, 4, MODE, ACT, OUTT>(a);
            else if constexpr (PASSES == 2) launch_dma<128, 128, 32, 3, MODE, ACT, OUTT>(a);
            else launch_dma<128, 128, 32, 2, MODE, ACT, OUTT>(a);
            return true;
        case 6:
            if constexpr (PASSES == 1) { launch_dma<256, 128, 32, 3, MODE, ACT, OUTT>(a); return true; }
            return false;
        case 7:
            if constexpr (PASSES == 1) launch_dma<128, 64, 32, 4, MODE, ACT, OUTT>(a);
            else launch_dma<128, 64, 32, 3, MODE, ACT, OUTT>(a);
            return true;
        case 8:
            launch_dma<64, 64, 32, 4, MODE, ACT, OUTT>(a);
            return true;
        // BK = 64: each row of a stage is one whole 128-byte line, so every
        // DMA instruction reads 8 full lines instead of 16 half lines.
        case 9:   // 512 rows x 128 B = 64 KiB a stage
            if constexpr (PASSES == 1) { launch_dma<256, 256, 64, 2, MODE, ACT, OUTT>(a); return true; }
            return false;
        case 10:  // 256 / 384 / 512 rows: 32 / 48 / 64 KiB
            if constexpr (PASSES == 1) launch_dma<128, 128, 64, 4, MODE, ACT, OUTT>(a);
            else if constexpr (PASSES == 2) launch_dma<128, 128, 64, 3, MODE, ACT, OUTT>(a);
            else launch_dma<128, 128, 64, 2, MODE, ACT, OUTT>(a);
            return true;
        case 11:  // 384 rows: 48 KiB
            if constexpr (PASSES == 1) { launch_dma<256, 128, 64, 3, MODE, ACT, OUTT>(a); return true; }
            return false;
        case 12:  // two workgroups a CU
            if constexpr (PASSES == 1) { launch_dma<128, 128, 64, 2, MODE, ACT, OUTT>(a); return true; }
            return false;
        case 13:  // 192 / 320 / 384 rows
            if constexpr (PASSES == 1) launch_dma<128, 64, 64, 3, MODE, ACT, OUTT>(a);
            else launch_dma<128, 64, 64, 2, MODE, ACT, OUTT>(a);
            return true;
        // 192x128: fewer, larger tiles where 128-row tiles leave a short
        // second wave of workgroups. 320 / 512 rows: 40 / 64 KiB a stage
        // (three passes would not fit two stages).
        case 14:
            if constexpr (PASSES == 1) { launch_dma<192, 128, 64, 3, MODE, ACT, OUTT>(a); return true; }
            else if constexpr (PASSES == 2) { launch_dma<192, 128, 64, 2, MODE, ACT, OUTT>(a); return true; }
            return false;
        // 8 waves (two per SIMD), each a 128x64 block of the tile.
        case 15:  // 256x256, 128-byte K rows, 2 stages of 64 KiB
            if constexpr (PASSES == 1) { launch_dma<256, 256, 64, 2, MODE, ACT, OUTT, 8>(a); return true; }
            return false;
        case 16:  // 256x256, 64-byte K rows, 4 stages of 32 KiB
            if constexpr (PASSES == 1) { launch_dma<256, 256, 32, 4, MODE, ACT, OUTT, 8>(a); return true; }
            return false;
        case 17:  // 256x128, 128-byte K rows, 3 stages of 48 KiB
            if constexpr (PASSES == 1) { launch_dma<256, 128, 64, 3, MODE, ACT, OUTT, 8>(a); return true; }
            return false;
        case 18:  // 128x256, 128-byte K rows, 3 stages of 48 KiB
            if constexpr (PASSES == 1) { launch_dma<128, 256, 64, 3, MODE, ACT, OUTT, 8>(a); return true; }
            return false;
        case 19:  // 192x128 with 8 waves (each 96x32), split x: 2 stages of 64 KiB
            if constexpr (PASSES == 2) { launch_dma<192, 128, 64, 2, MODE, ACT, OUTT, 8>(a); return true; }
            return false;
    }
    return false;
}

template <int LN>
bool dispatch_tile_ln(const DmaArgs& a, const LnEpi& ln, int tile) {
    // 128x256 only: the 256x256 tile's 128 accumulator registers leave no
    // room for the row reductions (it spilled ~300 registers)
    if (tile == 18) {
        launch_dma<128, 256, 64, 3, 0, DOTL_ACT_NONE, DOTL_F32, 8, LN>(a, ln);
        return true;
    }
    return false;
}

}  // namespace gemm_dma
}  // namespace dotl

// One mode's instances: fp32 output and the mode's 16-bit output (fp16 for
// the fp16 modes 0-3, bf16 for mode 4), with and without GELU.
#define DOTL_GEMM_DMA_INSTANTIATE(M)                                                            \
    namespace dotl {                                                                            \
    namespace gemm_dma {                                                                        \
    template bool dispatch_tile<M, DOTL_ACT_NONE, DOTL_F32>(const DmaArgs&, int);               \
    template bool dispatch_tile<M, DOTL_ACT_NONE, (M == 4 ? DOTL_BF16 : DOTL_F16)>(             \
        const DmaArgs&, int);                                                                   \
    template bool dispatch_tile<M, DOTL_ACT_GELU, DOTL_F32>(const DmaArgs&, int);               \
    template bool dispatch_tile<M, DOTL_ACT_GELU, (M == 4 ? DOTL_BF16 : DOTL_F16)>(             \
        const DmaArgs&, int);                                                                   \
    }                                                                                           \
    }

// The LayerNorm-epilogue instances (one pass): normed fp32, fp16 or split
// planes, with and without C stored.
#define DOTL_GEMM_DMA_INSTANTIATE_LN()                                                          \
    namespace dotl {                                                                            \
    namespace gemm_dma {                                                                        \
    template bool dispatch_tile_ln<DOTL_F32>(const DmaArgs&, const LnEpi&, int);                \
    template bool dispatch_tile_ln<DOTL_F16>(const DmaArgs&, const LnEpi&, int);                \
    template bool dispatch_tile_ln<DOTL_F16X2>(const DmaArgs&, const LnEpi&, int);              \
    template bool dispatch_tile_ln<DOTL_F32 + 4>(const DmaArgs&, const LnEpi&, int);            \
    template bool dispatch_tile_ln<DOTL_F16 + 4>(const DmaArgs&, const LnEpi&, int);            \
    template bool dispatch_tile_ln<DOTL_F16X2 + 4>(const DmaArgs&, const LnEpi&, int);          \
    }                                                                                           \
    }
