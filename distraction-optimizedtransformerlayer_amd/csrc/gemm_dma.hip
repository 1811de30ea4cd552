// The pipelined GEMM's tile choice and entry point. The kernels are in
// gemm_dma_impl.h, instantiated per arithmetic mode in gemm_dma_mode*.hip.
#include "gemm_dma.h"

namespace dotl {

using gemm_dma::DmaArgs;
using gemm_dma::dispatch_tile;

// Tile choice, from sweeps of every GEMM of the five layer configs on MI355X
// (passes = planes multiplied: 1 + split x + split W):
//   * one pass: 256x256 with 8 waves (tile 15) for K >= 1024 once that
//     gives about a workgroup per CU, or 256x128 with 8 waves (17) where
//     that fills the last wave of workgroups better; else the 128x128
//     two-stage tile (12, two workgroups a CU) when it fills the CUs four
//     times over, or at K <= 1024; else the 128x64 three-stage tile (13),
//     then the 64x64 one (8);
//   * split passes: two passes at K <= 512 on the 192x128 tile (C2's QKV,
//     M = 3487: 228 tiles in one wave instead of a short second wave of
//     128-row tiles, 20.5 vs 23.8 us; C5's: 125.8 vs 130.9 us; at K = 1024
//     and 2048 it loses), with 8 waves (tile 19, two a SIMD: C5's QKV 100
//     vs 110 us for the 4-wave tile 14, C2's 16.6 vs 18.0); else the 128x128
//     tile with 128-byte K rows when it fills the CUs, else the shallow
//     128x64, then 64x64.
int pick_dma_tile(int64_t M, int64_t N, int64_t K, int passes) {
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if (passes == 1) {
        // large products: the 8-wave 256x256 tile (two waves a SIMD hide
        // each other's waits) with the LDS-staged epilogue, measured on
        // MI355X against the 4-wave one: C4 QKV 181 vs 202 us, ffn_in 275 vs
        // 292, ffn_out (+ residual) 241 vs 242, out_proj 78 vs 80.
        // When its tiles leave the last of the waves of 256 workgroups (one
        // a CU) mostly empty, the 256x128 three-stage tile instead: C5's
        // ffn_out (N = 256, 333 tiles: 65% of two waves; 256x128: 666
        // tiles, 87% of three) 83 vs 93 us.
        if (K >= 1024 && tiles(256, 256) >= 240) {
            auto fill = [](int64_t t) { return static_cast<double>(t) / (((t + 255) / 256) * 256); };
            return fill(tiles(256, 128)) > fill(tiles(256, 256)) + 0.1 ? 17 : 15;
        }
        if (tiles(128, 128) >= 960) return 12;
        // a deep K on about one 128x128 tile a CU: the four-stage 128x128
        // tile (C3's ffn_out, K = 4096: 41.2 vs 43.2 us for the 128x64 tile
        // 13; an 8-wave two-stage 128x128 tile measured 46.5)
        if (tiles(128, 128) >= 240 && K >= 4096) return 10;
        // about one 128x128 tile a CU at K = 1024: the three-stage 128x64
        // tile's twice as many workgroups (C3's out_proj, 15.7 vs 18.4 us)
        if (tiles(128, 128) < 320 && tiles(128, 64) >= 480 && K >= 1024) return 13;
        if (tiles(128, 128) >= 240 && K <= 1024) return 12;
        if (tiles(128, 64) >= 200) return 13;
        return 8;
    }
    if (passes == 2 && K <= 512 && tiles(192, 128) >= 200) return 19;
    if (tiles(128, 128) >= 400) return 10;
    if (tiles(128, 64) >= 240) return 7;
    return 8;
}

bool launch_gemm_dma(const _Float16* A, const _Float16* Alo, const _Float16* W,
                     const _Float16* Wlo, const float* bias, const float* R, void* C, int64_t M,
                     int64_t N, int64_t K, int mode, int act, int out_dtype, int tile,
                     hipStream_t stream) {
    const DmaArgs a{A, Alo, W, Wlo, bias, R, C, M, N, K, stream};
    auto by_out = [&](auto m) {
        constexpr int MD = decltype(m)::value;
        constexpr int O16 = MD == 4 ? DOTL_BF16 : DOTL_F16;
        if (out_dtype != DOTL_F32 && out_dtype != O16) return false;
        const bool o32 = out_dtype == DOTL_F32;
        if (act == DOTL_ACT_GELU) {
            return o32 ? dispatch_tile<MD, DOTL_ACT_GELU, DOTL_F32>(a, tile)
                       : dispatch_tile<MD, DOTL_ACT_GELU, O16>(a, tile);
        }
        return o32 ? dispatch_tile<MD, DOTL_ACT_NONE, DOTL_F32>(a, tile)
                   : dispatch_tile<MD, DOTL_ACT_NONE, O16>(a, tile);
    };
    switch (mode) {
        case 0: return by_out(std::integral_constant<int, 0>{});
        case 1: return by_out(std::integral_constant<int, 1>{});
        case 2: return by_out(std::integral_constant<int, 2>{});
        case 3: return by_out(std::integral_constant<int, 3>{});
        case 4: return by_out(std::integral_constant<int, 4>{});
    }
    return false;
}

bool launch_gemm_dma_ln(const _Float16* A, const _Float16* W, const float* bias, const float* R,
                        float* C, int64_t M, int64_t N, int64_t K, const float* ln_w,
                        const float* ln_b, float eps, void* normed, int normed_dtype,
                        int64_t plane, const int32_t* out_row, const int64_t* io, int tile,
                        hipStream_t stream) {
    const DmaArgs a{A, nullptr, W, nullptr, bias, R, C, M, N, K, stream};
    const gemm_dma::LnEpi ln{ln_w, ln_b, eps, normed, plane, out_row, io};
    const bool wc = C != nullptr;
    switch (normed_dtype) {
        case DOTL_F32:
            return wc ? gemm_dma::dispatch_tile_ln<DOTL_F32 + 4>(a, ln, tile)
                      : gemm_dma::dispatch_tile_ln<DOTL_F32>(a, ln, tile);
        case DOTL_F16:
            return wc ? gemm_dma::dispatch_tile_ln<DOTL_F16 + 4>(a, ln, tile)
                      : gemm_dma::dispatch_tile_ln<DOTL_F16>(a, ln, tile);
        case DOTL_F16X2:
            return wc ? gemm_dma::dispatch_tile_ln<DOTL_F16X2 + 4>(a, ln, tile)
                      : gemm_dma::dispatch_tile_ln<DOTL_F16X2>(a, ln, tile);
    }
    return false;
}

}  // namespace dotl
