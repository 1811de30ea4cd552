// Declarations shared by the pipelined GEMM's translation units: the
// launch arguments and the per-mode tile dispatch (defined in
// gemm_dma_impl.h, instantiated one arithmetic mode per gemm_dma_mode*.hip so
// a full build compiles them in parallel).
#pragma once

#include "dotl_common.h"

namespace dotl {
namespace gemm_dma {

struct DmaArgs {
    const _Float16* A;
    const _Float16* Alo;
    const _Float16* W;
    const _Float16* Wlo;
    const float* bias;
    const float* R;      // nullable fp32 [M, N] residual added to an fp32 output
    void* C;
    int64_t M, N, K;
    hipStream_t stream;
};

// A LayerNorm of each output row, formed in the epilogue (tiles as wide as
// the row): normed = LN(C row) * w + b with the LayerNorm kernels' arithmetic
// (fp32 statistics, the corrected two-pass algorithm), written to `normed`
// at row out_row[r] (or r when out_row is null), split planes `plane`
// elements apart. With `io` (a graph I/O slot) the normed pointer is read
// from io[1] when the kernel runs.
struct LnEpi {
    const float* w;
    const float* b;
    float eps;
    void* normed;
    int64_t plane;
    const int32_t* out_row;
    const int64_t* io;
};

// Launches tile id `tile` for MODE (bit 0 split W, bit 1 split x; 4 bf16
// operands), ACT and the output dtype code (DOTL_F32, DOTL_F16 for modes
// 0-3, DOTL_BF16 for mode 4); false when that tile is not built for the mode.
template <int MODE, int ACT, int OUTT>
bool dispatch_tile(const DmaArgs& a, int tile);

// One pass, no activation, with the row LayerNorm: LN = normed dtype code
// (DOTL_F32, DOTL_F16, DOTL_F16X2) + 4 when C itself is stored too. Tile
// 18 (128x256); N <= 256.
template <int LN>
bool dispatch_tile_ln(const DmaArgs& a, const LnEpi& ln, int tile);

}  // namespace gemm_dma
}  // namespace dotl
