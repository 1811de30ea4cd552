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

// Launches tile id `tile` for MODE (bit 0 split W, bit 1 split x; 4 bf16
// operands), ACT and the output dtype code (DOTL_F32, DOTL_F16 for modes
// 0-3, DOTL_BF16 for mode 4); false when that tile is not built for the mode.
template <int MODE, int ACT, int OUTT>
bool dispatch_tile(const DmaArgs& a, int tile);

}  // namespace gemm_dma
}  // namespace dotl
