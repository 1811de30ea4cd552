// The pipelined GEMM's LayerNorm-epilogue instances (one pass, no activation,
// fp32 rows of up to 256 columns).
#include "gemm_dma_impl.h"

DOTL_GEMM_DMA_INSTANTIATE_LN()
