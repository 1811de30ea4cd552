// The pipelined GEMM's instances for arithmetic mode 4: bf16 operands, one pass.
#include "gemm_dma_impl.h"

DOTL_GEMM_DMA_INSTANTIATE(4)
