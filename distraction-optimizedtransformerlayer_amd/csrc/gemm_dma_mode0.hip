// The pipelined GEMM's instances for arithmetic mode 0: one pass.
#include "gemm_dma_impl.h"

DOTL_GEMM_DMA_INSTANTIATE(0)
