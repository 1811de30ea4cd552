// The pipelined GEMM's instances for arithmetic mode 2: split x (fp16x2).
#include "gemm_dma_impl.h"

DOTL_GEMM_DMA_INSTANTIATE(2)
