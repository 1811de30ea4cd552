// The pipelined GEMM's instances for arithmetic mode 3: split x and W (fp16x3 on split planes).
#include "gemm_dma_impl.h"

DOTL_GEMM_DMA_INSTANTIATE(3)
