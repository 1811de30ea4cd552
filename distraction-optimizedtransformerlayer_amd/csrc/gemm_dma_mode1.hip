// The pipelined GEMM's instances for arithmetic mode 1: split W (fp16x3 on an fp16 x).
#include "gemm_dma_impl.h"

DOTL_GEMM_DMA_INSTANTIATE(1)
