// The pipelined and short-sequence attention kernels for head_dim 32.
#include "attention_dma_impl.h"

DOTL_ATTN_DMA_INSTANTIATE(32)
