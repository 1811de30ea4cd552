// The pipelined and short-sequence attention kernels for head_dim 128.
#include "attention_dma_impl.h"

DOTL_ATTN_DMA_INSTANTIATE(128)
