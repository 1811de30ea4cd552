// Dispatch of the LDS-DMA attention kernels by head_dim. The kernels are in
// attention_dma_impl.h, instantiated per head_dim in attention_dma_hd*.hip.
#include "attention_params.h"

namespace dotl {

bool launch_attn_dma(const AttnParams& p, int head_dim, bool out_f32, int nw, int ns,
                     hipStream_t stream) {
    switch (head_dim) {
        case 32: return attn_dma::launch_head_dim<32>(p, out_f32, nw, ns, stream);
        case 64: return attn_dma::launch_head_dim<64>(p, out_f32, nw, ns, stream);
        case 128: return attn_dma::launch_head_dim<128>(p, out_f32, nw, ns, stream);
        default: return false;
    }
}

}  // namespace dotl
