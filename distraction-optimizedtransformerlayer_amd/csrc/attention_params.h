// Launch parameters shared by the two attention kernels (attention.hip:
// register-staged, any input dtype; attention_dma.hip: LDS-DMA pipelined,
// fp16 inputs).
#pragma once

#include "dotl_common.h"

namespace dotl {

struct AttnParams {
    const void* q;
    const void* k;
    const void* v;
    int64_t sb, sh, ss;          // q/k/v strides (elements): batch, head, seq
    const uint8_t* mask;         // nullable
    int64_t mb, mh, mq, mk;      // mask strides (elements)
    const int32_t* cu;           // nullable: sequence b is rows [cu[b], cu[b+1]) (packed rows)
    void* out;
    int out_layout;              // 0 [B,H,S,hd], 1 [B,S,H*hd]
    int B, H, S;
    int nqb;                     // query blocks per (b, h)
    int causal;
    float scale_log2;            // scale * log2(e)
    // Split-KV (LDS-DMA kernel only). With splits > 1 the grid is
    // splits x nqb x B*H: split s covers key tiles [s * tiles_per_split,
    // (s + 1) * tiles_per_split) and writes its unnormalised O and its
    // (running max, row sum) per query row to the partial buffers, which
    // attn_split_combine reduces into `out`.
    int splits;                  // 1: no split
    int tiles_per_split;         // key tiles (64 keys) per split
    int64_t part_rows;           // R: B*S, or the packed row count
    float* part_o;               // [splits][R][H][head_dim] fp32
    float2* part_ml;             // [splits][R][H]: (max, log2 domain; sum)
};

// Bytes of split-KV partials for `splits` splits over R rows of H heads.
inline int64_t attn_split_workspace_bytes(int64_t rows, int H, int head_dim, int splits) {
    if (splits <= 1) return 0;
    const int64_t per = rows * H;
    return static_cast<int64_t>(splits) * per * (static_cast<int64_t>(head_dim) * 4 + 8);
}

// Reduces the split partials of p (p.splits > 1) into p.out.
bool launch_attn_split_combine(const AttnParams& p, int head_dim, bool out_f32,
                               hipStream_t stream);

// Wavefronts per workgroup (32 queries each) for a sequence length: enough
// to cover short sequences without idle waves, 4 otherwise.
inline int attn_waves_for(int S) { return S <= 32 ? 1 : (S <= 64 ? 2 : 4); }
inline int attn_query_blocks(int S) {
    const int bm = 32 * attn_waves_for(S);
    return (S + bm - 1) / bm;
}

// The pipelined kernel for fp16 q/k/v with nw waves per workgroup (1, 2 or
// 4; p.nqb must be the matching query-block count) and ns pipeline stages
// (1 to 4, or 0 for the default); false when head_dim is not covered.
bool launch_attn_dma(const AttnParams& p, int head_dim, bool out_f32, int nw, int ns,
                     hipStream_t stream);

namespace attn_dma {
// launch_attn_dma for one head_dim (32, 64 or 128), in attention_dma_hd*.hip.
template <int HD>
bool launch_head_dim(const AttnParams& p, bool out_f32, int nw, int ns, hipStream_t stream);
}  // namespace attn_dma

// The exact fp32 kernel (attention_scalar.hip): q/k/v fp16, bf16 or fp32 (DOTL_*
// codes; bf16 in, bf16 out), any
// head_dim in [1, kMaxScalarHeadDim], `scale` applied to the raw dot
// products. Sizes its own grid (p.nqb is ignored); false when head_dim is
// out of range.
constexpr int kMaxScalarHeadDim = 2048;
bool launch_attn_scalar(const AttnParams& p, int head_dim, int in_dtype, int out_dtype,
                        float scale, hipStream_t stream);
int attn_scalar_query_blocks(int S, int head_dim);

}  // namespace dotl
