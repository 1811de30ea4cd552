// Dispatch of the LDS-DMA attention kernels by head_dim, and the split-KV
// combine. The attention kernels are in attention_dma_impl.h, instantiated
// per head_dim in attention_dma_hd*.hip.
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

namespace {

// Split-KV combine (replaces reference csrc/attention_wmma.cuh:1783-1826).
// Split s left, per query row and head, O_s unnormalised relative to its
// running max m_s (log2 domain) and its row sum l_s. With M = max_s m_s:
//   out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,
// and 0 when no split saw an allowed key (every m_s = -inf, or the sum is
// 0): the kernels' convention for a fully masked row. One thread per four
// output columns of one (row, head): 16-byte partial reads, the row's
// (m, l) pairs read by the HD / 4 threads that share them (L1 broadcast).
template <int HD, bool OUT_F32>
__global__ __launch_bounds__(256) void attn_split_combine_kernel(AttnParams p) {
    constexpr int C = HD / 4;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t plane = p.part_rows * p.H;
    if (t >= plane * C) return;
    const int c = static_cast<int>(t % C);
    const int64_t rh = t / C;                 // row * H + head
    const int h = static_cast<int>(rh % p.H);
    const int64_t r = rh / p.H;

    float M = -INFINITY;
    for (int s = 0; s < p.splits; ++s) M = fmaxf(M, p.part_ml[s * plane + rh].x);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
    if (M != -INFINITY) {
        for (int s = 0; s < p.splits; ++s) {
            const float2 ml = p.part_ml[s * plane + rh];
            const float w = __builtin_amdgcn_exp2f(ml.x - M);   // 0 for an empty split
            if (w == 0.f) continue;
            const float4 o = *reinterpret_cast<const float4*>(p.part_o + (s * plane + rh) * HD + 4 * c);
            acc.x = fmaf(w, o.x, acc.x);
            acc.y = fmaf(w, o.y, acc.y);
            acc.z = fmaf(w, o.z, acc.z);
            acc.w = fmaf(w, o.w, acc.w);
            den = fmaf(w, ml.y, den);
        }
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    int64_t obase;
    if (p.cu != nullptr || p.out_layout == 1) {
        obase = rh * HD;                      // [rows, H * HD]
    } else {
        const int64_t b = r / p.S, q = r - b * p.S;
        obase = ((b * p.H + h) * p.S + q) * HD;
    }
    const float4 v = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    if constexpr (OUT_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(p.out) + obase + 4 * c) = v;
    } else {
        store4f(static_cast<_Float16*>(p.out) + obase + 4 * c, v);
    }
}

template <int HD>
void launch_combine(const AttnParams& p, bool out_f32, hipStream_t stream) {
    const int64_t threads = p.part_rows * p.H * (HD / 4);
    const unsigned blocks = static_cast<unsigned>((threads + 255) / 256);
    if (out_f32) {
        hipLaunchKernelGGL((attn_split_combine_kernel<HD, true>), dim3(blocks), dim3(256), 0,
                           stream, p);
    } else {
        hipLaunchKernelGGL((attn_split_combine_kernel<HD, false>), dim3(blocks), dim3(256), 0,
                           stream, p);
    }
}

}  // namespace

bool launch_attn_split_combine(const AttnParams& p, int head_dim, bool out_f32,
                               hipStream_t stream) {
    if (p.part_rows <= 0 || p.H <= 0) return true;
    switch (head_dim) {
        case 32: launch_combine<32>(p, out_f32, stream); return true;
        case 64: launch_combine<64>(p, out_f32, stream); return true;
        case 128: launch_combine<128>(p, out_f32, stream); return true;
        default: return false;
    }
}

}  // namespace dotl
