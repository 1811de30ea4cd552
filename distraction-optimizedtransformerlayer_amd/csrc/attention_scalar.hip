// Exact fp32 attention: what fused_attention_forward runs for impl=1
// ("scalar") and for precision=fp32 (reference csrc/attention_scalar.cuh:90-248
// through launch_scalar, csrc/attention_dispatch.cuh:102-117), and the
// fallback of impl=0 for head dims the MFMA kernels do not cover. Any
// head_dim from 1 to 2048; q/k/v fp16 or fp32 (widened on load), every
// product and sum in fp32 FMA, exp from the accurate expf.
//
// MI355X design. Plain VALU arithmetic, so the job is keeping the 64 lanes
// busy without cross-lane work per score:
//   * a key tile is 64 keys, one per lane: lane j accumulates the full dot
//     product of key j with each of the wave's Q queries (q broadcast from
//     LDS, four floats per read), so a score costs no shuffle; the online
//     softmax then reduces across the wave once per tile and query;
//   * for P V the lanes switch roles: lane d owns output dimension d of each
//     64-wide head-dim chunk and sweeps the tile's 64 probabilities
//     (broadcast from LDS) against its column of the V chunk;
//   * the head dimension is streamed through LDS in chunks of 64, so one
//     kernel shape serves head_dim up to 2048 with 16 KiB K and V tiles; the
//     chunks per lane (HDC) fix the register budget of the output
//     accumulator, and Q (queries per wave) shrinks as HDC grows.
#include "attention_params.h"

namespace dotl {

namespace {

constexpr int kWaves = 4;
constexpr int kKT = 64;          // keys per tile
constexpr int kDC = 64;          // head-dim chunk
constexpr int kKP = kDC + 4;     // K chunk row pitch (floats): rows read one per lane

template <typename T>
__device__ __forceinline__ float widen(T v) {
    return static_cast<float>(v);
}

template <int HDC, int Q, typename T, typename TO>
__global__ __launch_bounds__(kWaves * 64) void attn_scalar_kernel(AttnParams p, int hd,
                                                                  float scale) {
    __shared__ __attribute__((aligned(16))) float sK[kKT * kKP];
    __shared__ __attribute__((aligned(16))) float sV[kKT * kDC];
    __shared__ __attribute__((aligned(16))) float sQ[kWaves][Q][kDC];
    __shared__ __attribute__((aligned(16))) float sP[kWaves][Q][kKT];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int BQ = kWaves * Q;   // queries per workgroup

    // Query-block index slowest, reversed under causal masking so the
    // longest blocks of every (b, h) are dispatched first.
    const int bh_count = p.B * p.H;
    int qb = blockIdx.x / bh_count;
    const int bh = blockIdx.x - qb * bh_count;
    if (p.causal) qb = p.nqb - 1 - qb;
    const int b = bh / p.H;
    const int h = bh - b * p.H;
    const int q_wg0 = qb * BQ;
    const int q_w0 = q_wg0 + wave * Q;

    int S = p.S;
    int64_t seq_off = static_cast<int64_t>(b) * p.sb;
    int64_t row0 = 0;
    if (p.cu != nullptr) {
        row0 = p.cu[b];
        S = p.cu[b + 1] - static_cast<int>(row0);
        seq_off = row0 * p.ss;
        if (q_wg0 >= S) return;   // whole workgroup, before any barrier
    }
    const T* qbase = static_cast<const T*>(p.q) + seq_off + h * p.sh;
    const T* kbase = static_cast<const T*>(p.k) + seq_off + h * p.sh;
    const T* vbase = static_cast<const T*>(p.v) + seq_off + h * p.sh;
    const uint8_t* mbase = p.mask ? p.mask + b * p.mb + h * p.mh : nullptr;

    int kend = S;
    if (p.causal) kend = min(S, q_wg0 + BQ);
    const int nkt = (kend + kKT - 1) / kKT;

    float o[Q][HDC];
    float m_run[Q], l_run[Q];
#pragma unroll
    for (int qi = 0; qi < Q; ++qi) {
        m_run[qi] = -INFINITY;
        l_run[qi] = 0.f;
#pragma unroll
        for (int c = 0; c < HDC; ++c) o[qi][c] = 0.f;
    }

    for (int kt = 0; kt < nkt; ++kt) {
        const int key0 = kt * kKT;
        const int key = key0 + lane;

        // ---- scores: lane = key, the head dimension in chunks -------------------
        float s[Q];
#pragma unroll
        for (int qi = 0; qi < Q; ++qi) s[qi] = 0.f;
#pragma unroll
        for (int c = 0; c < HDC; ++c) {
            __syncthreads();   // every wave is done with the previous chunk
#pragma unroll
            for (int i = 0; i < kKT * kDC / (kWaves * 64); ++i) {
                const int idx = threadIdx.x + i * kWaves * 64;
                const int r = idx / kDC;
                const int d = idx % kDC;
                const int kk = key0 + r;
                const int dd = c * kDC + d;
                sK[r * kKP + d] = (kk < S && dd < hd)
                                      ? widen(kbase[static_cast<int64_t>(kk) * p.ss + dd])
                                      : 0.f;
            }
#pragma unroll
            for (int qi = 0; qi < Q; ++qi) {
                const int qq = q_w0 + qi;
                const int dd = c * kDC + lane;
                sQ[wave][qi][lane] = (qq < S && dd < hd)
                                         ? widen(qbase[static_cast<int64_t>(qq) * p.ss + dd])
                                         : 0.f;
            }
            __syncthreads();
#pragma unroll 4
            for (int d = 0; d < kDC; d += 4) {
                const float4 kv = *reinterpret_cast<const float4*>(sK + lane * kKP + d);
#pragma unroll
                for (int qi = 0; qi < Q; ++qi) {
                    const float4 qv = *reinterpret_cast<const float4*>(&sQ[wave][qi][d]);
                    float a = s[qi];
                    a = fmaf(qv.x, kv.x, a);
                    a = fmaf(qv.y, kv.y, a);
                    a = fmaf(qv.z, kv.z, a);
                    a = fmaf(qv.w, kv.w, a);
                    s[qi] = a;
                }
            }
        }

        // ---- mask, online softmax (one wave reduction per query) ----------------
        float corr[Q];
#pragma unroll
        for (int qi = 0; qi < Q; ++qi) {
            const int qq = q_w0 + qi;
            bool ok = key < S && qq < S;
            if (p.causal) ok = ok && key <= qq;
            if (mbase != nullptr && ok)
                ok = mbase[static_cast<int64_t>(qq) * p.mq + static_cast<int64_t>(key) * p.mk] != 0;
            const float x = ok ? s[qi] * scale : -INFINITY;
            const float m_new = fmaxf(m_run[qi], wave_max(x));
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            corr[qi] = expf(m_run[qi] - m_use);
            const float pv = expf(x - m_use);
            l_run[qi] = l_run[qi] * corr[qi] + wave_sum(pv);
            m_run[qi] = m_new;
            sP[wave][qi][lane] = pv;
        }
#pragma unroll
        for (int qi = 0; qi < Q; ++qi)
#pragma unroll
            for (int c = 0; c < HDC; ++c) o[qi][c] *= corr[qi];

        // ---- P V: lane = output dimension within the chunk ----------------------
#pragma unroll
        for (int c = 0; c < HDC; ++c) {
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kKT * kDC / (kWaves * 64); ++i) {
                const int idx = threadIdx.x + i * kWaves * 64;
                const int r = idx / kDC;
                const int d = idx % kDC;
                const int kk = key0 + r;
                const int dd = c * kDC + d;
                sV[r * kDC + d] = (kk < S && dd < hd)
                                      ? widen(vbase[static_cast<int64_t>(kk) * p.ss + dd])
                                      : 0.f;
            }
            __syncthreads();
#pragma unroll 4
            for (int j = 0; j < kKT; j += 4) {
                const float v0 = sV[(j + 0) * kDC + lane];
                const float v1 = sV[(j + 1) * kDC + lane];
                const float v2 = sV[(j + 2) * kDC + lane];
                const float v3 = sV[(j + 3) * kDC + lane];
#pragma unroll
                for (int qi = 0; qi < Q; ++qi) {
                    const float4 pp = *reinterpret_cast<const float4*>(&sP[wave][qi][j]);
                    float a = o[qi][c];
                    a = fmaf(pp.x, v0, a);
                    a = fmaf(pp.y, v1, a);
                    a = fmaf(pp.z, v2, a);
                    a = fmaf(pp.w, v3, a);
                    o[qi][c] = a;
                }
            }
        }
    }

    // ---- normalise and store (a query with no allowed key gives 0) --------------
#pragma unroll
    for (int qi = 0; qi < Q; ++qi) {
        const int qq = q_w0 + qi;
        if (qq >= S) continue;
        const float inv = l_run[qi] > 0.f ? 1.0f / l_run[qi] : 0.f;
        const int64_t obase =
            p.cu != nullptr
                ? ((row0 + qq) * p.H + h) * hd
                : (p.out_layout == 1
                       ? ((static_cast<int64_t>(b) * S + qq) * p.H + h) * hd
                       : ((static_cast<int64_t>(b) * p.H + h) * S + qq) * hd);
#pragma unroll
        for (int c = 0; c < HDC; ++c) {
            const int dd = c * kDC + lane;
            if (dd >= hd) continue;
            const float v = o[qi][c] * inv;
            static_cast<TO*>(p.out)[obase + dd] = from_f32<TO>(v);
        }
    }
}

template <int HDC, int Q, typename T, typename TO>
void launch_q(AttnParams p, int hd, float scale, hipStream_t stream) {
    constexpr int BQ = kWaves * Q;
    p.nqb = (p.S + BQ - 1) / BQ;
    const int64_t blocks = static_cast<int64_t>(p.nqb) * p.B * p.H;
    hipLaunchKernelGGL((attn_scalar_kernel<HDC, Q, T, TO>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kWaves * 64), 0, stream, p, hd,
                       scale);
}

template <typename T, typename TO>
bool launch_hdc(const AttnParams& p, int hd, float scale, hipStream_t stream) {
    const int hdc = (hd + kDC - 1) / kDC;
    if (hdc <= 1) launch_q<1, 8, T, TO>(p, hd, scale, stream);
    else if (hdc <= 2) launch_q<2, 8, T, TO>(p, hd, scale, stream);
    else if (hdc <= 4) launch_q<4, 8, T, TO>(p, hd, scale, stream);
    else if (hdc <= 8) launch_q<8, 4, T, TO>(p, hd, scale, stream);
    else if (hdc <= 16) launch_q<16, 2, T, TO>(p, hd, scale, stream);
    else if (hdc <= 32) launch_q<32, 1, T, TO>(p, hd, scale, stream);
    else return false;
    return true;
}

}  // namespace

int attn_scalar_query_blocks(int S, int head_dim) {
    const int hdc = (head_dim + kDC - 1) / kDC;
    const int q = hdc <= 4 ? 8 : (hdc <= 8 ? 4 : (hdc <= 16 ? 2 : 1));
    const int bq = kWaves * q;
    return (S + bq - 1) / bq;
}

bool launch_attn_scalar(const AttnParams& p, int head_dim, int in_dtype, int out_dtype,
                        float scale, hipStream_t stream) {
    if (head_dim < 1 || head_dim > kMaxScalarHeadDim) return false;
    const bool out32 = out_dtype == DOTL_F32;
    switch (in_dtype) {
        case DOTL_F32:
            return out32 ? launch_hdc<float, float>(p, head_dim, scale, stream)
                         : launch_hdc<float, _Float16>(p, head_dim, scale, stream);
        case DOTL_F16:
            return out32 ? launch_hdc<_Float16, float>(p, head_dim, scale, stream)
                         : launch_hdc<_Float16, _Float16>(p, head_dim, scale, stream);
        case DOTL_BF16:
            return launch_hdc<__bf16, __bf16>(p, head_dim, scale, stream);
        default:
            return false;
    }
}

}  // namespace dotl
