// Flash attention forward on gfx950 MFMA.
//
// Replaces fused_attention_forward (reference csrc/attention_dispatch.cuh:332-519)
// and the tensor-core kernel behind it (reference csrc/attention_wmma.cuh:874-1770):
// softmax(Q K^T * scale  (+ causal / key mask)) V with fp16 operands and fp32
// accumulation and softmax, online (the S x S matrix never exists), a query
// row with no allowed key giving 0, output written straight into either
// [B, H, S, hd] or the [B, S, H*hd] layout out_proj consumes.
//
// MI355X design (not the reference's warp-shaped one):
//   * the score tile is computed TRANSPOSED, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_f16: K is the A operand (32 keys x 16 hd, one
//     16-byte LDS read per lane), Q^T the B operand (held in registers for
//     the whole key loop). In the 32x32 accumulator lane l then owns ONE
//     query (column l%32) and 16 keys, so the running max and the exponent
//     sums are in-lane; only one exchange with lane l^32 per key tile is
//     needed to finish a row maximum -- no quad shuffles per score;
//   * the probabilities never leave registers: the PV product is also
//     transposed, O^T += V^T P^T, and P^T's B-operand layout (lane l: query
//     l%32, 8 keys of lane group l/32) is exactly the score accumulator's
//     layout, so the fp32 -> fp16 narrowing of P is the only work between
//     the two matrix products. The key order inside each 16-key MFMA step is
//     permuted to match (a contraction does not care), and V is fetched in
//     the same permuted order;
//   * V is transposed while it is staged into LDS ([hd][keys]), two keys per
//     32-bit LDS write, so each V^T fragment is two 8-byte LDS reads;
//   * one wavefront per 32 queries, NW wavefronts per workgroup sharing one
//     K/V tile of 64 keys; the next tile's K/V are fetched from HBM into
//     registers while the current tile is multiplied (register double
//     buffering);
//   * causal: key tiles past the workgroup's last query are never visited,
//     and a wavefront skips the arithmetic of tiles wholly in its future;
//     workgroups are numbered so the heaviest (latest) query blocks of every
//     head are dispatched first;
//   * key-only masks ([B,1,1,S] broadcast, the padded-batch case): a tile
//     whose 64 keys are all masked is skipped outright, decided identically
//     by every wavefront from a ballot, so no barrier is needed;
//   * all mask/causal/bounds tests are compiled into a slow path taken only
//     by tiles that need it (boundary, diagonal, or masked tiles).
#include "attention_params.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace dotl {

int attention_fp16_default();
int attention_cp_async_mode();
void attention_pipeline(int* nw, int* ns);
void attention_split_knobs(int* enabled, int* forced);

namespace {

constexpr int kBN = 64;    // keys per tile
constexpr int kVPad = 8;   // halves of padding per V^T row
constexpr int kKPad = 8;   // halves of padding per K row


// MFMA operand type: fp16, or bf16 (fp32 tensors with precision=bf16).
template <bool BF16>
struct Ops;
template <>
struct Ops<false> {
    using E = _Float16;
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    typedef _Float16 v4 __attribute__((ext_vector_type(4)));
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    __device__ __forceinline__ static floatx16 mma(v8 a, v8 b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Ops<true> {
    using E = __bf16;
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    typedef __bf16 v4 __attribute__((ext_vector_type(4)));
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    __device__ __forceinline__ static floatx16 mma(v8 a, v8 b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

// Load 8 consecutive head-dim elements of a TIN tensor as the operand type
// (narrowing fp32 with round-to-nearest-even; 16-bit tensors are read as
// they are, in their own operand type).
template <typename TIN, bool BF16>
__device__ __forceinline__ typename Ops<BF16>::v8 load8(const TIN* p) {
    using O = Ops<BF16>;
    if constexpr (sizeof(TIN) == 4) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        typename O::v8 h;
        h[0] = static_cast<typename O::E>(a.x); h[1] = static_cast<typename O::E>(a.y);
        h[2] = static_cast<typename O::E>(a.z); h[3] = static_cast<typename O::E>(a.w);
        h[4] = static_cast<typename O::E>(b.x); h[5] = static_cast<typename O::E>(b.y);
        h[6] = static_cast<typename O::E>(b.z); h[7] = static_cast<typename O::E>(b.w);
        return h;
    } else {
        static_assert(std::is_same<TIN, typename O::E>::value,
                      "16-bit tensors contract in their own type");
        return *reinterpret_cast<const typename O::v8*>(p);
    }
}

template <int HD, int NW, typename TIN, typename TOUT, bool BF16>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(AttnParams p) {
    using T = TIN;
    using O = Ops<BF16>;
    using E = typename O::E;
    using v8 = typename O::v8;
    using v4 = typename O::v4;
    using v2 = typename O::v2;
    constexpr int NT = NW * 64;
    constexpr int BM = NW * 32;
    constexpr int KS = HD / 16;          // k-steps of the score product
    constexpr int HT = HD / 32;          // 32-row hd tiles of O^T
    constexpr int LDK = HD + kKPad;      // K row pitch (halves)
    constexpr int LDV = kBN + kVPad;     // V^T row pitch (halves)

    __shared__ __attribute__((aligned(16))) E sK[kBN * LDK];
    __shared__ __attribute__((aligned(16))) E sVt[HD * LDV];
    __shared__ uint8_t sMask[kBN];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 31;
    const int lg = lane >> 5;

    // Block numbering: the query-block index is the slowest-varying part so
    // that, under causal masking, the longest blocks of every (b, h) come first.
    const int bh_count = p.B * p.H;
    const int id = blockIdx.x;
    int qb = id / bh_count;
    const int bh = id - qb * bh_count;
    if (p.causal) qb = p.nqb - 1 - qb;
    const int b = bh / p.H;
    const int h = bh - b * p.H;

    const int q_wg0 = qb * BM;
    const int q_w0 = q_wg0 + wave * 32;   // this wavefront's first query
    const int my_q = q_w0 + lr;           // the query this lane's column is

    // Packed rows: this sequence's length and first row. p.S is then the
    // longest sequence (the grid's size); a block past this one's end exits
    // before any barrier, uniformly.
    int S = p.S;
    int64_t seq_off = static_cast<int64_t>(b) * p.sb;
    int64_t row0 = 0;
    if (p.cu != nullptr) {
        row0 = p.cu[b];
        S = p.cu[b + 1] - static_cast<int>(row0);
        seq_off = row0 * p.ss;
        if (q_wg0 >= S) return;
    }

    const T* qbase = static_cast<const T*>(p.q) + seq_off + h * p.sh;
    const T* kbase = static_cast<const T*>(p.k) + seq_off + h * p.sh;
    const T* vbase = static_cast<const T*>(p.v) + seq_off + h * p.sh;

    // Q^T fragments for the whole key loop: lane supplies Q[my_q][ks*16 + lg*8 .. +8].
    v8 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = v8{};
        if (my_q < S) qf[ks] = load8<TIN, BF16>(qbase + static_cast<int64_t>(my_q) * p.ss + ks * 16 + lg * 8);
    }

    const bool has_mask = p.mask != nullptr;
    const bool key_only_mask = has_mask && p.mq == 0;
    const uint8_t* mbase = has_mask ? p.mask + b * p.mb + h * p.mh : nullptr;

    // Key range this workgroup visits.
    int kend = S;
    if (p.causal) kend = min(S, q_wg0 + BM);
    const int nkt = (kend + kBN - 1) / kBN;

    // Live-tile test for a key-only mask: any allowed key in the tile.
    auto tile_live = [&](int kt) -> bool {
        if (!key_only_mask) return true;
        const int key = kt * kBN + lane;
        const bool ok = key < S && mbase[static_cast<int64_t>(key) * p.mk] != 0;
        return __ballot(ok) != 0ull;
    };

    // Staging registers. K: HD/8 chunks per key row, 64 rows.
    constexpr int KCH = kBN * HD / 8;
    constexpr int KPER = (KCH + NT - 1) / NT;
    // V: items are (key pair, 8-wide hd chunk): 32 * HD/8 of them.
    constexpr int VIT = 32 * HD / 8;
    constexpr int VPER = (VIT + NT - 1) / NT;
    v8 rk[KPER];
    v8 rv0[VPER], rv1[VPER];
    uint8_t rm = 0;

    auto fetch = [&](int kt) {
        const int key0 = kt * kBN;
#pragma unroll
        for (int i = 0; i < KPER; ++i) {
            const int c = threadIdx.x + i * NT;
            const int row = c / (HD / 8);
            const int col = (c % (HD / 8)) * 8;
            rk[i] = v8{};
            if (c < KCH && key0 + row < S)
                rk[i] = load8<TIN, BF16>(kbase + static_cast<int64_t>(key0 + row) * p.ss + col);
        }
#pragma unroll
        for (int i = 0; i < VPER; ++i) {
            const int it = threadIdx.x + i * NT;
            const int kp = it & 31;          // key pair
            const int ch = it >> 5;          // hd chunk
            rv0[i] = v8{};
            rv1[i] = v8{};
            if (it < VIT) {
                const int k0 = key0 + 2 * kp;
                if (k0 < S) rv0[i] = load8<TIN, BF16>(vbase + static_cast<int64_t>(k0) * p.ss + ch * 8);
                if (k0 + 1 < S) rv1[i] = load8<TIN, BF16>(vbase + static_cast<int64_t>(k0 + 1) * p.ss + ch * 8);
            }
        }
        if (key_only_mask && threadIdx.x < kBN) {
            const int key = key0 + threadIdx.x;
            rm = (key < S) ? mbase[static_cast<int64_t>(key) * p.mk] : 0;
        }
    };

    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < KPER; ++i) {
            const int c = threadIdx.x + i * NT;
            if (c < KCH) {
                const int row = c / (HD / 8);
                const int col = (c % (HD / 8)) * 8;
                *reinterpret_cast<v8*>(sK + row * LDK + col) = rk[i];
            }
        }
#pragma unroll
        for (int i = 0; i < VPER; ++i) {
            const int it = threadIdx.x + i * NT;
            if (it < VIT) {
                const int kp = it & 31;
                const int ch = it >> 5;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v2 pair;
                    pair[0] = rv0[i][e];
                    pair[1] = rv1[i][e];
                    *reinterpret_cast<v2*>(sVt + (ch * 8 + e) * LDV + 2 * kp) = pair;
                }
            }
        }
        if (key_only_mask && threadIdx.x < kBN) sMask[threadIdx.x] = rm;
    };

    floatx16 o[HT];
#pragma unroll
    for (int j = 0; j < HT; ++j) o[j] = floatx16{};
    float m_run = -INFINITY;   // running max (scaled log2 domain) of this lane's query
    float l_run = 0.f;         // this lane's share of the exponent sum

    // First live tile.
    int kt = 0;
    while (kt < nkt && !tile_live(kt)) ++kt;
    if (kt < nkt) fetch(kt);

    while (kt < nkt) {
        int nxt = kt + 1;
        while (nxt < nkt && !tile_live(nxt)) ++nxt;

        __syncthreads();
        commit();
        __syncthreads();
        if (nxt < nkt) fetch(nxt);

        const int key0 = kt * kBN;
        // A wavefront whose queries all precede this tile has nothing to add.
        const bool wave_active = !p.causal || key0 <= q_w0 + 31;
        if (wave_active) {
            floatx16 s[2];
            s[0] = floatx16{};
            s[1] = floatx16{};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
                    const v8 kf = *reinterpret_cast<const v8*>(sK + (t2 * 32 + lr) * LDK + ks * 16 + lg * 8);
                    s[t2] = O::mma(kf, qf[ks], s[t2]);
                }
            }

            // Scale into the log2 domain, then mask where this tile needs it.
            const bool full = key0 + kBN <= S;
            const bool diag = p.causal && key0 + kBN - 1 > q_w0;
            const bool needs_test = !full || diag || has_mask;
            float tmax = -INFINITY;
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float x = s[t2][r] * p.scale_log2;
                    if (needs_test) {
                        const int kl = t2 * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                        const int key = key0 + kl;
                        bool ok = key < S;
                        if (p.causal) ok = ok && key <= my_q;
                        if (has_mask) {
                            if (key_only_mask) {
                                ok = ok && sMask[kl] != 0;
                            } else if (ok && my_q < S) {
                                ok = mbase[static_cast<int64_t>(my_q) * p.mq +
                                           static_cast<int64_t>(key) * p.mk] != 0;
                            }
                        }
                        if (!ok) x = -INFINITY;
                    }
                    s[t2][r] = x;
                    tmax = fmaxf(tmax, x);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
            const float m_new = fmaxf(m_run, tmax);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
            m_run = m_new;

            float lsum = 0.f;
            v8 pf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float pv = __builtin_amdgcn_exp2f(s[t >> 1][8 * (t & 1) + e] - m_use);
                    lsum += pv;
                    pf[t][e] = static_cast<E>(pv);
                }
            }
            l_run = l_run * corr + lsum;
#pragma unroll
            for (int j = 0; j < HT; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[j][r] *= corr;

            // O^T[hd, q] += V^T[hd, keys] P^T[keys, q]. Key order within MFMA
            // step t: element e of lane group g is key
            // 32*(t/2) + 16*(t%2) + 8*(e/4) + 4*g + e%4.
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int kb = 32 * (t >> 1) + 16 * (t & 1) + 4 * lg;
#pragma unroll
                for (int j = 0; j < HT; ++j) {
                    const E* vrow = sVt + (j * 32 + lr) * LDV + kb;
                    const v4 lo = *reinterpret_cast<const v4*>(vrow);
                    const v4 hi = *reinterpret_cast<const v4*>(vrow + 8);
                    v8 vf;
                    vf[0] = lo[0]; vf[1] = lo[1]; vf[2] = lo[2]; vf[3] = lo[3];
                    vf[4] = hi[0]; vf[5] = hi[1]; vf[6] = hi[2]; vf[7] = hi[3];
                    o[j] = O::mma(vf, pf[t], o[j]);
                }
            }
        }
        kt = nxt;
    }

    // Normalise and store. O^T register r of tile j at lane l: hd row
    // 32*j + 8*(r/4) + 4*g + r%4, query column l%32.
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    if (my_q < S) {
        const int64_t obase =
            p.cu != nullptr
                ? ((row0 + my_q) * p.H + h) * HD
                : (p.out_layout == 1
                       ? ((static_cast<int64_t>(b) * S + my_q) * p.H + h) * HD
                       : ((static_cast<int64_t>(b) * p.H + h) * S + my_q) * HD);
#pragma unroll
        for (int j = 0; j < HT; ++j) {
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int d = 32 * j + 8 * rb + 4 * lg;
                store4f(static_cast<TOUT*>(p.out) + obase + d,
                        make_float4(o[j][4 * rb] * inv, o[j][4 * rb + 1] * inv,
                                    o[j][4 * rb + 2] * inv, o[j][4 * rb + 3] * inv));
            }
        }
    }
}

template <int HD, int NW, typename TIN, typename TOUT, bool BF16>
void launch_attn(const AttnParams& p, hipStream_t stream) {
    const int64_t blocks = static_cast<int64_t>(p.nqb) * p.B * p.H;
    hipLaunchKernelGGL((attn_fwd_kernel<HD, NW, TIN, TOUT, BF16>), dim3(static_cast<unsigned>(blocks)),
                       dim3(NW * 64), 0, stream, p);
}

int waves_for(int S) { return attn_waves_for(S); }

template <int HD, typename TIN, typename TOUT, bool BF16>
void launch_nw(const AttnParams& p, hipStream_t stream) {
    switch (waves_for(p.S)) {
        case 1: launch_attn<HD, 1, TIN, TOUT, BF16>(p, stream); break;
        case 2: launch_attn<HD, 2, TIN, TOUT, BF16>(p, stream); break;
        default: launch_attn<HD, 4, TIN, TOUT, BF16>(p, stream); break;
    }
}

template <typename TIN, typename TOUT, bool BF16>
bool launch_hd(int hd, const AttnParams& p, hipStream_t stream) {
    switch (hd) {
        case 32: launch_nw<32, TIN, TOUT, BF16>(p, stream); return true;
        case 64: launch_nw<64, TIN, TOUT, BF16>(p, stream); return true;
        case 128: launch_nw<128, TIN, TOUT, BF16>(p, stream); return true;
        default: return false;
    }
}

const char* impl_name(int impl) {
    switch (impl) {
        case 0: return "auto";
        case 1: return "scalar";
        case 2: return "wmma";
        case 3: return "tile";
    }
    return "?";
}

const char* precision_name(int prec) {
    switch (prec) {
        case 0: return "auto";
        case 1: return "fp32";
        case 2: return "tf32";
        case 3: return "fp16";
        case 4: return "bf16";
    }
    return "?";
}

}  // namespace
}  // namespace dotl

namespace dotl {
namespace {

// What one call will run: the kernel family and, for the LDS-DMA kernel,
// its workgroup shape and key-range split. Decided from the arguments alone
// (no device access), so dotl_attention_split_plan and the launch agree.
struct AttnPlan {
    bool use_scalar = false;
    int mfma_prec = 3;      // 3 fp16, 4 bf16, 2 tf32 (none on gfx950)
    bool dma = false;       // the LDS-DMA kernel (fp16 q/k/v)
    int nw = 4, ns = 0;
    int splits = 1;
    int tiles_per_split = 0;
};

// Split-KV for the LDS-DMA kernel (reference csrc/attention_wmma.cuh:706-759
// decides its split count from occupancy too). A grid of fewer workgroups
// than the 256 CUs can hold two of leaves CUs idle for the whole kernel:
// then the key range is cut into splits of at least two 64-key tiles, up to
// 16, so the grid reaches ~512 workgroups; a combine pass merges them.
// `requested`: 0 the knobs' choice (forced count, else this heuristic,
// else none when disabled), 1 none, n > 1 that many (capped by the tiles).
int split_count(const AttnPlan& plan, int B, int H, int S, bool masked, int requested) {
    if (!plan.dma || (S <= 32 && requested <= 1)) return 1;
    const int nkt = (S + 63) / 64;
    int want = requested;
    if (want == 0) {
        int enabled = 1, forced = 0;
        attention_split_knobs(&enabled, &forced);
        if (!enabled) return 1;
        if (forced > 0) {
            want = forced;
        } else {
            const int nqb = masked ? (S + 127) / 128 : (S + 32 * plan.nw - 1) / (32 * plan.nw);
            const int64_t blocks = static_cast<int64_t>(nqb) * B * H;
            if (blocks >= 256) return 1;
            want = static_cast<int>((512 + blocks - 1) / blocks);
            want = std::min(want, std::min(16, nkt / 2));
        }
    }
    if (want <= 1) return 1;
    want = std::min(want, nkt);
    const int per = (nkt + want - 1) / want;
    return (nkt + per - 1) / per;
}

int tiles_per_split(int S, int splits) {
    const int nkt = (S + 63) / 64;
    return (nkt + splits - 1) / splits;
}

// Validates the impl x precision request and picks the kernel (the
// reference's vocabulary, csrc/attention_dispatch.cuh:219-304,
// attention_wmma.cuh:2043-2084):
//   * scalar (impl 1) is the exact fp32 kernel and has only fp32;
//   * wmma (impl 2) has no fp32. fp16 tensors contract in fp16 whatever the
//     precision; fp32 tensors narrow to the requested type, "auto" meaning
//     the process-wide fp16 knob (on: fp16, off: tf32). gfx950 has no tf32
//     matrix instruction, so a forced wmma declines tf32; bf16 tensors
//     contract in bf16;
//   * auto (impl 0): fp32 -> scalar; otherwise the MFMA kernel where it
//     covers the head_dim and arithmetic, else the scalar kernel (whose
//     fp32 arithmetic is at least as precise as the request);
//   * "tile" is an NVIDIA programming model with no counterpart here and
//     always reports unavailable.
// Returns DOTL_OK with `plan` filled, or the error/decline code (message set).
int plan_attention(int dtype, int head_dim, int S, int impl, int precision, AttnPlan& plan) {
    if (impl == 3) {
        set_error("fused_attention_forward: impl=3 (tile) is not available in this build: the "
                  "tile programming model has no gfx950 counterpart");
        return DOTL_E_UNSUPPORTED;
    }
    if (impl == 2 && precision == 1) {
        set_error("fused_attention_forward: --attn-impl wmma has no fp32 arithmetic. It supports: "
                  "tf32 (declined on gfx950), fp16, bf16. Note this is the MATH type, not the "
                  "tensor dtype.");
        return DOTL_E_UNSUPPORTED;
    }
    if (impl == 1 && precision != 0 && precision != 1) {
        set_error(std::string("fused_attention_forward: --attn-impl scalar has no ") +
                  precision_name(precision) + " arithmetic. It supports: fp32.");
        return DOTL_E_UNSUPPORTED;
    }
    plan.mfma_prec = 3;
    if (dtype == DOTL_F32) {
        plan.mfma_prec = precision == 0 ? (attention_fp16_default() ? 3 : 2) : precision;
    } else if (dtype == DOTL_BF16) {
        plan.mfma_prec = 4;
    }
    const bool mfma_hd = head_dim == 32 || head_dim == 64 || head_dim == 128;
    const bool mfma_ok = mfma_hd && (plan.mfma_prec == 3 || plan.mfma_prec == 4);
    if (impl == 1 || (impl == 0 && precision == 1)) {
        plan.use_scalar = true;
    } else if (impl == 2) {
        if (!mfma_ok) {
            char buf[320];
            std::snprintf(buf, sizeof(buf),
                          "fused_attention_forward: impl=2 (wmma), precision=%s does not cover "
                          "head_dim=%d%s; the MFMA kernel covers head_dim in {32, 64, 128} with "
                          "fp16 or bf16 operands",
                          precision_name(plan.mfma_prec), head_dim,
                          plan.mfma_prec == 2 ? " (gfx950 has no tf32 matrix instruction)" : "");
            set_error(buf);
            return DOTL_DECLINED;
        }
        plan.use_scalar = false;
    } else {
        plan.use_scalar = !mfma_ok;
    }
    if (plan.use_scalar && head_dim > kMaxScalarHeadDim) {
        char buf[256];
        std::snprintf(buf, sizeof(buf),
                      "fused_attention_forward: impl=%d (%s), precision=%s does not cover "
                      "head_dim=%d; the scalar kernel covers head_dim up to %d",
                      impl, impl_name(impl), precision_name(precision), head_dim,
                      kMaxScalarHeadDim);
        set_error(buf);
        return DOTL_DECLINED;
    }
    plan.nw = waves_for(S);
    plan.ns = 0;
    plan.dma = !plan.use_scalar && dtype == DOTL_F16 && attention_cp_async_mode() != 0;
    if (plan.dma) {
        // The pipelined kernel: 8 waves (256 queries) a workgroup for
        // head_dim 128 from S = 2048, measured 4% faster there than 4.
        if (head_dim == 128 && S >= 2048) plan.nw = 8;
        int fnw = 0, fns = 0;
        attention_pipeline(&fnw, &fns);
        if (fnw == 1 || fnw == 2 || fnw == 4 || fnw == 8) plan.nw = fnw;
        if (fns >= 1 && fns <= 4) plan.ns = fns;
    }
    return DOTL_OK;
}

}  // namespace
}  // namespace dotl

extern "C" int dotl_attention_split_plan(int B, int H, int S, int head_dim, int is_causal,
                                         int dtype, int has_mask, int64_t rows, int impl,
                                         int precision, int splits, int* splits_out,
                                         int64_t* workspace_bytes_out) {
    using namespace dotl;
    (void)is_causal;
    clear_error();
    DOTL_REQUIRE(splits_out != nullptr && workspace_bytes_out != nullptr,
                 "attention_split_plan: null output");
    DOTL_REQUIRE(splits >= 0, "attention_split_plan: negative split count");
    *splits_out = 1;
    *workspace_bytes_out = 0;
    AttnPlan plan;
    const int rc = plan_attention(dtype, head_dim, S, impl, precision, plan);
    if (rc != DOTL_OK) return rc;
    const int n = split_count(plan, B, H, S, has_mask != 0, splits);
    *splits_out = n;
    *workspace_bytes_out = attn_split_workspace_bytes(rows, H, head_dim, n);
    return DOTL_OK;
}

extern "C" int dotl_attention_forward(const void* q, const void* k, const void* v, int dtype,
                                      const int64_t* qkv_strides, const uint8_t* mask,
                                      const int64_t* mask_strides, void* out, int out_dtype,
                                      int out_layout, int B, int H, int S, int head_dim,
                                      int is_causal, double scale, int impl, int precision,
                                      const int32_t* cu_seqlens, int64_t rows, int splits,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(out_layout == 0 || out_layout == 1,
                 "fused_attention_forward: out_layout must be 0 ([B,H,S,head_dim]) or 1 "
                 "([B,S,H*head_dim])");
    DOTL_REQUIRE(impl >= 0 && impl <= 3,
                 "fused_attention_forward: impl must be 0 (auto), 1 (scalar), 2 (wmma) or 3 (tile)");
    DOTL_REQUIRE(precision >= 0 && precision <= 4,
                 "fused_attention_forward: precision must be 0 (auto), 1 (fp32), 2 (tf32), "
                 "3 (fp16) or 4 (bf16)");
    DOTL_REQUIRE(dtype == DOTL_F16 || dtype == DOTL_F32 || dtype == DOTL_BF16,
                 "fused_attention_forward: q/k/v must be float16, bfloat16 or float32");
    DOTL_REQUIRE(out_dtype == dtype || (dtype != DOTL_BF16 && out_dtype != DOTL_BF16 &&
                                        (out_dtype == DOTL_F16 || out_dtype == DOTL_F32)),
                 "fused_attention_forward: out must be float16 or float32 (bfloat16 for "
                 "bfloat16 q/k/v)");
    DOTL_REQUIRE(B >= 0 && H >= 0 && S >= 0 && head_dim > 0,
                 "fused_attention_forward: negative extent");
    DOTL_REQUIRE(qkv_strides != nullptr, "fused_attention_forward: strides required");
    DOTL_REQUIRE(splits >= 0, "fused_attention_forward: negative split count");

    AttnPlan plan;
    const int prc = plan_attention(dtype, head_dim, S, impl, precision, plan);
    if (prc != DOTL_OK) return prc;
    if (B == 0 || H == 0 || S == 0) return DOTL_OK;
    DOTL_REQUIRE(cu_seqlens == nullptr || rows >= 0,
                 "fused_attention_forward: packed sequences need their row count");

    // Split-KV: the requested count resolved as dotl_attention_split_plan
    // does; the partials live in the caller's workspace.
    const int nsplit = split_count(plan, B, H, S, mask != nullptr, splits);
    const int64_t part_rows = cu_seqlens != nullptr ? rows : static_cast<int64_t>(B) * S;
    bool do_split = false;
    if (nsplit > 1) {
        const int64_t need = attn_split_workspace_bytes(part_rows, H, head_dim, nsplit);
        if (workspace != nullptr && workspace_bytes >= need) {
            do_split = part_rows > 0;
        } else if (splits > 1) {
            char buf[200];
            std::snprintf(buf, sizeof(buf),
                          "fused_attention_forward: %d key splits need %lld bytes of "
                          "workspace, %lld given",
                          nsplit, static_cast<long long>(need),
                          static_cast<long long>(workspace_bytes));
            set_error(buf);
            return DOTL_E_INVALID;
        }
    }
    DOTL_REQUIRE(q && k && v && out, "fused_attention_forward: null pointer");
    DOTL_REQUIRE(mask == nullptr || mask_strides != nullptr,
                 "fused_attention_forward: mask strides required with a mask");
    DOTL_REQUIRE(cu_seqlens == nullptr || (mask == nullptr && out_layout == 1),
                 "fused_attention_forward: packed sequences (cu_seqlens) take no mask and "
                 "write the packed [rows, H*head_dim] layout (out_layout 1)");
    const int64_t es = dtype == DOTL_F32 ? 4 : 2;
    const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                            reinterpret_cast<uintptr_t>(v) |
                            static_cast<uintptr_t>(qkv_strides[0] * es) |
                            static_cast<uintptr_t>(qkv_strides[1] * es) |
                            static_cast<uintptr_t>(qkv_strides[2] * es);
    DOTL_REQUIRE(plan.use_scalar || align % 16 == 0,
                 "fused_attention_forward: q/k/v rows must be 16-byte aligned for the MFMA kernel");

    AttnParams p{};
    p.q = q; p.k = k; p.v = v;
    p.sb = qkv_strides[0]; p.sh = qkv_strides[1]; p.ss = qkv_strides[2];
    p.mask = mask;
    if (mask) {
        p.mb = mask_strides[0]; p.mh = mask_strides[1];
        p.mq = mask_strides[2]; p.mk = mask_strides[3];
    }
    p.cu = cu_seqlens;
    p.out = out;
    p.out_layout = out_layout;
    p.B = B; p.H = H; p.S = S;
    p.causal = is_causal ? 1 : 0;
    p.splits = 1;
    const int nw = plan.nw, ns = plan.ns;
    p.nqb = plan.use_scalar ? attn_scalar_query_blocks(S, head_dim) : (S + 32 * nw - 1) / (32 * nw);
    DOTL_REQUIRE(static_cast<int64_t>(p.nqb) * B * H <= 0x7fffffff,
                 "fused_attention_forward: grid too large");
    p.scale_log2 = static_cast<float>(scale * 1.4426950408889634);
    const hipStream_t st = as_stream(stream);

    if (do_split) {
        DOTL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                     "fused_attention_forward: workspace must be 16-byte aligned");
        DOTL_REQUIRE(static_cast<int64_t>(p.nqb) * B * H * nsplit <= 0x7fffffff,
                     "fused_attention_forward: grid too large");
        p.splits = nsplit;
        p.tiles_per_split = tiles_per_split(S, nsplit);
        p.part_rows = part_rows;
        p.part_o = static_cast<float*>(workspace);
        p.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) +
                                              static_cast<int64_t>(nsplit) * part_rows * H *
                                                  head_dim * 4);
    }

    const bool in32 = dtype == DOTL_F32;
    const bool out32 = out_dtype == DOTL_F32;
    bool launched;
    if (plan.use_scalar) {
        launched = launch_attn_scalar(p, head_dim, dtype, out_dtype, static_cast<float>(scale), st);
    } else if (dtype == DOTL_BF16) {
        launched = launch_hd<__bf16, __bf16, true>(head_dim, p, st);
    } else if (in32 && plan.mfma_prec == 4) {
        launched = out32 ? launch_hd<float, float, true>(head_dim, p, st)
                         : launch_hd<float, _Float16, true>(head_dim, p, st);
    } else if (in32) {
        launched = out32 ? launch_hd<float, float, false>(head_dim, p, st)
                         : launch_hd<float, _Float16, false>(head_dim, p, st);
    } else if (plan.dma) {
        // fp16 q/k/v: K/V tiles streamed into LDS asynchronously (the
        // reference's cp_async staging; mode 0 selects the register-staged
        // kernel below).
        launched = launch_attn_dma(p, head_dim, out32, nw, ns, st);
        if (launched && p.splits > 1) {
            const int rc = check_launch("fused_attention_forward");
            if (rc != DOTL_OK) return rc;
            launched = launch_attn_split_combine(p, head_dim, out32, st);
        }
    } else {
        launched = out32 ? launch_hd<_Float16, float, false>(head_dim, p, st)
                         : launch_hd<_Float16, _Float16, false>(head_dim, p, st);
    }
    if (!launched) {
        set_error("fused_attention_forward: no kernel instance for this shape");
        return DOTL_E_INVALID;
    }
    return check_launch("fused_attention_forward");
}

// ---- no-allocation entry point --------------------------------------------
//
// dotl_attention_forward_noalloc: dotl_attention_forward with the split-KV
// partials in a fixed device array of this library instead of a caller
// workspace, for callers that cannot allocate (code under stream capture,
// serving loops that forbid hipMalloc). Every call on one GPU shares that
// GPU's copy of the array; calls that overlap on one GPU race on it.
namespace dotl {
namespace {

constexpr int64_t kNoAllocScratchBytes = 32ll << 20;
constexpr int kMaxDevices = 64;

// The scratch memory. In host code `scratch` names a host-side stand-in, not
// a device address: only the pointer hipGetSymbolAddress returns for the
// current device (kept in g_scratch_ptr) is ever handed to a kernel.
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's scratch address, resolved on the first call on the device
// (with that device current) and kept; nullptr with the error set on failure.
void* scratch_for_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("fused_attention_forward_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr) {
            set_error(std::string("fused_attention_forward_noalloc: hipGetSymbolAddress failed: ") +
                      hipGetErrorString(err));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace dotl

extern "C" int64_t dotl_attention_noalloc_scratch_bytes(void) {
    return dotl::kNoAllocScratchBytes;
}

extern "C" int dotl_attention_forward_noalloc(const void* q, const void* k, const void* v,
                                              int dtype, const int64_t* qkv_strides,
                                              const uint8_t* mask, const int64_t* mask_strides,
                                              void* out, int out_dtype, int out_layout, int B,
                                              int H, int S, int head_dim, int is_causal,
                                              double scale, int impl, int precision,
                                              const int32_t* cu_seqlens, int64_t rows,
                                              int splits, void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(splits >= 0, "fused_attention_forward_noalloc: negative split count");
    const int64_t part_rows = cu_seqlens != nullptr ? rows : static_cast<int64_t>(B) * S;
    // The split count the allocating entry would run, fitted to the scratch:
    // a library choice (splits = 0) drops to the largest count that fits (one
    // split needs no scratch); an explicit count that does not fit is refused.
    int n = 1;
    int64_t need = 0;
    int rc = dotl_attention_split_plan(B, H, S, head_dim, is_causal, dtype, mask != nullptr,
                                       part_rows, impl, precision, splits, &n, &need);
    if (rc != DOTL_OK) return rc;
    if (need > kNoAllocScratchBytes) {
        if (splits > 1) {
            char buf[256];
            std::snprintf(buf, sizeof(buf),
                          "fused_attention_forward_noalloc: %d key splits need %lld bytes of "
                          "scratch, over the %lld bytes this entry point holds per device; ask "
                          "for fewer splits or use dotl_attention_forward with a workspace",
                          n, static_cast<long long>(need),
                          static_cast<long long>(kNoAllocScratchBytes));
            set_error(buf);
            return DOTL_E_INVALID;
        }
        while (n > 1 && attn_split_workspace_bytes(part_rows, H, head_dim, n) >
                            kNoAllocScratchBytes) {
            --n;
        }
    }
    void* ws = nullptr;
    if (n > 1) {
        ws = scratch_for_current_device();
        if (ws == nullptr) return DOTL_E_LAUNCH;
    }
    return dotl_attention_forward(q, k, v, dtype, qkv_strides, mask, mask_strides, out, out_dtype,
                                  out_layout, B, H, S, head_dim, is_causal, scale, impl, precision,
                                  cu_seqlens, rows, n, ws, n > 1 ? kNoAllocScratchBytes : 0,
                                  stream);
}
