#pragma once
// Flash attention forward for fp16 q/k/v on gfx950, K/V streamed HBM -> LDS
// by LDS-DMA through an NS-stage pipeline.
//
// Same contract as the register-staged kernel in attention.hip (which keeps
// serving fp32 inputs): softmax(Q K^T * scale (+ causal / mask)) V, fp16
// operands, fp32 accumulation and softmax, a query row with no allowed key
// giving 0, packed sequences through cu_seqlens. Replaces the tensor-core
// kernel behind fused_attention_forward (reference
// csrc/attention_wmma.cuh:874-1770).
//
// MI355X design:
//   * scores transposed, S^T = K Q^T (v_mfma_f32_32x32x16_f16, K the A
//     operand from LDS, Q^T the B operand held in registers): lane l owns
//     query l % 32, so row max and sum are in-lane plus one exchange with
//     lane l ^ 32; P^T's B-operand layout is the score accumulator's layout,
//     so P never leaves registers and O^T += V^T P^T follows directly (the
//     key order inside each 16-key step is permuted to match);
//   * K and V tiles (64 keys) land in LDS by global_load_lds_dwordx4, NS
//     stages deep, with no staging registers and one barrier per tile; the
//     wave waits for exactly its own loads of the tile it reads next;
//   * V stays row-major in LDS and the V^T fragments come from
//     ds_read_b64_tr_b16. Measured on gfx950: in each 16-lane group, when
//     lane j points at 4 consecutive 16-bit elements c_j[0..3], lane i
//     receives c_{4e + i/4}[i % 4] for e = 0..3. Lanes 4e..4e+3 pointing at
//     key row kb + e, columns c0 + 4 (j % 4), hand lane i the column c0 + i
//     of keys kb .. kb + 3: the 4 keys of one V^T fragment row;
//   * LDS rows are HD * 2 bytes, 16-byte chunks XOR-swizzled per row so the
//     K fragment reads (16 rows x one chunk per 16 lanes) and the transposed
//     V reads (4 rows x 4 chunks per 16 lanes) are both bank-conflict free;
//     the swizzle is applied on the global side of the DMA;
//   * lazy rescaling: the running maximum moves only when a tile's maximum
//     exceeds it by more than 2^8 (log2 domain 8), so after the first tiles
//     the O^T rescale is skipped; P then stays <= 256, exact to fp16's
//     relative precision, and l and O^T absorb the scale in fp32;
//   * causal: key tiles past the workgroup's last query are never fetched;
//     the heavy query blocks are numbered first (descending) and the light
//     ones after them ascending, so co-resident workgroups pair heavy with
//     light.
#include "attention_params.h"
#include "dotl_dma.h"

// Kernels and launchers in dotl::attn_dma, one head_dim's instances per
// translation unit (attention_dma_hd*.hip, DOTL_ATTN_DMA_INSTANTIATE) so a
// full build compiles them in parallel.
namespace dotl {
namespace attn_dma {

constexpr int kKB = 64;          // keys per tile
constexpr float kLazyTau = 8.f;  // log2-domain growth tolerated before a rescale

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t* lds_fp16x4_ptr;

template <int HD>
struct AttnTile {
    static constexpr int CPR = HD / 8;                        // 16-byte chunks per row
    static constexpr int RPD = 64 / CPR;                      // rows one DMA instruction fills
    static constexpr int R2 = (256 / (HD * 2)) > 0 ? 256 / (HD * 2) : 1;  // rows per 256-byte sweep
    static constexpr int NDMA = kKB / RPD;                    // DMA instructions per operand
    static constexpr int HALVES = kKB * HD;                   // per operand per stage
    // K: 16 consecutive rows read one logical chunk -> 16 distinct bank groups.
    __device__ __forceinline__ static int fk(int r) { return (r / R2) % CPR; }
    // V: 4 consecutive rows read 4 consecutive chunks -> 16 distinct bank groups.
    __device__ __forceinline__ static int fv(int r) {
        if constexpr (CPR < 8) return 0;
        else return 4 * ((r / R2) % (CPR / 4));
    }
};

// Transposed LDS read, kept as a whole vector: extracting its elements one
// by one (the v4i16 form with per-element casts) was miscompiled by this
// toolchain into four copies of element 0; the vector form and a shuffle to
// assemble the fragment compile to the two loads and nothing else.
__device__ __forceinline__ half4 lds_read_tr(const _Float16* p) {
    return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4_ptr)(p)));
}

// MASK: an explicit mask may be present. Its per-element loads hold many
// registers, so unmasked calls (the sequence tail and causal limits are
// compares only) take the variant without that code.
template <int HD, int NW, int NS, bool OUT_F32, bool MASK>
__global__ __launch_bounds__(NW * 64, NW >= 8 ? 1 : 2) void attn_dma_kernel(AttnParams p) {
    using TL = AttnTile<HD>;
    constexpr int KS = HD / 16;            // k-steps of the score product
    constexpr int HT = HD / 32;            // 32-row hd tiles of O^T
    constexpr int NI = 2 * TL::NDMA;       // DMA instructions per stage (K then V)
    static_assert(NI % NW == 0, "DMA instructions split evenly over the waves");
    constexpr int L = NI / NW;             // per wave per stage
    static_assert(NS >= 1 && NS <= 4, "1 to 4 stages");
    static_assert(NS < 2 || (NS - 2) * L < 64, "vmcnt is 6 bits");
    constexpr int SZ = TL::HALVES;

    __shared__ __attribute__((aligned(1024))) _Float16 k0s[SZ];
    __shared__ __attribute__((aligned(1024))) _Float16 v0s[SZ];
    __shared__ __attribute__((aligned(1024))) _Float16 k1s[NS > 1 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 v1s[NS > 1 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 k2s[NS > 2 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 v2s[NS > 2 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 k3s[NS > 3 ? SZ : 8];
    __shared__ __attribute__((aligned(1024))) _Float16 v3s[NS > 3 ? SZ : 8];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lr = lane & 31;
    const int lg = lane >> 5;

    const int bh_count = p.B * p.H;
    int id = blockIdx.x;
    int split = 0;
    if (p.splits > 1) {
        const int per_split = p.nqb * bh_count;
        split = id / per_split;
        id -= split * per_split;
    }
    int qb = id / bh_count;
    const int bh = id - qb * bh_count;
    if (p.causal) {
        // Causal work grows with the query block. The first half of the grid
        // takes the heavy blocks in descending order and the second half the
        // light ones ascending, so blocks id and id + grid/2 -- which the
        // dispatcher places on the same CU when the whole grid is resident --
        // sum to the same work.
        const int half = (p.nqb + 1) / 2;
        qb = qb < half ? p.nqb - 1 - qb : qb - half;
    }
    const int b = bh / p.H;
    const int h = bh - b * p.H;

    const int q_wg0 = qb * (32 * NW);
    const int q_w0 = q_wg0 + wave * 32;
    const int my_q = q_w0 + lr;

    int S = p.S;
    int64_t seq_off = static_cast<int64_t>(b) * p.sb;
    int64_t row0 = 0;
    if (p.cu != nullptr) {
        row0 = p.cu[b];
        S = min(p.cu[b + 1] - static_cast<int>(row0), p.S);
        seq_off = row0 * p.ss;
        if (q_wg0 >= S) return;   // uniform over the workgroup, before any barrier
    }

    const _Float16* qbase = static_cast<const _Float16*>(p.q) + seq_off + h * p.sh;
    const _Float16* kbase = static_cast<const _Float16*>(p.k) + seq_off + h * p.sh;
    const _Float16* vbase = static_cast<const _Float16*>(p.v) + seq_off + h * p.sh;

    half8 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = half8{};
        if (my_q < S)
            qf[ks] = *reinterpret_cast<const half8*>(qbase + static_cast<int64_t>(my_q) * p.ss +
                                                     ks * 16 + lg * 8);
    }
    // Q in registers before the DMA stream starts, so the per-tile waits
    // below count DMAs only.
    wait_vmcnt<0>();

    const bool has_mask = MASK && p.mask != nullptr;
    const bool key_only_mask = has_mask && p.mq == 0;
    const uint8_t* mbase = has_mask ? p.mask + b * p.mb + h * p.mh : nullptr;

    const int kend = p.causal ? min(S, q_wg0 + 32 * NW) : S;
    const int nkt = (kend + kKB - 1) / kKB;
    // This workgroup's key tiles: all of them, or its split's share (empty
    // for a split past the causal limit or the sequence end: the loops then
    // run no tile and the partials record an empty row).
    int kt_begin = 0, kt_end = nkt;
    if (p.splits > 1) {
        kt_begin = split * p.tiles_per_split;
        kt_end = min(nkt, kt_begin + p.tiles_per_split);
    }

    auto kst = [&](auto s) __attribute__((always_inline)) -> _Float16*  {
        constexpr int I = decltype(s)::value;
        if constexpr (I == 0) return k0s;
        else if constexpr (I == 1) return k1s;
        else if constexpr (I == 2) return k2s;
        else return k3s;
    };
    auto vst = [&](auto s) __attribute__((always_inline)) -> _Float16*  {
        constexpr int I = decltype(s)::value;
        if constexpr (I == 0) return v0s;
        else if constexpr (I == 1) return v1s;
        else if constexpr (I == 2) return v2s;
        else return v3s;
    };

    // This wave's share of tile kt's DMAs: instructions wave, wave + NW, ...;
    // 0 .. NDMA-1 fill K rows, NDMA .. 2 NDMA-1 fill V rows. Each lane's
    // byte offset within a tile (row r, swizzled chunk) is fixed, so a full
    // tile is addressed as a scalar base (the tile's first key) plus that
    // offset. The last tile clamps keys past the sequence to its last row
    // (finite data, masked later).
    unsigned lane_off[L];
#pragma unroll
    for (int j = 0; j < L; ++j) {
        const int i = wave + NW * j;
        const bool is_v = i >= TL::NDMA;
        const int r = (is_v ? i - TL::NDMA : i) * TL::RPD + lane / TL::CPR;
        const int lc = (lane % TL::CPR) ^ (is_v ? TL::fv(r) : TL::fk(r));
        lane_off[j] = static_cast<unsigned>((static_cast<int64_t>(r) * p.ss + lc * 8) * 2);
    }
    auto issue_one = [&](auto jj, int kt, _Float16* ks_, _Float16* vs_) __attribute__((always_inline)) {
        constexpr int j = decltype(jj)::value;
        const int key0 = kt * kKB;
        const int i = wave + NW * j;
        const bool is_v = i >= TL::NDMA;
        const int ii = is_v ? i - TL::NDMA : i;
        _Float16* dst = (is_v ? vs_ : ks_) + ii * TL::RPD * HD;
        if (key0 + kKB <= S) {
            const _Float16* base = (is_v ? vbase : kbase) + static_cast<int64_t>(key0) * p.ss;
            dma16_off(base, lane_off[j], dst);
        } else {
            const int r = ii * TL::RPD + lane / TL::CPR;
            const int lc = (lane % TL::CPR) ^ (is_v ? TL::fv(r) : TL::fk(r));
            const int key = min(key0 + r, S - 1);
            dma16((is_v ? vbase : kbase) + static_cast<int64_t>(key) * p.ss + lc * 8, dst);
        }
    };
    auto issue = [&](int kt, _Float16* ks_, _Float16* vs_) __attribute__((always_inline)) {
        static_for<0, L>([&](auto jj) { issue_one(jj, kt, ks_, vs_); });
    };

    floatx16 o[HT];
#pragma unroll
    for (int j = 0; j < HT; ++j) o[j] = floatx16{};
    float m_run = -INFINITY;
    float l_run = 0.f;

    // V^T fragment (key step t, hd tile j) for O^T += V^T P^T: MFMA step t
    // covers keys 32 (t/2) + 16 (t%2) + {8 (e/4) + 4 lg + e%4}, two transposed
    // reads of 4 keys each (rows kb .. kb+3 and kb+8 .. kb+11).
    //
    // Fragment addresses. K fragment (k-step ks, keys 32 t2 + lr) is chunk
    // (2 ks + lg) ^ fk(row) of its row; V^T fragment (t, j) reads rows
    // 16 t + 4 lg + trow (+ 8), chunk (4 j + tchunk) ^ fv(row). fk and fv are
    // periodic in the row with a period dividing 8, and the chunk index terms
    // 2 ks and 4 j occupy bits the lane's own terms leave clear, so every
    // fragment's byte offset within a stage is the lane's first one XOR
    // 32 ks (K) or 64 j (V), plus a constant for t2, t and the second row
    // group. Only the two base offsets stay live across the loop.
    const int trow = (lane & 15) >> 2;
    const int tchunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int thalf = 4 * (lane & 1);
    const unsigned k_off0 = static_cast<unsigned>((lr * HD + ((lg ^ TL::fk(lr)) * 8)) * 2);
    const unsigned v_off0 = static_cast<unsigned>(
        ((4 * lg + trow) * HD + ((tchunk ^ TL::fv(4 * lg + trow)) * 8) + thalf) * 2);
    auto vread = [&](const _Float16* vs_, unsigned vofs, int t, int j) __attribute__((always_inline))
        -> half8 {
        const char* a = reinterpret_cast<const char*>(vs_) + (vofs ^ (64u * j)) + t * (32 * HD);
        const half4 a4 = lds_read_tr(reinterpret_cast<const _Float16*>(a));
        const half4 b4 = lds_read_tr(reinterpret_cast<const _Float16*>(a + 16 * HD));
        return __builtin_shufflevector(a4, b4, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    auto kread = [&](const _Float16* ks_, unsigned kofs, int ks, int t2) __attribute__((always_inline))
        -> half8 {
        const char* a = reinterpret_cast<const char*>(ks_) + (kofs ^ (32u * ks)) + t2 * (64 * HD);
        return *reinterpret_cast<const half8*>(a);
    };

    // One key tile. LDS fragments are read KD k-steps (K) and VD MFMAs (V)
    // ahead of their MFMAs, with scheduling fences holding that order: left
    // to itself the compiler reads each fragment into one register set right
    // before its MFMA, exposing the full LDS latency on every MFMA. `dma(j)`
    // issues this wave's j-th DMA of the tile being refilled; the L of them
    // are spread over the score k-steps instead of leaving every wave of the
    // workgroup queued on the address unit at once after the barrier.
    // `check` (a bool constant): whether the tile can lie wholly after this
    // wave's queries under the causal limit, in which case it is skipped.
    // Tiles that no wave skips run without the test, whose merge of skipped
    // and updated accumulators would otherwise cost a register copy of O^T
    // every tile.
    auto compute = [&](int kt, const _Float16* ks_, const _Float16* vs_, auto&& dma, auto check)
                       __attribute__((always_inline)) {
        const int key0 = kt * kKB;
        if constexpr (decltype(check)::value) {
            if (p.causal && key0 > q_w0 + 31) {   // every query of this wave precedes the tile
                static_for<0, L>(dma);
                return;
            }
        }

        // Opaque per tile, so the compiler derives the addresses here instead
        // of hoisting one register per fragment and stage out of the loop.
        unsigned kofs = k_off0, vofs = v_off0;
        asm volatile("" : "+v"(kofs), "+v"(vofs));

        constexpr int KD = KS < 2 ? KS : 2;
        half8 kf[KS][2];
        static_for<0, KD>([&](auto kk) {
            kf[kk][0] = kread(ks_, kofs, kk, 0);
            kf[kk][1] = kread(ks_, kofs, kk, 1);
        });
        floatx16 s[2];
        s[0] = floatx16{};
        s[1] = floatx16{};
        static_for<0, KS>([&](auto kk) {
            constexpr int ks = decltype(kk)::value;
            if constexpr (ks + KD < KS) {
                kf[ks + KD][0] = kread(ks_, kofs, ks + KD, 0);
                kf[ks + KD][1] = kread(ks_, kofs, ks + KD, 1);
            }
            static_for<0, L>([&](auto jj) {
                if constexpr (decltype(jj)::value * KS / L == ks) dma(jj);
            });
            __builtin_amdgcn_sched_barrier(0);
            s[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks][0], qf[ks], s[0], 0, 0, 0);
            s[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks][1], qf[ks], s[1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        });

        // The first V fragments load while the softmax runs.
        constexpr int NV = 4 * HT;
        constexpr int VD = NV < 4 ? NV : 4;
        half8 vf[NV];
        static_for<0, VD>([&](auto ii) { vf[ii] = vread(vs_, vofs, ii / HT, ii % HT); });
        __builtin_amdgcn_sched_barrier(0);

        // Softmax in the log2 domain with c = scale * log2(e): the maximum is
        // taken over the raw scores and scaled once, and each probability is
        // exp2(fma(s, c, -m)). A non-positive c (possible only through the C
        // ABI) scales the scores first and runs the same code with c = 1.
        float c = p.scale_log2;
        if (!(c > 0.f)) {
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                for (int r = 0; r < 16; ++r) s[t2][r] *= c;
            c = 1.f;
        }
        const bool full = key0 + kKB <= S;
        const bool diag = p.causal && key0 + kKB - 1 > q_w0;
        if (!full || diag || has_mask) {
            uint64_t live = ~0ull;
            if (key_only_mask) {
                const int key = key0 + lane;
                live = __ballot(key < S && mbase[static_cast<int64_t>(key) * p.mk] != 0);
            }
            // Key key0 + 4 lg + c is in range (and not after this lane's
            // query) iff c <= lim: one compare against a literal per score.
            int lim = S - 1 - key0;
            if (p.causal) lim = min(lim, my_q - key0);
            lim -= 4 * lg;
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int cl = t2 * 32 + 8 * (r >> 2) + (r & 3);
                    const int kl = cl + 4 * lg;
                    const int key = key0 + kl;
                    bool ok = cl <= lim;
                    if (has_mask) {
                        if (key_only_mask) {
                            ok = ok && ((live >> kl) & 1ull);
                        } else if (ok && my_q < S) {
                            ok = mbase[static_cast<int64_t>(my_q) * p.mq +
                                       static_cast<int64_t>(key) * p.mk] != 0;
                        }
                    }
                    if (!ok) s[t2][r] = -INFINITY;
                }
            }
        }
        // Row maximum over NCH independent chains (max is exact, so the order
        // does not matter). Four chains cut the dependent depth; measured on
        // MI355X that gains 2-3% at head_dim 128 and loses 1-3% at 64.
        constexpr int NCH = HD >= 128 ? 4 : 1;
        float mx[NCH];
#pragma unroll
        for (int k = 0; k < NCH; ++k) mx[k] = -INFINITY;
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx[r % NCH] = fmaxf(mx[r % NCH], s[t2][r]);
        float tmax = mx[0];
#pragma unroll
        for (int k = 1; k < NCH; ++k) tmax = fmaxf(tmax, mx[k]);
        {
            // Lanes l and l ^ 32 hold the two halves of one query's keys:
            // v_permlane32_swap exchanges the wave's halves in registers.
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax),
                                                             __float_as_uint(tmax), false, false);
            tmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;
        }
        float corr = 1.f;
        if (tmax > m_run + kLazyTau) {
            corr = __builtin_amdgcn_exp2f(m_run - tmax);   // 0 while m_run is -inf
            m_run = tmax;
        }
        const float neg_m = (m_run == -INFINITY) ? 0.f : -m_run;

        // P in fp16 (the PV operand), and its row sum from those same fp16
        // values, two at a time in fp32 (v_dot2_f32_f16 against 1).
        const half2v one2 = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
        float lsum = 0.f;
        half8 pf[4];
        auto make_p = [&](auto tt) __attribute__((always_inline)) {
            constexpr int t = decltype(tt)::value;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                pf[t][e] = to_half(__builtin_amdgcn_exp2f(fmaf(s[t >> 1][8 * (t & 1) + e], c, neg_m)));
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const half2v pr = {pf[t][e], pf[t][e + 1]};
                lsum = __builtin_amdgcn_fdot2(pr, one2, lsum, false);
            }
        };
        if (__any(corr != 1.f)) {
#pragma unroll
            for (int j = 0; j < HT; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[j][r] *= corr;
        }

        // O^T[hd, q] += V^T[hd, keys] P^T[keys, q], key step t outer. P of
        // step t + 1 is formed while the MFMAs of step t run: they do not
        // depend on it, so the wave issues that VALU work in their shadow.
        // The group barriers lay each step out as: per MFMA, the V reads it
        // prefetches, the MFMA, then a share of the next step's P.
        make_p(std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        constexpr int kValuPerMfma = (24 + HT - 1) / HT;
        static_for<0, 4>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            static_for<0, HT>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                constexpr int i = t * HT + j;
                if constexpr (i + VD < NV) vf[i + VD] = vread(vs_, vofs, (i + VD) / HT, (i + VD) % HT);
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i], pf[t], o[j], 0, 0, 0);
            });
            if constexpr (t + 1 < 4) make_p(std::integral_constant<int, t + 1>{});
            static_for<0, HT>([&](auto jj) {
                constexpr int i = t * HT + decltype(jj)::value;
                if constexpr (i + VD < NV) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if constexpr (t + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        l_run = l_run * corr + lsum;
    };
    auto no_dma = [](auto) __attribute__((always_inline)) {};

    // Wait for tile kt's DMAs: younger tiles already issued are
    // min(NS - 2, nkt - 1 - kt), each L instructions.
    auto wait_tile = [&](int kt) __attribute__((always_inline)) {
        const int younger = kt_end - 1 - kt;
        if constexpr (NS >= 4) {
            if (younger >= 2) { wait_vmcnt<2 * L>(); return; }
        }
        if constexpr (NS >= 3) {
            if (younger >= 1) { wait_vmcnt<L>(); return; }
        }
        wait_vmcnt<0>();
    };

    if constexpr (NS == 1) {
        // One stage (short sequences: usually a single tile): load, wait,
        // multiply; a barrier before each refill.
#pragma unroll 1
        for (int kt = kt_begin; kt < kt_end; ++kt) {
            if (kt > kt_begin) stage_barrier();
            issue(kt, k0s, v0s);
            wait_vmcnt<0>();
            stage_barrier();
            compute(kt, k0s, v0s, no_dma, std::true_type{});
        }
    } else {
    auto prologue = [&](auto s) __attribute__((always_inline)) {
        constexpr int I = decltype(s)::value;
        if constexpr (I < NS - 1) {
            if (kt_begin + I < kt_end) issue(kt_begin + I, kst(s), vst(s));
        }
    };
    prologue(std::integral_constant<int, 0>{});
    prologue(std::integral_constant<int, 1>{});
    prologue(std::integral_constant<int, 2>{});

    auto step = [&](auto s, int kt, auto check) __attribute__((always_inline)) {
        constexpr int I = decltype(s)::value;
        if constexpr (I < NS) {
            constexpr int NEXT = (I + NS - 1) % NS;
            wait_tile(kt);
            stage_barrier();
            const bool refill = kt + NS - 1 < kt_end;
            auto dma = [&](auto jj) __attribute__((always_inline)) {
                if (refill)
                    issue_one(jj, kt + NS - 1, kst(std::integral_constant<int, NEXT>{}),
                              vst(std::integral_constant<int, NEXT>{}));
            };
            compute(kt, kst(s), vst(s), dma, check);
        }
    };
    // Tiles every wave computes: all of them, or under the causal limit
    // those up to the first query of the workgroup.
    const int nfree = p.causal ? min(kt_end, (q_wg0 + 31) / kKB + 1) : kt_end;
    const std::false_type all_waves;
    const std::true_type some_waves;
    int kt = kt_begin;
    for (; kt + NS <= nfree; kt += NS) {
        step(std::integral_constant<int, 0>{}, kt, all_waves);
        step(std::integral_constant<int, 1>{}, kt + 1, all_waves);
        step(std::integral_constant<int, 2>{}, kt + 2, all_waves);
        step(std::integral_constant<int, 3>{}, kt + 3, all_waves);
    }
    for (; kt + NS <= kt_end; kt += NS) {
        step(std::integral_constant<int, 0>{}, kt, some_waves);
        step(std::integral_constant<int, 1>{}, kt + 1, some_waves);
        step(std::integral_constant<int, 2>{}, kt + 2, some_waves);
        step(std::integral_constant<int, 3>{}, kt + 3, some_waves);
    }
    if (kt < kt_end) step(std::integral_constant<int, 0>{}, kt, some_waves);
    if (kt + 1 < kt_end) step(std::integral_constant<int, 1>{}, kt + 1, some_waves);
    if (kt + 2 < kt_end) step(std::integral_constant<int, 2>{}, kt + 2, some_waves);
    }

    // Normalise and store: O^T register r of tile j at lane l is hd row
    // 32 j + 8 (r/4) + 4 lg + r%4 of query l%32.
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    if (p.splits > 1) {
        // A split's partial: O unnormalised, with the max it is relative to
        // (equal in lanes l and l ^ 32, which exchanged their tile maxima)
        // and the row sum.
        if (my_q < S) {
            const int64_t r = p.cu != nullptr ? row0 + my_q : static_cast<int64_t>(b) * p.S + my_q;
            const int64_t pr = (static_cast<int64_t>(split) * p.part_rows + r) * p.H + h;
            if (lg == 0) p.part_ml[pr] = make_float2(m_run, l_tot);
            float* po = p.part_o + pr * HD;
#pragma unroll
            for (int j = 0; j < HT; ++j)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    *reinterpret_cast<float4*>(po + 32 * j + 8 * rb + 4 * lg) =
                        make_float4(o[j][4 * rb], o[j][4 * rb + 1], o[j][4 * rb + 2],
                                    o[j][4 * rb + 3]);
        }
        return;
    }
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
                if constexpr (OUT_F32) {
                    const float4 w4 = make_float4(o[j][4 * rb] * inv, o[j][4 * rb + 1] * inv,
                                                  o[j][4 * rb + 2] * inv, o[j][4 * rb + 3] * inv);
                    *reinterpret_cast<float4*>(static_cast<float*>(p.out) + obase + d) = w4;
                } else {
                    half4 w4;
                    w4[0] = to_half(o[j][4 * rb] * inv);
                    w4[1] = to_half(o[j][4 * rb + 1] * inv);
                    w4[2] = to_half(o[j][4 * rb + 2] * inv);
                    w4[3] = to_half(o[j][4 * rb + 3] * inv);
                    *reinterpret_cast<half4*>(static_cast<_Float16*>(p.out) + obase + d) = w4;
                }
            }
        }
    }
}


// Sequences of at most 32 keys (the mass-batch case: 16-token sequences,
// thousands of them). One wavefront per (sequence, head) pair, four
// independent pairs per workgroup and no barriers: K fragments are loaded
// straight from HBM in MFMA layout (like Q), V goes by LDS-DMA into a
// wave-private 32-row tile read back transposed as in the main kernel, and
// the score tile is a single 32x32 accumulator (keys x queries).
//
// Eight waves a SIMD asked of the register allocator: each wave is one short
// dependent chain (loads, two MFMA steps, store), so time goes with how many
// are in flight; head_dim 64 then fits 52 VGPRs instead of 76 (6 waves a
// SIMD) without spilling, bit-identical, C5's 40 000 pairs 37.7 -> 36.8 us.
// (head_dim 128 keeps its 140.)
template <int HD, bool OUT_F32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void attn_short_kernel(AttnParams p) {
    using TL = AttnTile<HD>;
    constexpr int KS = HD / 16;
    constexpr int HT = HD / 32;
    constexpr int ROWS = 32;
    constexpr int SZ = ROWS * HD;                 // halves of V per wave
    constexpr int ND = SZ * 2 / 1024;             // DMA instructions per wave
    __shared__ __attribute__((aligned(1024))) _Float16 vsh[4 * SZ];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lr = lane & 31;
    const int lg = lane >> 5;
    const int pair = blockIdx.x * 4 + wave;
    if (pair >= p.B * p.H) return;   // wave-uniform; this kernel has no barrier
    const int b = pair / p.H;
    const int h = pair - b * p.H;

    int S = p.S;
    int64_t seq_off = static_cast<int64_t>(b) * p.sb;
    int64_t row0 = 0;
    if (p.cu != nullptr) {
        row0 = p.cu[b];
        S = min(p.cu[b + 1] - static_cast<int>(row0), p.S);
        seq_off = row0 * p.ss;
    }
    if (S <= 0) return;

    const _Float16* qbase = static_cast<const _Float16*>(p.q) + seq_off + h * p.sh;
    const _Float16* kbase = static_cast<const _Float16*>(p.k) + seq_off + h * p.sh;
    const _Float16* vbase = static_cast<const _Float16*>(p.v) + seq_off + h * p.sh;
    _Float16* vs = vsh + wave * SZ;

    // V rows 0..15, and 16..31 when the sequence reaches them (keys past the
    // sequence clamped to its last row). Without them the second PV step
    // is skipped: its P is 0 there, and unloaded rows could hold NaNs.
    const bool two_steps = S > 16;
#pragma unroll
    for (int j = 0; j < ND; ++j) {
        if (j < ND / 2 || two_steps) {
            const int r = j * TL::RPD + lane / TL::CPR;
            const int lc = (lane % TL::CPR) ^ TL::fv(r);
            const int key = min(r, S - 1);
            dma16(vbase + static_cast<int64_t>(key) * p.ss + lc * 8, vs + j * TL::RPD * HD);
        }
    }

    const int my_q = lr;
    half8 qf[KS], kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = half8{};
        kf[ks] = half8{};
        if (my_q < S) {
            qf[ks] = *reinterpret_cast<const half8*>(qbase + static_cast<int64_t>(my_q) * p.ss + ks * 16 + lg * 8);
            kf[ks] = *reinterpret_cast<const half8*>(kbase + static_cast<int64_t>(my_q) * p.ss + ks * 16 + lg * 8);
        }
    }
    floatx16 s = {};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks], qf[ks], s, 0, 0, 0);

    float c = p.scale_log2;
    if (!(c > 0.f)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] *= c;
        c = 1.f;
    }
    const bool has_mask = p.mask != nullptr;
    const uint8_t* mbase = has_mask ? p.mask + b * p.mb + h * p.mh : nullptr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * lg + (r & 3);
        bool ok = key < S;
        if (p.causal) ok = ok && key <= my_q;
        if (has_mask && ok && my_q < S)
            ok = mbase[static_cast<int64_t>(my_q) * p.mq + static_cast<int64_t>(key) * p.mk] != 0;
        if (!ok) s[r] = -INFINITY;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave)) * c;
    const float neg_m = (tmax == -INFINITY) ? 0.f : -tmax;
    const half2v one2 = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
    float lsum = 0.f;
    half8 pf[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[t][e] = to_half(__builtin_amdgcn_exp2f(fmaf(s[8 * t + e], c, neg_m)));
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const half2v pr = {pf[t][e], pf[t][e + 1]};
            lsum = __builtin_amdgcn_fdot2(pr, one2, lsum, false);
        }
    }
    const float l_tot = lsum + __shfl_xor(lsum, 32, kWave);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;

    wait_vmcnt<0>();   // this wave's V tile has landed (only this wave reads it)
    floatx16 o[HT];
#pragma unroll
    for (int j = 0; j < HT; ++j) o[j] = floatx16{};
    const int hsel = (lane >> 4) & 1;
    const int trow = (lane & 15) >> 2;
    const int tchunk = 2 * hsel + ((lane & 3) >> 1);
    const int thalf = 4 * (lane & 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        if (t == 1 && !two_steps) break;
        const int ra = 16 * t + 4 * lg + trow;
        const int rb = ra + 8;
#pragma unroll
        for (int j = 0; j < HT; ++j) {
            const int cc = 4 * j + tchunk;
            const half4 a4 = lds_read_tr(vs + ra * HD + ((cc ^ TL::fv(ra)) * 8) + thalf);
            const half4 b4 = lds_read_tr(vs + rb * HD + ((cc ^ TL::fv(rb)) * 8) + thalf);
            const half8 vf = __builtin_shufflevector(a4, b4, 0, 1, 2, 3, 4, 5, 6, 7);
            o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[t], o[j], 0, 0, 0);
        }
    }
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
                if constexpr (OUT_F32) {
                    const float4 w4 = make_float4(o[j][4 * rb] * inv, o[j][4 * rb + 1] * inv,
                                                  o[j][4 * rb + 2] * inv, o[j][4 * rb + 3] * inv);
                    *reinterpret_cast<float4*>(static_cast<float*>(p.out) + obase + d) = w4;
                } else {
                    half4 w4;
                    w4[0] = to_half(o[j][4 * rb] * inv);
                    w4[1] = to_half(o[j][4 * rb + 1] * inv);
                    w4[2] = to_half(o[j][4 * rb + 2] * inv);
                    w4[3] = to_half(o[j][4 * rb + 3] * inv);
                    *reinterpret_cast<half4*>(static_cast<_Float16*>(p.out) + obase + d) = w4;
                }
            }
        }
    }
}

template <int HD, bool OUT_F32>
void launch_short(const AttnParams& p, hipStream_t stream) {
    const int64_t blocks = (static_cast<int64_t>(p.B) * p.H + 3) / 4;
    hipLaunchKernelGGL((attn_short_kernel<HD, OUT_F32>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, p);
}

template <int HD, int NW, int NS, bool OUT_F32>
void launch_one(const AttnParams& p, hipStream_t stream) {
    if (p.mask != nullptr) {
        // Masked calls run one configuration (4 waves, 2 stages) whatever
        // the pipeline choice: the result does not depend on it.
        AttnParams pm = p;
        pm.nqb = (p.S + 127) / 128;
        const int64_t blocks = static_cast<int64_t>(pm.nqb) * p.B * p.H * p.splits;
        hipLaunchKernelGGL((attn_dma_kernel<HD, 4, 2, OUT_F32, true>),
                           dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, pm);
        return;
    }
    const int64_t blocks = static_cast<int64_t>(p.nqb) * p.B * p.H * p.splits;
    hipLaunchKernelGGL((attn_dma_kernel<HD, NW, NS, OUT_F32, false>),
                       dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), 0, stream, p);
}

// Deepest pipeline whose in-flight DMA count fits vmcnt (6 bits).
template <int HD, int NW>
constexpr int max_stages() {
    constexpr int L = 2 * AttnTile<HD>::NDMA / NW;
    return (2 * L < 64) ? 4 : ((L < 64) ? 3 : 2);
}

template <int HD, int NW, int NS, bool OUT_F32>
void launch_capped(const AttnParams& p, hipStream_t stream) {
    constexpr int N = NS < max_stages<HD, NW>() ? NS : max_stages<HD, NW>();
    launch_one<HD, NW, N, OUT_F32>(p, stream);
}

template <int HD, int NS, bool OUT_F32>
void launch_nw(const AttnParams& p, int nw, hipStream_t stream) {
    switch (nw) {
        case 1: launch_capped<HD, 1, NS, OUT_F32>(p, stream); break;
        case 2: launch_capped<HD, 2, NS, OUT_F32>(p, stream); break;
        case 8: launch_capped<HD, 8, NS, OUT_F32>(p, stream); break;
        default: launch_capped<HD, 4, NS, OUT_F32>(p, stream); break;
    }
}

// Pipeline depth: 2 stages (one tile in flight while one is multiplied),
// one when a head_dim <= 64 sequence is a single tile. Measured on MI355X at
// the layer configs, 2 stages beat 3 and 4 at 4 waves a workgroup: at 2
// waves per SIMD the co-resident workgroup hides the load latency, and
// deeper pipelines cost LDS, hence workgroups per CU. The exception is the
// 8-wave workgroup (head_dim 128, long sequences): one workgroup a CU, so
// its own third stage hides the latency.
template <int HD, bool OUT_F32>
void launch_ns(const AttnParams& p, int nw, int ns, hipStream_t stream) {
    if (ns <= 0) ns = nw == 8 ? 3 : ((HD < 128 && p.S <= kKB) ? 1 : 2);
    switch (ns) {
        case 1: launch_nw<HD, 1, OUT_F32>(p, nw, stream); break;
        case 2: launch_nw<HD, 2, OUT_F32>(p, nw, stream); break;
        case 3: launch_nw<HD, 3, OUT_F32>(p, nw, stream); break;
        default: launch_nw<HD, 4, OUT_F32>(p, nw, stream); break;
    }
}

// Either kernel for head_dim HD: the short one for sequences of <= 32 keys
// at the default pipeline, else the pipelined one.
template <int HD>
bool launch_head_dim(const AttnParams& p, bool out_f32, int nw, int ns, hipStream_t stream) {
    if (p.S <= 32 && nw == attn_waves_for(p.S) && ns == 0 && p.splits <= 1) {
        out_f32 ? launch_short<HD, true>(p, stream) : launch_short<HD, false>(p, stream);
        return true;
    }
    out_f32 ? launch_ns<HD, true>(p, nw, ns, stream) : launch_ns<HD, false>(p, nw, ns, stream);
    return true;
}

}  // namespace attn_dma
}  // namespace dotl

#define DOTL_ATTN_DMA_INSTANTIATE(HD)                                                         \
    namespace dotl {                                                                          \
    namespace attn_dma {                                                                      \
    template bool launch_head_dim<HD>(const AttnParams&, bool, int, int, hipStream_t);        \
    }                                                                                         \
    }
