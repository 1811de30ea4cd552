// Residual add + LayerNorm, and plain LayerNorm, for gfx950.
//
// Optional row index (the packed-row path of a padded batch): output row t
// reads input row row_index[t] of x and sub -- a gather when the output
// holds the packed valid rows, a scatter-back when it holds the padded
// layout -- and an entry outside [0, in_rows) writes zeros to every output
// of row t (the padded rows the reference zeroes with masked_fill).
//
// Replaces fused_add_layernorm / fused_layernorm (reference
// csrc/add_layernorm.cuh:491-692). Same contract: x_new = x + sub, normed =
// (x_new - mean) * rsqrt(var + eps) * w + b with the biased variance, fp32
// statistics, the normed output optionally narrowed to fp16 with RNE, or
// split into fp16 hi/lo planes for the fp16x3 GEMM that consumes it.
//
// Layout and mapping (MI355X):
//   * one 64-lane wavefront per row, the whole row held in registers, so the
//     row is read from HBM exactly once and both statistics passes run on
//     registers -- the traffic is the algorithmic minimum: 4 B/elem read of x
//     (+4 of sub), 4 B/elem write of x_new, 4 or 2 B/elem write of normed;
//   * 16-byte loads and stores: lane `l` owns float4 chunks l, l+64, l+128...
//     of the row, so each wave instruction moves 1 KiB of consecutive bytes;
//   * 4 wavefronts (4 rows) per 256-thread workgroup, and the row loop is
//     grid-strided so the grid can be capped near the resident-wave limit;
//   * statistics: the corrected two-pass algorithm (Chan, Golub & LeVeque):
//     an estimate m of the mean, then the centred sums sum(d), sum(d^2) with
//     d = x - m, giving mean = m + sum(d)/D and var = sum(d^2)/D - (sum(d)/D)^2;
//     the output uses (x - m) - sum(d)/D, never a rounded m + sum(d)/D.
//     It stays accurate for rows whose mean is large against their spread
//     (reference csrc/add_layernorm.cuh:168-207 uses the same algorithm).
//     Both sums are reduced in one butterfly over the wavefront.
#include "dotl_common.h"

namespace dotl {
namespace {

constexpr int kRowsPerBlock = 4;

// Graph I/O slot (optional): io[0] replaces the x pointer when bit 0 of
// io_mode is set, io[1] the normed pointer when bit 1 is. A captured graph
// bakes in the slot's address, not the tensors', so each replay reads the
// caller's input and writes the caller's output where the slot points.
#define DOTL_LN_RESOLVE_IO()                                                \
    do {                                                                    \
        if (io_mode & 1) x = reinterpret_cast<const TI*>(io[0]);            \
        if (io_mode & 2) normed = reinterpret_cast<void*>(io[1]);           \
    } while (0)

// x (+ sub), as the tensor dtype holds the sum: x_new = TI(x + sub).
template <typename TI, bool HAS_SUB>
__device__ __forceinline__ float4 load_sum4(const TI* __restrict__ x, const TI* __restrict__ sub,
                                            int64_t off) {
    float4 a = load4f(x + off);
    if constexpr (HAS_SUB) {
        const float4 s = load4f(sub + off);
        a.x = round_via<TI>(a.x + s.x); a.y = round_via<TI>(a.y + s.y);
        a.z = round_via<TI>(a.z + s.z); a.w = round_via<TI>(a.w + s.w);
    }
    return a;
}

template <int NORMED>
__device__ __forceinline__ void store_normed1(void* __restrict__ normed, int64_t plane,
                                              int64_t off, float o) {
    using TO = typename normed_type<NORMED>::type;
    TO* out = static_cast<TO*>(normed);
    if constexpr (NORMED != DOTL_F32) opaque(o);
    if constexpr (NORMED == DOTL_F16X2) {
        const _Float16 h = to_half(o);
        out[off] = h;
        out[plane + off] = split_lo(o, h);
    } else {
        out[off] = from_f32<TO>(o);
    }
}

// Vector path: D % 4 == 0 and D <= 256 * CH. Chunk c of lane l covers row
// elements [4 * (c * 64 + l), +4): 16-byte accesses for fp32, 8-byte for
// the 16-bit types.
//
// Each wave takes RPW rows per iteration: their row indices, then all their
// loads, are issued before any reduction, and the RPW butterflies
// interleave. Up to 1024 columns the weight and bias chunks are loaded once
// per wave, not per row. Measured on MI355X at the configs' shapes: two rows
// a wave at D <= 256 (C5's gathered norm1 54.5 -> 46.1 us, norm2 54.8 ->
// 52.7, the scattering final norm 78.0 -> 68.9), one above; more rows lose
// (fewer waves, and the last round of resident waves runs part-empty: four
// at D = 256 gave 47.3 / 56.7 / 71.7 us, eight 51.1 / 68.9 / 91.9).
template <typename TI, int CH, int RPW, bool HAS_SUB, bool WRITE_XNEW, int NORMED>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(
    const TI* __restrict__ x, const TI* __restrict__ sub,
    const TI* __restrict__ w, const TI* __restrict__ b,
    TI* __restrict__ x_new, void* __restrict__ normed,
    const int32_t* __restrict__ row_index, int64_t in_rows, int64_t rows, int D, float eps,
    const int64_t* __restrict__ io, int io_mode) {
    DOTL_LN_RESOLVE_IO();
    const int lane = threadIdx.x & 63;
    const int64_t wave_global = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    const int64_t wave_stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
    const int nchunk = D >> 2;
    const float inv_d = 1.0f / static_cast<float>(D);
    const int64_t plane = rows * D;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);

    constexpr bool HOIST = CH <= 4;
    float4 wv[HOIST ? CH : 1], bv[HOIST ? CH : 1];
    if constexpr (HOIST) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int idx = c * 64 + lane;
            wv[c] = idx < nchunk ? load4f(w + 4 * idx) : z;
            bv[c] = idx < nchunk ? load4f(b + 4 * idx) : z;
        }
    }

    for (int64_t g = wave_global; g * RPW < rows; g += wave_stride) {
        const int64_t row0 = g * RPW;
        // per row: its input row, -1 for a row of zeros, -2 past the end
        int64_t src[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int64_t row = row0 + r;
            int64_t s_ = -2;
            if (row < rows) {
                s_ = row_index ? static_cast<int64_t>(row_index[row]) : row;
                if (s_ >= in_rows || s_ < 0) s_ = -1;
            }
            src[r] = s_;
        }
        float4 v[RPW][CH];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int idx = c * 64 + lane;
                v[r][c] = (src[r] >= 0 && idx < nchunk)
                              ? load_sum4<TI, HAS_SUB>(x, sub, src[r] * D + 4 * idx)
                              : z;
            }
        float mean_est[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            float s_ = 0.f;
#pragma unroll
            for (int c = 0; c < CH; ++c) s_ += (v[r][c].x + v[r][c].y) + (v[r][c].z + v[r][c].w);
            mean_est[r] = s_;
        }
        wave_sum_n(mean_est);
        float sd[RPW], sd2[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            mean_est[r] *= inv_d;
            sd[r] = 0.f;
            sd2[r] = 0.f;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int idx = c * 64 + lane;
                if (idx < nchunk) {
                    const float d0 = v[r][c].x - mean_est[r], d1 = v[r][c].y - mean_est[r];
                    const float d2 = v[r][c].z - mean_est[r], d3 = v[r][c].w - mean_est[r];
                    sd[r] += (d0 + d1) + (d2 + d3);
                    sd2[r] += ln_sq4(d0, d1, d2, d3);
                }
            }
        }
        {
            float both[2 * RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) { both[2 * r] = sd[r]; both[2 * r + 1] = sd2[r]; }
            wave_sum_n(both);
#pragma unroll
            for (int r = 0; r < RPW; ++r) { sd[r] = both[2 * r]; sd2[r] = both[2 * r + 1]; }
        }

        // x - mean as (x - m) - delta: x - m is exact (both near the mean),
        // whereas forming m + delta first would round the mean to ulp(mean).
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if (src[r] == -2) continue;   // wave-uniform
            const int64_t base = (row0 + r) * D;
            const bool zero = src[r] < 0;
            const float delta = sd[r] * inv_d;
            const float var = ln_var(sd2[r], delta, inv_d);
            const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int idx = c * 64 + lane;
                if (idx < nchunk) {
                    const int col = 4 * idx;
                    if constexpr (WRITE_XNEW) store4f(x_new + base + col, zero ? z : v[r][c]);
                    float4 ww, bb;
                    if constexpr (HOIST) {
                        ww = wv[c];
                        bb = bv[c];
                    } else {
                        ww = load4f(w + col);
                        bb = load4f(b + col);
                    }
                    float4 o;
                    o.x = ln_out(v[r][c].x, mean_est[r], delta, rstd, ww.x, bb.x);
                    o.y = ln_out(v[r][c].y, mean_est[r], delta, rstd, ww.y, bb.y);
                    o.z = ln_out(v[r][c].z, mean_est[r], delta, rstd, ww.z, bb.z);
                    o.w = ln_out(v[r][c].w, mean_est[r], delta, rstd, ww.w, bb.w);
                    store_normed4<NORMED>(normed, plane, base + col, zero ? z : o);
                }
            }
        }
    }
}

// Scalar path for any D in [1, 64 * EPL]: element e of lane l is column
// e * 64 + l. Used when D % 4 != 0 or a tensor is not aligned for the
// vector accesses.
template <typename TI, int EPL, bool HAS_SUB, bool WRITE_XNEW, int NORMED>
__global__ __launch_bounds__(256) void layernorm_scalar_kernel(
    const TI* __restrict__ x, const TI* __restrict__ sub,
    const TI* __restrict__ w, const TI* __restrict__ b,
    TI* __restrict__ x_new, void* __restrict__ normed,
    const int32_t* __restrict__ row_index, int64_t in_rows, int64_t rows, int D, float eps,
    const int64_t* __restrict__ io, int io_mode) {
    DOTL_LN_RESOLVE_IO();
    const int lane = threadIdx.x & 63;
    const int64_t wave_global = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    const int64_t wave_stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
    const float inv_d = 1.0f / static_cast<float>(D);
    const int64_t plane = rows * D;

    for (int64_t row = wave_global; row < rows; row += wave_stride) {
        const int64_t base = row * D;   // output row
        int64_t src = row_index ? static_cast<int64_t>(row_index[row]) : row;
        if (src >= in_rows) src = -1;
        if (src < 0) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int col = e * 64 + lane;
                if (col < D) {
                    if constexpr (WRITE_XNEW) x_new[base + col] = from_f32<TI>(0.f);
                    store_normed1<NORMED>(normed, plane, base + col, 0.f);
                }
            }
            continue;
        }
        const int64_t ibase = src * D;  // input row
        float v[EPL];
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int col = e * 64 + lane;
            float a = 0.f;
            if (col < D) {
                a = static_cast<float>(x[ibase + col]);
                if constexpr (HAS_SUB) a = round_via<TI>(a + static_cast<float>(sub[ibase + col]));
            }
            v[e] = a;
            s += a;
        }
        const float mean_est = wave_sum(s) * inv_d;
        float sd = 0.f, sd2 = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            if (e * 64 + lane < D) {
                const float d = v[e] - mean_est;
                sd += d;
                sd2 = fmaf(d, d, sd2);
            }
        }
        {
            float both[2] = {sd, sd2};
            wave_sum_n(both);
            sd = both[0];
            sd2 = both[1];
        }
        const float delta = sd * inv_d;
        const float var = ln_var(sd2, delta, inv_d);
        const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int col = e * 64 + lane;
            if (col < D) {
                if constexpr (WRITE_XNEW) x_new[base + col] = from_f32<TI>(v[e]);
                const float o = ln_out(v[e], mean_est, delta, rstd, static_cast<float>(w[col]),
                                       static_cast<float>(b[col]));
                store_normed1<NORMED>(normed, plane, base + col, o);
            }
        }
    }
}

struct LnArgs {
    const void* x;
    const void* sub;
    const void* w;
    const void* b;
    void* x_new;
    void* normed;
    const int32_t* row_index;
    int64_t in_rows;
    int64_t rows;
    int D;
    float eps;
    const int64_t* io;
    int io_mode;
    hipStream_t stream;
};

unsigned grid_for(int64_t rows) {
    // Enough 4-row workgroups to cover every row, capped so the grid-stride
    // loop takes over on very tall inputs: 256 CUs x 32 waves in flight.
    const int64_t want = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t cap = 256 * 8 * 16;
    return static_cast<unsigned>(want < cap ? (want > 0 ? want : 1) : cap);
}

template <typename TI, int CH, bool HAS_SUB, bool WX, int NO>
void launch_vec(const LnArgs& a) {
    constexpr int RPW = CH <= 1 ? 2 : 1;
    hipLaunchKernelGGL((layernorm_vec_kernel<TI, CH, RPW, HAS_SUB, WX, NO>),
                       dim3(grid_for((a.rows + RPW - 1) / RPW)),
                       dim3(256), 0, a.stream, static_cast<const TI*>(a.x),
                       static_cast<const TI*>(a.sub), static_cast<const TI*>(a.w),
                       static_cast<const TI*>(a.b), static_cast<TI*>(a.x_new), a.normed,
                       a.row_index, a.in_rows, a.rows, a.D, a.eps, a.io, a.io_mode);
}

template <typename TI, int EPL, bool HAS_SUB, bool WX, int NO>
void launch_scalar(const LnArgs& a) {
    hipLaunchKernelGGL((layernorm_scalar_kernel<TI, EPL, HAS_SUB, WX, NO>), dim3(grid_for(a.rows)),
                       dim3(256), 0, a.stream, static_cast<const TI*>(a.x),
                       static_cast<const TI*>(a.sub), static_cast<const TI*>(a.w),
                       static_cast<const TI*>(a.b), static_cast<TI*>(a.x_new), a.normed,
                       a.row_index, a.in_rows, a.rows, a.D, a.eps, a.io, a.io_mode);
}

template <typename TI, bool HAS_SUB, bool WX, int NO>
void dispatch_width(const LnArgs& a, bool vec) {
    const int D = a.D;
    if (vec) {
        if (D <= 256) launch_vec<TI, 1, HAS_SUB, WX, NO>(a);
        else if (D <= 512) launch_vec<TI, 2, HAS_SUB, WX, NO>(a);
        else if (D <= 1024) launch_vec<TI, 4, HAS_SUB, WX, NO>(a);
        else if (D <= 2048) launch_vec<TI, 8, HAS_SUB, WX, NO>(a);
        else if (D <= 4096) launch_vec<TI, 16, HAS_SUB, WX, NO>(a);
        else launch_vec<TI, 32, HAS_SUB, WX, NO>(a);
    } else {
        if (D <= 64) launch_scalar<TI, 1, HAS_SUB, WX, NO>(a);
        else if (D <= 256) launch_scalar<TI, 4, HAS_SUB, WX, NO>(a);
        else if (D <= 1024) launch_scalar<TI, 16, HAS_SUB, WX, NO>(a);
        else if (D <= 4096) launch_scalar<TI, 64, HAS_SUB, WX, NO>(a);
        else launch_scalar<TI, 128, HAS_SUB, WX, NO>(a);
    }
}

template <typename TI, int NO>
void dispatch_flags(const LnArgs& a, bool vec) {
    if (a.sub) {
        if (a.x_new) dispatch_width<TI, true, true, NO>(a, vec);
        else dispatch_width<TI, true, false, NO>(a, vec);
    } else {
        if (a.x_new) dispatch_width<TI, false, true, NO>(a, vec);
        else dispatch_width<TI, false, false, NO>(a, vec);
    }
}

}  // namespace
}  // namespace dotl

extern "C" int dotl_layernorm(const void* x, const void* sub, const void* weight,
                              const void* bias, void* x_new, void* normed,
                              const int32_t* row_index, int64_t in_rows, int64_t rows,
                              int64_t D, double eps, int dtype, int normed_dtype,
                              const int64_t* io, int io_mode, void* stream) {
    using namespace dotl;
    clear_error();
    const char* who = sub ? "fused_add_layernorm" : "fused_layernorm";
    DOTL_REQUIRE(dtype == DOTL_F32 || dtype == DOTL_F16 || dtype == DOTL_BF16,
                 "%s: x must be float32, float16 or bfloat16", who);
    if (dtype == DOTL_F32) {
        DOTL_REQUIRE(normed_dtype == DOTL_F32 || normed_dtype == DOTL_F16 ||
                         normed_dtype == DOTL_F16X2,
                     "%s: the normed output of a float32 x is float32, float16 or split float16",
                     who);
    } else {
        DOTL_REQUIRE(normed_dtype == dtype, "%s: the normed output of a %s x has x's dtype", who,
                     dtype == DOTL_F16 ? "float16" : "bfloat16");
    }
    DOTL_REQUIRE(D >= 1 && D <= 8192, "%s: last dimension %lld outside [1, 8192]", who,
                 static_cast<long long>(D));
    DOTL_REQUIRE(rows >= 0, "%s: negative row count", who);
    DOTL_REQUIRE(row_index == nullptr || in_rows >= 0, "%s: negative input row count", who);
    DOTL_REQUIRE(io_mode >= 0 && io_mode <= 3, "%s: io_mode must be in [0, 3]", who);
    DOTL_REQUIRE(io_mode == 0 || io != nullptr, "%s: io_mode %d needs an io slot", who, io_mode);
    if (rows == 0) return DOTL_OK;
    DOTL_REQUIRE((x || (io_mode & 1)) && weight && bias && (normed || (io_mode & 2)),
                 "%s: null pointer", who);

    // Slot-addressed tensors are not known here; the caller guarantees they
    // are allocations of the shapes given (16-byte aligned, as torch's are).
    const size_t esize = dtype == DOTL_F32 ? 4 : 2;
    const uintptr_t addr_or =
        reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(sub) |
        reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias) |
        reinterpret_cast<uintptr_t>(x_new) | reinterpret_cast<uintptr_t>(normed);
    const bool vec = (D % 4 == 0) && addr_or % (4 * esize) == 0 && (io_mode == 0 || D % 4 == 0);

    LnArgs a{x, sub, weight, bias, x_new, normed, row_index, row_index ? in_rows : rows, rows,
             static_cast<int>(D), static_cast<float>(eps), io, io_mode, as_stream(stream)};
    switch (dtype) {
        case DOTL_F16: dispatch_flags<_Float16, DOTL_F16>(a, vec); break;
        case DOTL_BF16: dispatch_flags<__bf16, DOTL_BF16>(a, vec); break;
        default:
            switch (normed_dtype) {
                case DOTL_F16: dispatch_flags<float, DOTL_F16>(a, vec); break;
                case DOTL_F16X2: dispatch_flags<float, DOTL_F16X2>(a, vec); break;
                default: dispatch_flags<float, DOTL_F32>(a, vec); break;
            }
            break;
    }
    return check_launch(who);
}

// Writes two addresses into a graph I/O slot, in stream order: the launch
// that rebinds a captured graph's input and output before each replay.
namespace dotl {
namespace {
__global__ void bind_io_kernel(int64_t* __restrict__ slot, int64_t a, int64_t b) {
    if (threadIdx.x == 0) {
        slot[0] = a;
        slot[1] = b;
    }
}
}  // namespace
}  // namespace dotl

extern "C" int dotl_bind_io(int64_t* slot, const void* in, void* out, void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(slot != nullptr, "bind_io: null slot");
    hipLaunchKernelGGL(bind_io_kernel, dim3(1), dim3(64), 0, as_stream(stream), slot,
                       static_cast<int64_t>(reinterpret_cast<uintptr_t>(in)),
                       static_cast<int64_t>(reinterpret_cast<uintptr_t>(out)));
    return check_launch("bind_io");
}

// Zero rows of a padded output, rows with row_map[r] >= 0 (written by the
// producer) left alone. Each wave reads the map entries of 64 rows at once
// (one a lane) and then stores zeros to the padded ones back to back: with a
// wave per row, every row first waited out its own map load.
namespace dotl {
namespace {
__global__ __launch_bounds__(256) void zero_rows_kernel(float* __restrict__ out,
                                                        const int32_t* __restrict__ row_map,
                                                        int64_t rows, int64_t width,
                                                        const int64_t* __restrict__ io) {
    if (io != nullptr) out = reinterpret_cast<float*>(io[1]);
    const int lane = threadIdx.x & 63;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
    for (int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6)) * 64;
         r0 < rows; r0 += waves * 64) {
        const int64_t r = r0 + lane;
        const bool pad = r < rows && row_map[r] < 0;
        uint64_t todo = __ballot(pad);
        while (todo != 0) {   // wave-uniform
            const int i = __builtin_ctzll(todo);
            todo &= todo - 1;
            float* row = out + (r0 + i) * width;
            if ((width & 3) == 0) {
                for (int64_t c = 4 * lane; c < width; c += 256)
                    *reinterpret_cast<float4*>(row + c) = make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                for (int64_t c = lane; c < width; c += 64) row[c] = 0.f;
            }
        }
    }
}
}  // namespace
}  // namespace dotl

extern "C" int dotl_zero_rows(float* out, const int32_t* row_map, int64_t rows, int64_t width,
                              const int64_t* io, void* stream) {
    using namespace dotl;
    clear_error();
    DOTL_REQUIRE(rows >= 0 && width >= 0, "zero_rows: negative extent");
    if (rows == 0 || width == 0) return DOTL_OK;
    DOTL_REQUIRE((out || io) && row_map, "zero_rows: null pointer");
    DOTL_REQUIRE(reinterpret_cast<uintptr_t>(out) % 16 == 0, "zero_rows: out must be 16-byte aligned");
    hipLaunchKernelGGL(zero_rows_kernel, dim3(grid_for((rows + 63) / 64)), dim3(256), 0,
                       as_stream(stream), out, row_map, rows, width, io);
    return check_launch("zero_rows");
}
