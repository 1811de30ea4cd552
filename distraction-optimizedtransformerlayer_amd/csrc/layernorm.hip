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

__device__ __forceinline__ int64_t D_of(int nchunk) { return 4 * static_cast<int64_t>(nchunk); }

template <bool HAS_SUB>
__device__ __forceinline__ float4 load_sum4(const float* __restrict__ x,
                                            const float* __restrict__ sub, int64_t off) {
    float4 a = *reinterpret_cast<const float4*>(x + off);
    if constexpr (HAS_SUB) {
        const float4 s = *reinterpret_cast<const float4*>(sub + off);
        a.x += s.x; a.y += s.y; a.z += s.z; a.w += s.w;
    }
    return a;
}

// A row whose index entry is negative: every output of the row is zero.
template <int CH, bool WRITE_XNEW, int NORMED>
__device__ __forceinline__ void zero_row_vec(float* __restrict__ x_new, void* __restrict__ normed,
                                             int64_t rows, int64_t base, int nchunk, int lane) {
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int idx = c * 64 + lane;
        if (idx < nchunk) {
            const int col = 4 * idx;
            if constexpr (WRITE_XNEW) *reinterpret_cast<float4*>(x_new + base + col) = z;
            if constexpr (NORMED == DOTL_F16 || NORMED == DOTL_F16X2) {
                const half4 hz = {};
                *reinterpret_cast<half4*>(static_cast<_Float16*>(normed) + base + col) = hz;
                if constexpr (NORMED == DOTL_F16X2)
                    *reinterpret_cast<half4*>(static_cast<_Float16*>(normed) + rows * D_of(nchunk) + base + col) = hz;
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(normed) + base + col) = z;
            }
        }
    }
}

// Vector path: D % 4 == 0 and D <= 256 * CH. Chunk c of lane l covers row
// elements [4 * (c * 64 + l), +4).
template <int CH, bool HAS_SUB, bool WRITE_XNEW, int NORMED>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(
    const float* __restrict__ x, const float* __restrict__ sub,
    const float* __restrict__ w, const float* __restrict__ b,
    float* __restrict__ x_new, void* __restrict__ normed,
    const int32_t* __restrict__ row_index, int64_t in_rows, int64_t rows, int D, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t wave_global = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    const int64_t wave_stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
    const int nchunk = D >> 2;
    const float inv_d = 1.0f / static_cast<float>(D);

    for (int64_t row = wave_global; row < rows; row += wave_stride) {
        const int64_t base = row * D;   // output row
        int64_t src = row_index ? static_cast<int64_t>(row_index[row]) : row;
        if (src >= in_rows) src = -1;
        if (src < 0) {
            zero_row_vec<CH, WRITE_XNEW, NORMED>(x_new, normed, rows, base, nchunk, lane);
            continue;
        }
        const int64_t ibase = src * D;  // input row
        float4 v[CH];
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int idx = c * 64 + lane;
            if (idx < nchunk) {
                v[c] = load_sum4<HAS_SUB>(x, sub, ibase + 4 * idx);
            } else {
                v[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            s += (v[c].x + v[c].y) + (v[c].z + v[c].w);
        }
        const float mean_est = wave_sum(s) * inv_d;

        float sd = 0.f, sd2 = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int idx = c * 64 + lane;
            if (idx < nchunk) {
                const float d0 = v[c].x - mean_est, d1 = v[c].y - mean_est;
                const float d2 = v[c].z - mean_est, d3 = v[c].w - mean_est;
                sd += (d0 + d1) + (d2 + d3);
                sd2 += ln_sq4(d0, d1, d2, d3);
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            sd += __shfl_xor(sd, off, kWave);
            sd2 += __shfl_xor(sd2, off, kWave);
        }
        const float delta = sd * inv_d;
        const float var = ln_var(sd2, delta, inv_d);
        const float rstd = 1.0f / sqrtf(var + eps);

        // x - mean as (x - m) - delta: x - m is exact (both near the mean),
        // whereas forming m + delta first would round the mean to ulp(mean).
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int idx = c * 64 + lane;
            if (idx < nchunk) {
                const int col = 4 * idx;
                if constexpr (WRITE_XNEW) {
                    *reinterpret_cast<float4*>(x_new + base + col) = v[c];
                }
                const float4 ww = *reinterpret_cast<const float4*>(w + col);
                const float4 bb = *reinterpret_cast<const float4*>(b + col);
                float4 o;
                o.x = ln_out(v[c].x, mean_est, delta, rstd, ww.x, bb.x);
                o.y = ln_out(v[c].y, mean_est, delta, rstd, ww.y, bb.y);
                o.z = ln_out(v[c].z, mean_est, delta, rstd, ww.z, bb.z);
                o.w = ln_out(v[c].w, mean_est, delta, rstd, ww.w, bb.w);
                if constexpr (NORMED == DOTL_F16 || NORMED == DOTL_F16X2) {
                    half4 h;
                    h[0] = to_half(o.x); h[1] = to_half(o.y);
                    h[2] = to_half(o.z); h[3] = to_half(o.w);
                    *reinterpret_cast<half4*>(static_cast<_Float16*>(normed) + base + col) = h;
                    if constexpr (NORMED == DOTL_F16X2) {
                        half4 l;
                        l[0] = split_lo(o.x, h[0]); l[1] = split_lo(o.y, h[1]);
                        l[2] = split_lo(o.z, h[2]); l[3] = split_lo(o.w, h[3]);
                        *reinterpret_cast<half4*>(static_cast<_Float16*>(normed) + rows * D + base + col) = l;
                    }
                } else {
                    *reinterpret_cast<float4*>(static_cast<float*>(normed) + base + col) = o;
                }
            }
        }
    }
}

// Scalar path for any D in [1, 64 * EPL]: element e of lane l is column
// e * 64 + l. Used when D % 4 != 0 (the vector path's 16-byte accesses need it).
template <int EPL, bool HAS_SUB, bool WRITE_XNEW, int NORMED>
__global__ __launch_bounds__(256) void layernorm_scalar_kernel(
    const float* __restrict__ x, const float* __restrict__ sub,
    const float* __restrict__ w, const float* __restrict__ b,
    float* __restrict__ x_new, void* __restrict__ normed,
    const int32_t* __restrict__ row_index, int64_t in_rows, int64_t rows, int D, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t wave_global = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    const int64_t wave_stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
    const float inv_d = 1.0f / static_cast<float>(D);

    for (int64_t row = wave_global; row < rows; row += wave_stride) {
        const int64_t base = row * D;   // output row
        int64_t src = row_index ? static_cast<int64_t>(row_index[row]) : row;
        if (src >= in_rows) src = -1;
        if (src < 0) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int col = e * 64 + lane;
                if (col < D) {
                    if constexpr (WRITE_XNEW) x_new[base + col] = 0.f;
                    if constexpr (NORMED == DOTL_F16 || NORMED == DOTL_F16X2) {
                        static_cast<_Float16*>(normed)[base + col] = static_cast<_Float16>(0.f);
                        if constexpr (NORMED == DOTL_F16X2)
                            static_cast<_Float16*>(normed)[rows * D + base + col] = static_cast<_Float16>(0.f);
                    } else {
                        static_cast<float*>(normed)[base + col] = 0.f;
                    }
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
                a = x[ibase + col];
                if constexpr (HAS_SUB) a += sub[ibase + col];
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
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            sd += __shfl_xor(sd, off, kWave);
            sd2 += __shfl_xor(sd2, off, kWave);
        }
        const float delta = sd * inv_d;
        const float var = ln_var(sd2, delta, inv_d);
        const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int col = e * 64 + lane;
            if (col < D) {
                if constexpr (WRITE_XNEW) x_new[base + col] = v[e];
                const float o = ln_out(v[e], mean_est, delta, rstd, w[col], b[col]);
                if constexpr (NORMED == DOTL_F16 || NORMED == DOTL_F16X2) {
                    const _Float16 h = to_half(o);
                    static_cast<_Float16*>(normed)[base + col] = h;
                    if constexpr (NORMED == DOTL_F16X2)
                        static_cast<_Float16*>(normed)[rows * D + base + col] = split_lo(o, h);
                } else {
                    static_cast<float*>(normed)[base + col] = o;
                }
            }
        }
    }
}

struct LnArgs {
    const float* x;
    const float* sub;
    const float* w;
    const float* b;
    float* x_new;
    void* normed;
    const int32_t* row_index;
    int64_t in_rows;
    int64_t rows;
    int D;
    float eps;
    hipStream_t stream;
};

unsigned grid_for(int64_t rows) {
    // Enough 4-row workgroups to cover every row, capped so the grid-stride
    // loop takes over on very tall inputs: 256 CUs x 32 waves in flight.
    const int64_t want = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t cap = 256 * 8 * 16;
    return static_cast<unsigned>(want < cap ? (want > 0 ? want : 1) : cap);
}

template <int CH, bool HAS_SUB, bool WX, int F16>
void launch_vec(const LnArgs& a) {
    hipLaunchKernelGGL((layernorm_vec_kernel<CH, HAS_SUB, WX, F16>), dim3(grid_for(a.rows)),
                       dim3(256), 0, a.stream, a.x, a.sub, a.w, a.b, a.x_new, a.normed,
                       a.row_index, a.in_rows, a.rows, a.D, a.eps);
}

template <int EPL, bool HAS_SUB, bool WX, int F16>
void launch_scalar(const LnArgs& a) {
    hipLaunchKernelGGL((layernorm_scalar_kernel<EPL, HAS_SUB, WX, F16>), dim3(grid_for(a.rows)),
                       dim3(256), 0, a.stream, a.x, a.sub, a.w, a.b, a.x_new, a.normed,
                       a.row_index, a.in_rows, a.rows, a.D, a.eps);
}

template <bool HAS_SUB, bool WX, int F16>
void dispatch_width(const LnArgs& a, bool vec) {
    const int D = a.D;
    if (vec) {
        if (D <= 256) launch_vec<1, HAS_SUB, WX, F16>(a);
        else if (D <= 512) launch_vec<2, HAS_SUB, WX, F16>(a);
        else if (D <= 1024) launch_vec<4, HAS_SUB, WX, F16>(a);
        else if (D <= 2048) launch_vec<8, HAS_SUB, WX, F16>(a);
        else if (D <= 4096) launch_vec<16, HAS_SUB, WX, F16>(a);
        else launch_vec<32, HAS_SUB, WX, F16>(a);
    } else {
        if (D <= 64) launch_scalar<1, HAS_SUB, WX, F16>(a);
        else if (D <= 256) launch_scalar<4, HAS_SUB, WX, F16>(a);
        else if (D <= 1024) launch_scalar<16, HAS_SUB, WX, F16>(a);
        else if (D <= 4096) launch_scalar<64, HAS_SUB, WX, F16>(a);
        else launch_scalar<128, HAS_SUB, WX, F16>(a);
    }
}

}  // namespace
}  // namespace dotl

extern "C" int dotl_layernorm(const void* x, const void* sub, const float* weight,
                              const float* bias, void* x_new, void* normed,
                              const int32_t* row_index, int64_t in_rows, int64_t rows,
                              int64_t D, double eps, int dtype, int normed_dtype,
                              void* stream) {
    using namespace dotl;
    clear_error();
    const char* who = sub ? "fused_add_layernorm" : "fused_layernorm";
    if (dtype != DOTL_F32) {
        set_error(std::string(who) + ": this build serves float32 tensors only");
        return DOTL_DECLINED;
    }
    DOTL_REQUIRE(normed_dtype == DOTL_F32 || normed_dtype == DOTL_F16 || normed_dtype == DOTL_F16X2,
                 "%s: normed dtype must be float32, float16 or split float16", who);
    DOTL_REQUIRE(D >= 1 && D <= 8192, "%s: last dimension %lld outside [1, 8192]", who,
                 static_cast<long long>(D));
    DOTL_REQUIRE(rows >= 0, "%s: negative row count", who);
    DOTL_REQUIRE(row_index == nullptr || in_rows >= 0, "%s: negative input row count", who);
    if (rows == 0) return DOTL_OK;
    DOTL_REQUIRE(x && weight && bias && normed, "%s: null pointer", who);

    const bool aligned =
        (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(sub) |
         reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias) |
         reinterpret_cast<uintptr_t>(x_new) | reinterpret_cast<uintptr_t>(normed)) % 16 == 0;
    const bool vec = (D % 4 == 0) && aligned;

    LnArgs a{static_cast<const float*>(x), static_cast<const float*>(sub), weight, bias,
             static_cast<float*>(x_new), normed, row_index, row_index ? in_rows : rows, rows,
             static_cast<int>(D),
             static_cast<float>(eps), as_stream(stream)};
    auto by_out = [&](auto has_sub, auto wx) {
        constexpr bool HS = decltype(has_sub)::value;
        constexpr bool WX = decltype(wx)::value;
        switch (normed_dtype) {
            case DOTL_F16: dispatch_width<HS, WX, DOTL_F16>(a, vec); break;
            case DOTL_F16X2: dispatch_width<HS, WX, DOTL_F16X2>(a, vec); break;
            default: dispatch_width<HS, WX, DOTL_F32>(a, vec); break;
        }
    };
    if (sub) {
        if (x_new) by_out(std::true_type{}, std::true_type{});
        else by_out(std::true_type{}, std::false_type{});
    } else {
        if (x_new) by_out(std::false_type{}, std::true_type{});
        else by_out(std::false_type{}, std::false_type{});
    }
    return check_launch(who);
}
