// Shared device and host helpers for the gfx950 kernels behind include/dotl.h.
//
// Everything here is CDNA4-specific on purpose: 64-lane wavefronts, MFMA
// vector types, and the one error channel every C-ABI entry point reports
// through.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/dotl.h"

namespace dotl {

constexpr int kWave = 64;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ---- tensor element types --------------------------------------------------
// float, _Float16 and __bf16 are the tensor dtypes DOTL_F32 / DOTL_F16 /
// DOTL_BF16. Conversions to 16-bit types round to nearest even (the hardware
// v_cvt_f16_f32 / v_cvt_pk_bf16_f32).

template <typename T> struct dtype_code;
template <> struct dtype_code<float> { static constexpr int value = DOTL_F32; };
template <> struct dtype_code<_Float16> { static constexpr int value = DOTL_F16; };
template <> struct dtype_code<__bf16> { static constexpr int value = DOTL_BF16; };

template <typename T>
__device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }

// v rounded through T and back (the identity for float).
template <typename T>
__device__ __forceinline__ float round_via(float v) { return static_cast<float>(static_cast<T>(v)); }

// Four consecutive elements as a float4; p is aligned to 4 * sizeof(T).
template <typename T>
__device__ __forceinline__ float4 load4f(const T* p) {
    if constexpr (sizeof(T) == 4) {
        return *reinterpret_cast<const float4*>(p);
    } else {
        typedef T t4 __attribute__((ext_vector_type(4)));
        const t4 h = *reinterpret_cast<const t4*>(p);
        return make_float4(static_cast<float>(h[0]), static_cast<float>(h[1]),
                           static_cast<float>(h[2]), static_cast<float>(h[3]));
    }
}

template <typename T>
__device__ __forceinline__ void store4f(T* p, float4 v) {
    if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(p) = v;
    } else {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 h;
        h[0] = static_cast<T>(v.x); h[1] = static_cast<T>(v.y);
        h[2] = static_cast<T>(v.z); h[3] = static_cast<T>(v.w);
        *reinterpret_cast<t4*>(p) = h;
    }
}

// ---- error channel ---------------------------------------------------------

void set_error(const std::string& msg);
void clear_error();

// Returns DOTL_E_LAUNCH with a message naming `who` if the last launch failed.
int check_launch(const char* who);

#define DOTL_REQUIRE(cond, ...)                                   \
    do {                                                          \
        if (!(cond)) {                                            \
            char _dotl_buf[512];                                  \
            std::snprintf(_dotl_buf, sizeof(_dotl_buf), __VA_ARGS__); \
            ::dotl::set_error(_dotl_buf);                         \
            return DOTL_E_INVALID;                                \
        }                                                         \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device helpers --------------------------------------------------------

// One step of a wavefront's xor butterfly: v + (v of lane l ^ OFF). The
// partner's value comes by the cheapest exact route on gfx950 instead of a
// ds_bpermute (an LDS round trip) every step: v_permlane32_swap /
// v_permlane16_swap across the 32- and 16-lane halves (with v in both
// operands, the two results are v and the partner's v), ds_swizzle (xor
// mode, within 32 lanes) for 8 and 4, DPP quad permutations for 2 and 1.
// Each lane gets exactly the sum __shfl_xor would give (fp addition
// commutes), so butterflies written either way agree bit for bit.
template <int OFF>
__device__ __forceinline__ float xor_add(float v) {
    static_assert(OFF == 32 || OFF == 16 || OFF == 8 || OFF == 4 || OFF == 2 || OFF == 1,
                  "a power-of-two lane offset below 64");
    if constexpr (OFF == 32) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                         false, false);
        return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    } else if constexpr (OFF == 16) {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                         false, false);
        return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    } else if constexpr (OFF == 8 || OFF == 4) {
        // bitmask mode: and 0x1f, or 0, xor OFF
        return v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (OFF << 10)));
    } else {
        // quad_perm [2,3,0,1] (xor 2) or [1,0,3,2] (xor 1)
        constexpr int kQuad = OFF == 2 ? 0x4E : 0xB1;
        return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kQuad, 0xF, 0xF,
                                                              false));
    }
}

// The full butterfly (offsets 32, 16, ..., 1) over K values at once, their
// steps interleaved so one value's fetch latency hides under the others'.
template <int OFF, int K>
__device__ __forceinline__ void xor_step(float (&v)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = xor_add<OFF>(v[k]);
}
template <int K>
__device__ __forceinline__ void wave_sum_n(float (&v)[K]) {
    xor_step<32>(v);
    xor_step<16>(v);
    xor_step<8>(v);
    xor_step<4>(v);
    xor_step<2>(v);
    xor_step<1>(v);
}

// Butterfly sum over the full 64-lane wavefront. Every lane ends with the total.
__device__ __forceinline__ float wave_sum(float v) {
    float a[1] = {v};
    wave_sum_n<1>(a);
    return a[0];
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// A value the compiler must treat as computed: narrowing it cannot be fused
// into the multiply-add that produced it. Left free, the backend may turn
// fp32 fma + fp16 conversion into one v_fma_mixlo_f16 (a single rounding to
// fp16), which differs in the last fp16 bit from the fp32 result narrowed
// with RNE -- the arithmetic the reference and every other kernel here use --
// and whether it does depends on the surrounding code.
__device__ __forceinline__ void opaque(float& v) { asm volatile("" : "+v"(v)); }

// erf GELU, 0.5 x (1 + erf(x / sqrt 2)), with erf from Abramowitz &
// Stegun, Handbook of Mathematical Functions, formula 7.1.26:
//   erfc(z) ~= (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),
//   t = 1 / (1 + p z), z >= 0, |error in erf| <= 1.5e-7.
// Written on erfc so neither sign cancels: with z = |x| / sqrt 2 and
// q = erfc(z), GELU(x) = x - |x| q / 2 for x >= 0 and -|x| q / 2 for x < 0,
// i.e. max(x, 0) + (-q / 2) |x|, one fma. The -1/2 is folded into the
// coefficients (a power of two: the Horner steps round exactly as before,
// scaled). |x| is clamped at 2^64 in that product so that x = +-inf, where
// q = 0, gives inf and 0 rather than 0 * inf. One reciprocal, one exp2 and
// nine other operations; the device library's erff costs several times
// that, and an epilogue that applies it to every output of a GEMM with a
// short K spends more time there than in the MFMAs.
// The fp32 result is fenced before any narrowing (see opaque), so an fp16
// output is that value rounded, in every kernel. VOL picks the fence: a
// volatile asm, which also bounds the compiler's scheduling regions, or a
// plain one; the bits are the same. Measured on MI355X, the volatile one
// schedules faster in the 8-wave GEMM tiles (C4 ffn_in 263 vs 270 us), the
// plain one everywhere else (C2 ffn_in 15.5 vs 17.5 us, the C5 fused FFN
// 161 vs 164).
template <bool VOL>
__device__ __forceinline__ float gelu_erf(float x) {
    const float ax = fabsf(x);
    const float z = ax * 0.70710678118654752440f;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
    float poly = fmaf(-0.5307027145f, t, 0.7265760135f);     // -a5 / 2, -a4 / 2
    poly = fmaf(poly, t, -0.7107068705f);                     // -a3 / 2
    poly = fmaf(poly, t, 0.142248368f);                       // -a2 / 2
    poly = fmaf(poly, t, -0.127414796f);                      // -a1 / 2
    poly *= t;
    // exp(-z^2) = exp2(-x^2 log2(e) / 2)
    const float hq = poly * __builtin_amdgcn_exp2f(x * (x * -0.72134752044448170368f));
    float g = fmaf(hq, fminf(ax, 0x1p64f), fmaxf(x, 0.f));
    if constexpr (VOL) {
        opaque(g);
    } else {
        asm("" : "+v"(g));
    }
    return g;
}

// LayerNorm arithmetic shared by every kernel that normalises a row, each
// multiply-add written as an explicit fmaf. Left to the compiler, a sum of
// two products contracts either way round (fma(a, a, b*b) or fma(b, b, a*a)),
// and two kernels computing the same expression could differ in the last bit.
__device__ __forceinline__ float ln_sq4(float d0, float d1, float d2, float d3) {
    return fmaf(d1, d1, d0 * d0) + fmaf(d3, d3, d2 * d2);
}
// Biased variance from the centred sums: E[d^2] - E[d]^2, clamped at 0.
__device__ __forceinline__ float ln_var(float sd2, float delta, float inv_d) {
    return fmaxf(fmaf(-delta, delta, sd2 * inv_d), 0.f);
}
// (x - mean) * rstd * w + b, with x - mean formed as (x - mean_est) - delta:
// x - mean_est is exact for x near the mean, whereas forming mean_est + delta
// first would round the mean to ulp(mean).
__device__ __forceinline__ float ln_out(float v, float mean_est, float delta, float rstd,
                                        float w, float b) {
    return fmaf(((v - mean_est) - delta) * rstd, w, b);
}

// fp32 -> fp16 with round-to-nearest-even (the hardware conversion).
__device__ __forceinline__ _Float16 to_half(float x) { return static_cast<_Float16>(x); }

// Split x into hi = fp16(x) and lo = fp16((x - hi) * 2^12). hi + lo * 2^-12
// carries ~22 significant bits for |x| in fp16's normal range; the 2^12 scale
// keeps lo out of fp16's subnormals, whose flushing behaviour inside MFMA we
// do not rely on.
constexpr float kLoScale = 4096.0f;
constexpr float kLoUnscale = 1.0f / 4096.0f;

__device__ __forceinline__ _Float16 split_lo(float x, _Float16 hi) {
    return static_cast<_Float16>((x - static_cast<float>(hi)) * kLoScale);
}

// Storage type of each normed-output code.
template <int NORMED> struct normed_type { using type = float; };
template <> struct normed_type<DOTL_F16> { using type = _Float16; };
template <> struct normed_type<DOTL_F16X2> { using type = _Float16; };
template <> struct normed_type<DOTL_BF16> { using type = __bf16; };


// Four normalised values to a LayerNorm's normed output (split planes: hi,
// then lo in the second plane, `plane` elements further on).
template <int NORMED>
__device__ __forceinline__ void store_normed4(void* __restrict__ normed, int64_t plane,
                                             int64_t off, float4 o) {
    using TO = typename normed_type<NORMED>::type;
    TO* out = static_cast<TO*>(normed);
    if constexpr (NORMED != DOTL_F32) {
        opaque(o.x); opaque(o.y); opaque(o.z); opaque(o.w);
    }
    if constexpr (NORMED == DOTL_F16X2) {
        half4 h, l;
        h[0] = to_half(o.x); h[1] = to_half(o.y); h[2] = to_half(o.z); h[3] = to_half(o.w);
        l[0] = split_lo(o.x, h[0]); l[1] = split_lo(o.y, h[1]);
        l[2] = split_lo(o.z, h[2]); l[3] = split_lo(o.w, h[3]);
        *reinterpret_cast<half4*>(out + off) = h;
        *reinterpret_cast<half4*>(out + plane + off) = l;
    } else {
        store4f(out + off, o);
    }
}

}  // namespace dotl
