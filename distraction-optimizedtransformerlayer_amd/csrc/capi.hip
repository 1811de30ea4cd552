// Library-wide C-ABI entries: error channel, version, knobs, the build smoke
// test and the MFMA accumulator-layout probe.
#include "dotl_common.h"

#include <atomic>

namespace dotl {

namespace {
thread_local std::string g_last_error;
std::atomic<int> g_wmma_fp16{1};
std::atomic<int> g_cp_async{2};
std::atomic<int> g_attn_nw{0};
std::atomic<int> g_attn_ns{0};
std::atomic<int> g_split_enabled{1};
std::atomic<int> g_split_forced{0};
}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int check_launch(const char* who) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error(std::string(who) + ": kernel launch failed: " + hipGetErrorString(err));
        return DOTL_E_LAUNCH;
    }
    return DOTL_OK;
}

int attention_fp16_default() { return g_wmma_fp16.load(std::memory_order_relaxed); }
int attention_cp_async_mode() { return g_cp_async.load(std::memory_order_relaxed); }
void attention_pipeline(int* nw, int* ns) {
    *nw = g_attn_nw.load(std::memory_order_relaxed);
    *ns = g_attn_ns.load(std::memory_order_relaxed);
}
void attention_split_knobs(int* enabled, int* forced) {
    *enabled = g_split_enabled.load(std::memory_order_relaxed);
    *forced = g_split_forced.load(std::memory_order_relaxed);
}

namespace {

__global__ void identity_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = x[i];
}

// One wavefront. Two MFMAs per instruction shape, each with a single nonzero
// K slot (lane group 0, element 0): A[i][0] = i + 1 against B[0][j] = 1 gives
// C[i][j] = i + 1, and A[i][0] = 1 against B[0][j] = j + 1 gives j + 1, so
// every accumulator register reports its own (row, col). Exact for i, j < 32.
__global__ void mfma_probe_kernel(int32_t* out) {
    const int lane = threadIdx.x;
    // 32x32x16: lane supplies A[l % 32][8 * (l / 32) + e] and B[8 * (l / 32) + e][l % 32].
    {
        half8 a_row = {}, b_one = {}, a_one = {}, b_col = {};
        if (lane < 32) {  // k == 0 lives in lane group 0, element 0
            a_row[0] = static_cast<_Float16>(lane % 32 + 1);
            b_one[0] = static_cast<_Float16>(1.0f);
            a_one[0] = static_cast<_Float16>(1.0f);
            b_col[0] = static_cast<_Float16>(lane % 32 + 1);
        }
        floatx16 zero = {};
        floatx16 rows = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_row, b_one, zero, 0, 0, 0);
        floatx16 cols = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_one, b_col, zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = static_cast<int>(rows[r]) - 1;
            const int col = static_cast<int>(cols[r]) - 1;
            out[lane * 16 + r] = row * 32 + col;
        }
    }
    // 16x16x32: lane supplies A[l % 16][8 * (l / 16) + e] and B[8 * (l / 16) + e][l % 16].
    {
        half8 a_row = {}, b_one = {}, a_one = {}, b_col = {};
        if (lane < 16) {
            a_row[0] = static_cast<_Float16>(lane % 16 + 1);
            b_one[0] = static_cast<_Float16>(1.0f);
            a_one[0] = static_cast<_Float16>(1.0f);
            b_col[0] = static_cast<_Float16>(lane % 16 + 1);
        }
        floatx4 zero = {};
        floatx4 rows = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_row, b_one, zero, 0, 0, 0);
        floatx4 cols = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_one, b_col, zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = static_cast<int>(rows[r]) - 1;
            const int col = static_cast<int>(cols[r]) - 1;
            out[1024 + lane * 4 + r] = row * 16 + col;
        }
    }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// One wave: zero a 2 KiB LDS region, DMA 16 bytes per lane into its start,
// copy the region out.
__global__ void lds_dma_probe_kernel(const int32_t* __restrict__ src, int32_t* __restrict__ out) {
    __shared__ __attribute__((aligned(1024))) int32_t region[512];
    const int lane = threadIdx.x;
    for (int i = lane; i < 512; i += 64) region[i] = 0;
    __syncthreads();
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + 4 * lane),
                                     (lds_void_t*)(region), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int i = lane; i < 512; i += 64) out[i] = region[i];
}

// Sustained MFMA rate: each wave chains `iters` rounds of 16 independent
// v_mfma_f32_32x32x16_f16 on register operands (4 A x 4 B fragments, no
// memory traffic). random != 0 fills the fragments with random values, as a
// GEMM's are; on MI355X the matrix cores then draw enough power to pull the
// clock from ~2.2 to ~1.7 GHz, and that -- not the datasheet rate -- is the
// roof every MFMA kernel here runs against.
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int iters, int random, float* sink) {
    floatx16 acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = floatx16{};
    half8 a[4], b[4];
    uint32_t st = threadIdx.x * 7919u + blockIdx.x * 104729u + 1u;
    for (int r = 0; r < 4; ++r)
        for (int e = 0; e < 8; ++e) {
            float x = e * 0.25f, y = e * 0.5f;
            if (random) {
                st = st * 1664525u + 1013904223u;
                x = (((st >> 9) & 0x3fff) / 16384.0f - 0.5f) * 4.f;
                st = st * 1664525u + 1013904223u;
                y = (((st >> 9) & 0x3fff) / 16384.0f - 0.5f) * 4.f;
            }
            a[r][e] = static_cast<_Float16>(x);
            b[r][e] = static_cast<_Float16>(y);
        }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[i % 4], a[i / 4], acc[i], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[i][threadIdx.x & 15];
    if (s == 1234.5f) sink[0] = s;   // keeps the products live; never true in practice
}

}  // namespace
}  // namespace dotl

extern "C" {

const char* dotl_last_error(void) { return dotl::g_last_error.c_str(); }

int dotl_abi_version(void) { return DOTL_ABI_VERSION; }

const char* dotl_target(void) { return "gfx950"; }

int dotl_smoke_test_identity(const float* x, float* y, int64_t n, void* stream) {
    dotl::clear_error();
    DOTL_REQUIRE(n >= 0, "smoke_test_identity: n must be non-negative, got %lld",
                 static_cast<long long>(n));
    if (n == 0) return DOTL_OK;
    DOTL_REQUIRE(x != nullptr && y != nullptr, "smoke_test_identity: null pointer");
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    DOTL_REQUIRE(blocks <= 0x7fffffff, "smoke_test_identity: n too large");
    hipLaunchKernelGGL(dotl::identity_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads),
                       0, dotl::as_stream(stream), x, y, n);
    return dotl::check_launch("smoke_test_identity");
}

int dotl_mfma_layout_probe(int32_t* out, void* stream) {
    dotl::clear_error();
    DOTL_REQUIRE(out != nullptr, "mfma_layout_probe: null output");
    hipLaunchKernelGGL(dotl::mfma_probe_kernel, dim3(1), dim3(64), 0, dotl::as_stream(stream), out);
    return dotl::check_launch("mfma_layout_probe");
}

int dotl_mfma_ceiling_probe(int64_t workgroups, int32_t iters, int32_t random_operands, float* sink,
                            void* stream) {
    dotl::clear_error();
    DOTL_REQUIRE(sink != nullptr, "mfma_ceiling_probe: null sink");
    DOTL_REQUIRE(workgroups >= 1 && workgroups <= 0x7fffffff && iters >= 0 && iters <= (1 << 20),
                 "mfma_ceiling_probe: workgroups must be in [1, 2^31) and iters in [0, 2^20]");
    hipLaunchKernelGGL(dotl::mfma_ceiling_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(256),
                       0, dotl::as_stream(stream), static_cast<int>(iters),
                       random_operands ? 1 : 0, sink);
    return dotl::check_launch("mfma_ceiling_probe");
}

int dotl_lds_dma_probe(const int32_t* src, int32_t* out, void* stream) {
    dotl::clear_error();
    DOTL_REQUIRE(src != nullptr && out != nullptr, "lds_dma_probe: null pointer");
    hipLaunchKernelGGL(dotl::lds_dma_probe_kernel, dim3(1), dim3(64), 0, dotl::as_stream(stream),
                       src, out);
    return dotl::check_launch("lds_dma_probe");
}

void dotl_wmma_set_fp16(int on) { dotl::g_wmma_fp16.store(on ? 1 : 0); }
int dotl_wmma_fp16(void) { return dotl::g_wmma_fp16.load(); }
void dotl_wmma_set_cp_async(int mode) { dotl::g_cp_async.store(mode); }
void dotl_attention_set_pipeline(int waves, int stages) {
    dotl::g_attn_nw.store(waves);
    dotl::g_attn_ns.store(stages);
}
int dotl_wmma_cp_async_mode(void) { return dotl::g_cp_async.load(); }
void dotl_wmma_set_split_kv(int on) { dotl::g_split_enabled.store(on ? 1 : 0); }
int dotl_wmma_split_kv_enabled(void) { return dotl::g_split_enabled.load(); }
void dotl_wmma_set_split_count(int n) { dotl::g_split_forced.store(n > 0 ? n : 0); }

}  // extern "C"
