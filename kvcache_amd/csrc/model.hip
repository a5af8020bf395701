// model.hip -- the decoder-step operations around the attention path (a Qwen2-shaped
// layer, qwen_kernels.h:7-13,23-29): embedding gather, RMSNorm, bias, residual,
// rotary position embedding (rotate-half form), SwiGLU, argmax over fp32 logits, and
// the linear layers as fp16 GEMMs through rocBLAS (the reference uses cuBLAS).
//
// Activations and weights are fp16 in memory; every kernel computes in fp32 and
// rounds once on store.  Row-wise kernels use 16-byte (8 x fp16) vectors, so the
// row widths must be multiples of 8.
#include "internal.hpp"
#include "kvc_abi.h"

#include <rocblas/rocblas.h>

#include <cfloat>
#include <climits>
#include <cmath>
#include <mutex>
#include <vector>

namespace kvc {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
constexpr int kThreads = 256;

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// out[r, :] = table[ids[r], :]; ids outside [0, V) give a zero row.
__global__ __launch_bounds__(kThreads) void embed_kernel(_Float16* out, const _Float16* table, const int* ids, int V,
                                                         int H, const int* dev_rows) {
    const int r = blockIdx.x;
    if (dev_rows && r >= *dev_rows) return;
    const int id = ids[r];
    const bool ok = id >= 0 && id < V;
    const f16x8* src = reinterpret_cast<const f16x8*>(table + (size_t)(ok ? id : 0) * H);
    f16x8* dst = reinterpret_cast<f16x8*>(out + (size_t)r * H);
    for (int i = threadIdx.x; i < H / 8; i += kThreads) dst[i] = ok ? src[i] : f16x8{};
}

// out[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w   (qwen_kernels.cu:24-40)
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(_Float16* out, const _Float16* in, const _Float16* w,
                                                           int H, float eps) {
    __shared__ float red[kThreads / 64];
    const int r = blockIdx.x;
    const f16x8* x = reinterpret_cast<const f16x8*>(in + (size_t)r * H);
    float ss = 0.f;
    for (int i = threadIdx.x; i < H / 8; i += kThreads) {
        const f16x8 v = x[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __builtin_fmaf((float)v[e], (float)v[e], ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k) tot += red[k];
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
    const f16x8* wv = reinterpret_cast<const f16x8*>(w);
    f16x8* y = reinterpret_cast<f16x8*>(out + (size_t)r * H);
    for (int i = threadIdx.x; i < H / 8; i += kThreads) {
        const f16x8 v = x[i], g = wv[i];
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (_Float16)((float)v[e] * inv * (float)g[e]);
        y[i] = o;
    }
}

// x[r, c] += bias[c]   (x is [rows, W], W % 8 == 0)
__global__ __launch_bounds__(kThreads) void bias_kernel(_Float16* x, const _Float16* bias, size_t nvec, int wvec) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nvec) return;
    f16x8* xv = reinterpret_cast<f16x8*>(x);
    const f16x8 b = reinterpret_cast<const f16x8*>(bias)[i % wvec];
    f16x8 v = xv[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)b[e]);
    xv[i] = v;
}

// x[i] += y[i]
__global__ __launch_bounds__(kThreads) void residual_kernel(_Float16* x, const _Float16* y, size_t nvec) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nvec) return;
    f16x8* xv = reinterpret_cast<f16x8*>(x);
    const f16x8 b = reinterpret_cast<const f16x8*>(y)[i];
    f16x8 v = xv[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)b[e]);
    xv[i] = v;
}

// out[i] = silu(gate[i]) * up[i],  silu(g) = g / (1 + e^-g)
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(_Float16* out, const _Float16* gate, const _Float16* up,
                                                            size_t nvec) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nvec) return;
    const f16x8 g = reinterpret_cast<const f16x8*>(gate)[i], u = reinterpret_cast<const f16x8*>(up)[i];
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float gf = (float)g[e];
        o[e] = (_Float16)(gf / (1.0f + expf(-gf)) * (float)u[e]);
    }
    reinterpret_cast<f16x8*>(out)[i] = o;
}

// Rotary embedding, rotate-half form (qwen_kernels.cu:64-79): x is [rows, heads, D];
// row r sits at position pos[r] (or pos_base + r); for t < D/2 the pair
// (x_t, x_{t+D/2}) turns by angle pos * theta^(-2t/D).
__global__ __launch_bounds__(kThreads) void rope_kernel(_Float16* x, const int* pos, int pos_base, size_t pairs,
                                                        int heads, int D, float log2_theta,
                                                        const int* dev_base = nullptr) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= pairs) return;
    const int hd = D / 2;
    const int t = (int)(i % hd);
    const size_t rh = i / hd;  // row * heads + head
    const int r = (int)(rh / heads);
    const float p = (float)(pos ? pos[r] : (dev_base ? *dev_base : pos_base) + r);
    const float inv = exp2f(-log2_theta * (2.0f * (float)t / (float)D));
    float s, c;
    sincosf(p * inv, &s, &c);
    _Float16* b = x + rh * D;
    const float x1 = (float)b[t], x2 = (float)b[t + hd];
    b[t] = (_Float16)(x1 * c - x2 * s);
    b[t + hd] = (_Float16)(x2 * c + x1 * s);
}

// out[r] = argmax_j logits[r, j] (first index of the maximum; NaN never wins)
constexpr int kArgThreads = 1024;
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float* logits, int V, int* out) {
    __shared__ float sv[kArgThreads / 64];
    __shared__ int si[kArgThreads / 64];
    const float* row = logits + (size_t)blockIdx.x * V;
    float best = -FLT_MAX;
    int bi = INT_MAX;
    for (int j = threadIdx.x; j < V; j += kArgThreads) {
        const float v = row[j];
        if (v > best) { best = v; bi = j; }  // strided scan: the first max of this thread's indices
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kArgThreads / 64; ++k)
            if (sv[k] > best || (sv[k] == best && si[k] < bi)) { best = sv[k]; bi = si[k]; }
        out[blockIdx.x] = bi == INT_MAX ? 0 : bi;
    }
}

inline unsigned blocks_for(size_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// rocBLAS handle per device, created on first use.
std::mutex g_blas_mu;
std::vector<rocblas_handle> g_blas;

int blas_handle(rocblas_handle* h) {
    int dev = 0;
    int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_blas_mu);
    if ((int)g_blas.size() <= dev) g_blas.resize(dev + 1, nullptr);
    if (!g_blas[dev] && rocblas_create_handle(&g_blas[dev]) != rocblas_status_success)
        return set_error(KVC_ERR_HIP, "rocblas_create_handle failed");
    *h = g_blas[dev];
    return KVC_OK;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

namespace {
template <typename F>
int guard_model(F&& f) {
    try {
        return f();
    } catch (...) {
        return set_error(KVC_ERR_STATE, "unexpected exception");
    }
}
bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
}  // namespace

extern "C" {

int kvc_embed_gather(void* out, const void* embed, const int* ids, int L, int H, int V, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L < 0 || H <= 0 || H % 8 || V <= 0) return set_error(KVC_ERR_ARG, "embed: L >= 0, H > 0 (multiple of 8), V > 0");
        if (L == 0) return KVC_OK;
        if (!out || !embed || !ids || !a16(out) || !a16(embed)) return set_error(KVC_ERR_ARG, "embed: bad pointers");
        hipLaunchKernelGGL(embed_kernel, dim3(L), dim3(kThreads), 0, (hipStream_t)st, (_Float16*)out,
                           (const _Float16*)embed, ids, V, H, nullptr);
        return hip_check(hipGetLastError(), "embed launch");
    });
}

int kvc_embed_gather_dev(void* out, const void* embed, const int* ids, const int* dev_rows, int L_cap, int H, int V,
                         kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L_cap <= 0 || H <= 0 || H % 8 || V <= 0) return set_error(KVC_ERR_ARG, "embed: L_cap > 0, H > 0 (multiple of 8), V > 0");
        if (!out || !embed || !ids || !dev_rows || !a16(out) || !a16(embed))
            return set_error(KVC_ERR_ARG, "embed: bad pointers");
        hipLaunchKernelGGL(embed_kernel, dim3(L_cap), dim3(kThreads), 0, (hipStream_t)st, (_Float16*)out,
                           (const _Float16*)embed, ids, V, H, dev_rows);
        return hip_check(hipGetLastError(), "embed launch");
    });
}

int kvc_rmsnorm(void* out, const void* in, const void* w, int L, int H, float eps, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L < 0 || H <= 0 || H % 8 || !(eps >= 0.f)) return set_error(KVC_ERR_ARG, "rmsnorm: bad shape or eps");
        if (L == 0) return KVC_OK;
        if (!out || !in || !w || !a16(out) || !a16(in) || !a16(w)) return set_error(KVC_ERR_ARG, "rmsnorm: bad pointers");
        hipLaunchKernelGGL(rmsnorm_kernel, dim3(L), dim3(kThreads), 0, (hipStream_t)st, (_Float16*)out,
                           (const _Float16*)in, (const _Float16*)w, H, eps);
        return hip_check(hipGetLastError(), "rmsnorm launch");
    });
}

int kvc_add_bias(void* x, const void* bias, int L, int N, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L < 0 || N <= 0 || N % 8) return set_error(KVC_ERR_ARG, "add_bias: bad shape");
        if (L == 0) return KVC_OK;
        if (!x || !bias || !a16(x) || !a16(bias)) return set_error(KVC_ERR_ARG, "add_bias: bad pointers");
        const size_t nvec = (size_t)L * N / 8;
        hipLaunchKernelGGL(bias_kernel, dim3(blocks_for(nvec)), dim3(kThreads), 0, (hipStream_t)st, (_Float16*)x,
                           (const _Float16*)bias, nvec, N / 8);
        return hip_check(hipGetLastError(), "add_bias launch");
    });
}

int kvc_add_residual(void* x, const void* y, size_t n, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (n % 8) return set_error(KVC_ERR_ARG, "add_residual: n must be a multiple of 8");
        if (n == 0) return KVC_OK;
        if (!x || !y || !a16(x) || !a16(y)) return set_error(KVC_ERR_ARG, "add_residual: bad pointers");
        hipLaunchKernelGGL(residual_kernel, dim3(blocks_for(n / 8)), dim3(kThreads), 0, (hipStream_t)st,
                           (_Float16*)x, (const _Float16*)y, n / 8);
        return hip_check(hipGetLastError(), "add_residual launch");
    });
}

int kvc_silu_mul(void* out, const void* gate, const void* up, size_t n, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (n % 8) return set_error(KVC_ERR_ARG, "silu_mul: n must be a multiple of 8");
        if (n == 0) return KVC_OK;
        if (!out || !gate || !up || !a16(out) || !a16(gate) || !a16(up))
            return set_error(KVC_ERR_ARG, "silu_mul: bad pointers");
        hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(n / 8)), dim3(kThreads), 0, (hipStream_t)st,
                           (_Float16*)out, (const _Float16*)gate, (const _Float16*)up, n / 8);
        return hip_check(hipGetLastError(), "silu_mul launch");
    });
}

int kvc_rope(void* x, const int* pos, int pos_base, int L, int n_heads, int D, float theta, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L < 0 || n_heads <= 0 || D <= 0 || D % 2 || !(theta > 1.f)) return set_error(KVC_ERR_ARG, "rope: bad shape");
        if (L == 0) return KVC_OK;
        if (!x) return set_error(KVC_ERR_ARG, "rope: null x");
        const size_t pairs = (size_t)L * n_heads * (D / 2);
        hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(pairs)), dim3(kThreads), 0, (hipStream_t)st, (_Float16*)x, pos,
                           pos_base, pairs, n_heads, D, log2f(theta));
        return hip_check(hipGetLastError(), "rope launch");
    });
}

int kvc_rope_dev(void* x, const int* dev_pos_base, int L, int n_heads, int D, float theta, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L < 0 || n_heads <= 0 || D <= 0 || D % 2 || !(theta > 1.f)) return set_error(KVC_ERR_ARG, "rope: bad shape");
        if (L == 0) return KVC_OK;
        if (!x || !dev_pos_base) return set_error(KVC_ERR_ARG, "rope: null pointer");
        const size_t pairs = (size_t)L * n_heads * (D / 2);
        hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(pairs)), dim3(kThreads), 0, (hipStream_t)st, (_Float16*)x,
                           nullptr, 0, pairs, n_heads, D, log2f(theta), dev_pos_base);
        return hip_check(hipGetLastError(), "rope launch");
    });
}

int kvc_argmax(const float* logits, int L, int V, int* out, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (L < 0 || V <= 0) return set_error(KVC_ERR_ARG, "argmax: bad shape");
        if (L == 0) return KVC_OK;
        if (!logits || !out) return set_error(KVC_ERR_ARG, "argmax: null pointer");
        hipLaunchKernelGGL(argmax_kernel, dim3(L), dim3(kArgThreads), 0, (hipStream_t)st, logits, V, out);
        return hip_check(hipGetLastError(), "argmax launch");
    });
}

int kvc_linear(void* y, const void* x, const void* w, int M, int N, int K, int out_dtype, kvc_stream_t st) {
    return guard_model([&]() -> int {
        if (M < 0 || N <= 0 || K <= 0) return set_error(KVC_ERR_ARG, "linear: bad shape");
        if (out_dtype != KVC_F16 && out_dtype != KVC_F32) return set_error(KVC_ERR_ARG, "linear: bad out dtype");
        if (M == 0) return KVC_OK;
        if (!y || !x || !w) return set_error(KVC_ERR_ARG, "linear: null pointer");
        rocblas_handle h;
        int rc = blas_handle(&h);
        if (rc) return rc;
        if (rocblas_set_stream(h, (hipStream_t)st) != rocblas_status_success)
            return set_error(KVC_ERR_HIP, "rocblas_set_stream failed");
        // row-major y[M,N] = x[M,K] w[N,K]^T  <=>  column-major y^T[N,M] = w^T' [N,K] x^T [K,M]
        const float one = 1.f, zero = 0.f;
        const rocblas_datatype od = out_dtype == KVC_F16 ? rocblas_datatype_f16_r : rocblas_datatype_f32_r;
        const rocblas_status s = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &one,
                                                 w, rocblas_datatype_f16_r, K, x, rocblas_datatype_f16_r, K, &zero, y,
                                                 od, N, y, od, N, rocblas_datatype_f32_r, rocblas_gemm_algo_standard,
                                                 0, 0);
        if (s != rocblas_status_success)
            return set_error(KVC_ERR_HIP, std::string("rocblas_gemm_ex failed: ") + rocblas_status_to_string(s));
        return KVC_OK;
    });
}

}  // extern "C"
