// append.hip -- K/V row writes into contiguous caches and paged pools, plus a
// deterministic N(0,1) device fill used for synthetic workloads.
//
// Every K/V row ([D] elements of one token and one head) is contiguous in both
// the source [rows, heads, D] and the destination, so a thread moves one
// 16-byte vector and consecutive lanes cover consecutive bytes of a row: one
// wave64 moves eight 128-byte fp16 D=64 rows per instruction, K and V together.
// Destination row per mode:
//   kWriteAppend  : cache[h, start_pos, :] of [H, S, D]            (kv_cache.cu:5-13)
//   kWriteTable   : pool row of position start_pos + r via table    (qwen_kernels.cu:111-122;
//                   start_pos from device memory: kcuda_write_kv, qwen_kernels.cu:128-143)
//   kWriteBatched : pool row of position wpos[r] via table_all+tab_off[r] (qwen_kernels.cu:270-285)
//   kWriteSlots   : pool row of slot_map[r] = phys*BLOCK + in        (slot-mapped form)
// Rows whose position / slot is negative are skipped.
#include "internal.hpp"
#include "kvc_abi.h"

namespace kvc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename W>
__global__ __launch_bounds__(256) void write_kernel(WriteParams p, int vpr) {
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)p.rows * p.heads * vpr;
    if (gid >= total) return;
    const int v = (int)(gid % vpr);
    const long long rh = gid / vpr;
    const int h = (int)(rh % p.heads);
    const int r = (int)(rh / p.heads);
    long long drow;
    if (p.mode == kWriteAppend) {
        drow = (long long)h * p.S + p.start_pos;
    } else {
        int phys, in;
        if (p.mode == kWriteSlots) {
            const int slot = p.idx[r];
            if (slot < 0) return;
            phys = slot / p.block;
            in = slot - phys * p.block;
        } else {
            int pos;
            const int* table = p.table;
            if (p.mode == kWriteTable) {
                pos = (p.dev_start ? *p.dev_start : p.start_pos) + r;
                if (pos < 0) return;
            } else {
                pos = p.idx[r];
                if (pos < 0) return;
                table += p.tab_off[r];
            }
            const int b = pos / p.block;
            phys = table[b];
            in = pos - b * p.block;
        }
        drow = ((long long)phys * p.heads + h) * p.block + in;
    }
    const long long src = rh * vpr + v, dst = drow * vpr + v;
    static_cast<W*>(p.kd)[dst] = static_cast<const W*>(p.k)[src];
    static_cast<W*>(p.vd)[dst] = static_cast<const W*>(p.v)[src];
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Element i takes one output of a Box-Muller pair drawn from hash(seed, i/2).
template <typename T>
__global__ __launch_bounds__(256) void fill_normal_kernel(T* dst, size_t n, uint64_t seed, float stddev) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t h = mix64(seed * 0xD1B54A32D192ED03ull + (i >> 1));
        const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);       // (0, 1]
        const float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);  // [0, 1)
        const float r = sqrtf(-2.0f * logf(u1));
        const float a = 6.283185307179586f * u2;
        const float z = (i & 1) ? r * sinf(a) : r * cosf(a);
        dst[i] = (T)(z * stddev);
    }
}

}  // namespace

int launch_write(const WriteParams& p, int dtype, hipStream_t st) {
    const int esz = dtype == KVC_F16 ? 2 : 4;
    const long long row_bytes = (long long)p.D * esz;
    if (p.rows <= 0 || p.heads <= 0) return KVC_OK;
    const bool vec16 = row_bytes % 16 == 0 &&
                       ((uintptr_t)p.k | (uintptr_t)p.v | (uintptr_t)p.kd | (uintptr_t)p.vd) % 16 == 0;
    const int vpr = vec16 ? (int)(row_bytes / 16) : p.D;
    const long long total = (long long)p.rows * p.heads * vpr;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (vec16) {
        hipLaunchKernelGGL(write_kernel<u32x4>, grid, dim3(256), 0, st, p, vpr);
    } else if (esz == 2) {
        hipLaunchKernelGGL(write_kernel<uint16_t>, grid, dim3(256), 0, st, p, vpr);
    } else {
        hipLaunchKernelGGL(write_kernel<uint32_t>, grid, dim3(256), 0, st, p, vpr);
    }
    return hip_check(hipGetLastError(), "kv write launch");
}

int launch_fill_normal(void* dst, size_t n, int dtype, uint64_t seed, float stddev, hipStream_t st) {
    if (n == 0) return KVC_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (dtype == KVC_F16)
        hipLaunchKernelGGL(fill_normal_kernel<_Float16>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<_Float16*>(dst), n, seed, stddev);
    else
        hipLaunchKernelGGL(fill_normal_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<float*>(dst), n, seed, stddev);
    return hip_check(hipGetLastError(), "fill launch");
}

}  // namespace kvc
