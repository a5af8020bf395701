// decode.hip -- gfx950 decode attention: split phase + log-sum-exp merge.
//
// One wave64 processes one unit = (sequence s, KV head hk, query-head subgroup,
// token chunk [j0, j1)).  Inside a unit the 64 lanes are laid out as
// TPW token slots x LPT lanes per token: every lane owns 16 contiguous bytes of a
// K/V row (8 fp16 or 4 fp32 elements), so one wave-wide 16-byte load reads
// TPW = 64/LPT whole rows.  For D = 64 fp16 that is 8 tokens x 128 B = 1 KiB per
// load instruction, fully coalesced.
//
//   QK^T  : each lane dots its 16-byte slice against q (v_dot2_f32_f16 for fp16,
//           fp32 FMAs for fp32), then an LPT-lane butterfly made of DPP adds
//           (quad_perm, row_half_mirror, row_mirror) finishes the dot product.
//   softmax: every token slot keeps its own fp32 online (max, sum, acc) state in
//           log2 units (exp2 via v_exp_f32); the slots are merged once at the end
//           of the unit, so no per-token barrier or cross-slot exchange exists.
//   GQA   : all G query heads of a KV group are processed by the same wave from
//           the same K/V registers -- each KV byte is read from HBM once.
//   paged : the unit's block-table slice is loaded once into one VGPR (one entry
//           per lane) and each 16-token block's physical id is taken with
//           v_readlane into an SGPR, so K/V addresses are scalar base + constant
//           lane offset (mode kPagedUniform).  kPagedPerLane handles blocks that
//           are smaller than one wave-load (per-lane table lookup).
//
// A unit that covers its whole sequence writes the normalised output directly;
// otherwise it writes (acc[D], m, l) partials and merge_kernel combines them:
//   M = max_c m_c,  out = sum_c 2^(m_c-M) acc_c / sum_c 2^(m_c-M) l_c
// (the flash-decode merge of reference flash_decode.cu:82-101, in log2 units).
// Contiguous and paged layouts share every arithmetic instruction, so paged and
// contiguous results are bit-identical on the same logical data.
#include "internal.hpp"
#include "kvc_abi.h"

#include <cfloat>
#include <climits>

namespace kvc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kThreads = kWave * kWavesPerBlock;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float shfl_xor(float x, int mask) {
    const int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

// Sum over each aligned group of LPT consecutive lanes, result in every lane.
// quad_perm[1,0,3,2] / [2,3,0,1] give the 4-lane sum; row_half_mirror (lane i
// reads 7-i) then adds the other quad of the 8-lane half row, row_mirror (lane i
// reads 15-i) the other half of the 16-lane row.
template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LPT >= 2) x += dpp<0xB1>(x);
    if constexpr (LPT >= 4) x += dpp<0x4E>(x);
    if constexpr (LPT >= 8) x += dpp<0x141>(x);
    if constexpr (LPT >= 16) x += dpp<0x140>(x);
    if constexpr (LPT >= 32) x += shfl_xor(x, 16);
    if constexpr (LPT >= 64) x += shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T> struct Traits;
template <> struct Traits<float> {
    static constexpr int EPL = 4;
    static __device__ __forceinline__ float dot(u32x4 a, u32x4 b) {
        const f32x4 x = __builtin_bit_cast(f32x4, a), y = __builtin_bit_cast(f32x4, b);
        float s = x[0] * y[0];
        s = __builtin_fmaf(x[1], y[1], s);
        s = __builtin_fmaf(x[2], y[2], s);
        s = __builtin_fmaf(x[3], y[3], s);
        return s;
    }
    static __device__ __forceinline__ void to_float(u32x4 a, float* f) {
        const f32x4 x = __builtin_bit_cast(f32x4, a);
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = x[e];
    }
    static __device__ __forceinline__ u32x4 from_float(const float* f) {
        f32x4 x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = f[e];
        return __builtin_bit_cast(u32x4, x);
    }
};
template <> struct Traits<_Float16> {
    static constexpr int EPL = 8;
    static __device__ __forceinline__ float dot(u32x4 a, u32x4 b) {
        const f16x8 x = __builtin_bit_cast(f16x8, a), y = __builtin_bit_cast(f16x8, b);
        float s = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 0, 1), __builtin_shufflevector(y, y, 0, 1), 0.0f, false);
        s = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 2, 3), __builtin_shufflevector(y, y, 2, 3), s, false);
        s = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 4, 5), __builtin_shufflevector(y, y, 4, 5), s, false);
        s = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 6, 7), __builtin_shufflevector(y, y, 6, 7), s, false);
        return s;
    }
    static __device__ __forceinline__ void to_float(u32x4 a, float* f) {
        const f16x8 x = __builtin_bit_cast(f16x8, a);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float)x[e];
    }
    static __device__ __forceinline__ u32x4 from_float(const float* f) {
        f16x8 x;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (_Float16)f[e];
        return __builtin_bit_cast(u32x4, x);
    }
};

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Length and chunk range of unit chunk c of sequence s.  Returns false when the
// unit has no chunk (beyond the sequence's chunk count).
__device__ __forceinline__ bool chunk_range(const DecodeParams& p, int s, int c, int& nc, int& j0, int& j1) {
    int L = p.cur_len ? p.cur_len[s] : p.fixed_len;
    L = L > 0 ? L : 0;
    if (p.num_splits > 0) {
        nc = p.num_splits;
        const int ch = (L + nc - 1) / nc;
        j0 = min(c * ch, L);
        j1 = min(j0 + ch, L);
        return c < nc;
    }
    const int ch = p.chunk_tokens;
    L = min(L, ch * p.max_chunks);  // lengths beyond cap stay inside grid and workspace
    nc = max(1, (L + ch - 1) / ch);
    j0 = c * ch;
    j1 = min(j0 + ch, L);
    return c < nc;
}

// Log-sum-exp merge of the nc chunk partials of (sequence s, query head hq):
//   M = max_c m_c,  out = sum_c 2^(m_c-M) acc_c / sum_c 2^(m_c-M) l_c.
// One wave; lane d owns output dims d, d+64, ...
template <typename T, int D>
__device__ __forceinline__ void merge_head(const DecodeParams& p, int s, int hq, int nc, int lane) {
    constexpr int DPL = (D + kWave - 1) / kWave;
    const size_t rec0 = (size_t)s * p.max_chunks * p.Hq + hq;
    float M = -FLT_MAX;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, p.part_ml[(rec0 + (size_t)c * p.Hq) * 2]);
    float l = 0.f, acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
    for (int c = 0; c < nc; ++c) {
        const size_t rec = rec0 + (size_t)c * p.Hq;
        const float w = fast_exp2(p.part_ml[rec * 2] - M);
        l = __builtin_fmaf(w, p.part_ml[rec * 2 + 1], l);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            const int d = lane + j * kWave;
            if (d < D) acc[j] = __builtin_fmaf(w, p.part_acc[rec * D + d], acc[j]);
        }
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    T* ob = static_cast<T*>(p.out) + ((size_t)s * p.Hq + hq) * D;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
        const int d = lane + j * kWave;
        if (d < D) ob[d] = (T)(acc[j] * inv);
    }
}

// Arrival count of a (sequence, KV head, head subgroup) before this unit, in a
// 64-bit counter tagged with the call's epoch in the high word: a counter from
// another call (or never initialised) counts as zero, and the last arriver
// resets it to zero, so neither fresh nor replayed workspaces need clearing.
__device__ __forceinline__ unsigned arrive(unsigned long long* ctr, unsigned epoch) {
    unsigned long long old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        const unsigned base = (unsigned)(old >> 32) == epoch ? (unsigned)old : 0u;
        const unsigned long long next = ((unsigned long long)epoch << 32) | (unsigned long long)(base + 1u);
        if (__hip_atomic_compare_exchange_strong(ctr, &old, next, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return base;
    }
}

template <typename T, int D, int G, int MODE>
__global__ __launch_bounds__(kThreads) void split_kernel(DecodeParams p) {
    using Tr = Traits<T>;
    constexpr int EPL = Tr::EPL;
    constexpr int LPT = D / EPL;      // lanes per K/V row
    constexpr int TPW = kWave / LPT;  // rows (tokens) per wave-wide load
    constexpr int U = G <= 2 ? 4 : 2; // wave-loads in flight per iteration
    static_assert(LPT >= 1 && LPT <= kWave && D % EPL == 0, "unsupported head_dim");

    const int lane = threadIdx.x & (kWave - 1);
    const int tslot = lane / LPT;
    const int dl = lane % LPT;

    int unit = uniform(blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6));
    const int sub = unit % p.nsub;  unit /= p.nsub;
    const int hk = unit % p.Hkv;    unit /= p.Hkv;
    const int s = unit % p.N;
    const int c = unit / p.N;
    if (c >= p.max_chunks) return;
    int nc, j0, j1;
    if (!chunk_range(p, s, c, nc, j0, j1)) return;
    const int hq0 = hk * p.group + sub * G;

    u32x4 qv[G];
    {
        const T* qb = static_cast<const T*>(p.q) + ((size_t)s * p.Hq + hq0) * D + dl * EPL;
#pragma unroll
        for (int g = 0; g < G; ++g) qv[g] = *reinterpret_cast<const u32x4*>(qb + (size_t)g * D);
    }

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -FLT_MAX;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
    }

    const T* kb = static_cast<const T*>(p.k);
    const T* vb = static_cast<const T*>(p.v);
    const int lane_off = tslot * D + dl * EPL;
    size_t cbase = 0;
    const int* table = nullptr;
    if constexpr (MODE == kContiguous) {
        cbase = (size_t)s * p.seq_stride + (size_t)hk * p.head_stride;
    } else {
        table = p.table_all + (p.tab_off ? p.tab_off[s] : 0);
    }

    // kPagedUniform: block-table window of 64 entries held one per lane.
    int win = 0, tbl = 0, cur_b = 0, cur_in = 0, nblk = 0;
    if constexpr (MODE == kPagedUniform) {
        cur_b = j0 / p.block;
        cur_in = j0 - cur_b * p.block;
        nblk = (j1 + p.block - 1) / p.block;
        win = cur_b;
        if (win + lane < nblk) tbl = table[win + lane];
    }

    for (int base = j0; base < j1; base += U * TPW) {
        u32x4 kr[U], vr[U];
        bool valid[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int t0 = base + i * TPW;
            const int tt = t0 + tslot;
            valid[i] = tt < j1;
            size_t off = 0;
            if constexpr (MODE == kContiguous) {
                off = cbase + (size_t)t0 * D + lane_off;
            } else if constexpr (MODE == kPagedUniform) {
                int phys = 0;
                if (t0 < j1) {
                    if (cur_b - win >= kWave) {
                        win += kWave;
                        tbl = (win + lane < nblk) ? table[win + lane] : 0;
                    }
                    phys = __builtin_amdgcn_readlane(tbl, cur_b - win);
                }
                off = ((size_t)(phys * p.Hkv + hk) * p.block + cur_in) * D + lane_off;
                cur_in += TPW;
                if (cur_in >= p.block) { cur_in -= p.block; ++cur_b; }
            } else {
                int phys = 0, in = 0;
                if (valid[i]) {
                    const int b = tt / p.block;
                    in = tt - b * p.block;
                    phys = table[b];
                }
                off = ((size_t)(phys * p.Hkv + hk) * p.block + in) * D + dl * EPL;
            }
            kr[i] = u32x4{0, 0, 0, 0};
            vr[i] = u32x4{0, 0, 0, 0};
            if (valid[i]) {
                kr[i] = *reinterpret_cast<const u32x4*>(kb + off);
                vr[i] = *reinterpret_cast<const u32x4*>(vb + off);
            }
        }

        float vf[U][EPL];
#pragma unroll
        for (int i = 0; i < U; ++i) Tr::to_float(vr[i], vf[i]);

#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sc[U];
            float mx = m[g];
#pragma unroll
            for (int i = 0; i < U; ++i) {
                sc[i] = group_sum<LPT>(Tr::dot(qv[g], kr[i])) * p.scale_log2;
                mx = valid[i] ? fmaxf(mx, sc[i]) : mx;
            }
            const float corr = fast_exp2(m[g] - mx);
            float pi[U], ps = 0.f;
#pragma unroll
            for (int i = 0; i < U; ++i) {
                pi[i] = valid[i] ? fast_exp2(sc[i] - mx) : 0.f;
                ps += pi[i];
            }
            l[g] = __builtin_fmaf(l[g], corr, ps);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                float a = acc[g][e] * corr;
#pragma unroll
                for (int i = 0; i < U; ++i) a = __builtin_fmaf(pi[i], vf[i][e], a);
                acc[g][e] = a;
            }
            m[g] = mx;
        }
    }

    // Merge the TPW token slots (lanes that differ in bits >= log2(LPT)).
#pragma unroll
    for (int msk = LPT; msk < kWave; msk <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = shfl_xor(m[g], msk), lo = shfl_xor(l[g], msk);
            const float mx = fmaxf(m[g], mo);
            const float ws = fast_exp2(m[g] - mx), wo = fast_exp2(mo - mx);
            l[g] = l[g] * ws + lo * wo;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[g][e] = acc[g][e] * ws + shfl_xor(acc[g][e], msk) * wo;
            m[g] = mx;
        }
    }

    if (nc == 1) {
        if (tslot == 0) {
            T* ob = static_cast<T*>(p.out) + ((size_t)s * p.Hq + hq0) * D + dl * EPL;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float inv = l[g] > 0.f ? 1.0f / l[g] : 0.f;
                float o[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) o[e] = acc[g][e] * inv;
                *reinterpret_cast<u32x4*>(ob + (size_t)g * D) = Tr::from_float(o);
            }
        }
    } else {
        const size_t rec0 = ((size_t)s * p.max_chunks + c) * p.Hq + hq0;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (tslot == 0) {
                float* pa = p.part_acc + (rec0 + g) * D + dl * EPL;
#pragma unroll
                for (int e = 0; e < EPL; e += 4)
                    *reinterpret_cast<f32x4*>(pa + e) = f32x4{acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]};
            }
            if (lane == 0) {
                p.part_ml[(rec0 + g) * 2] = m[g];
                p.part_ml[(rec0 + g) * 2 + 1] = l[g];
            }
        }
        if (p.counters == nullptr) return;  // a separate merge kernel follows
        // Fused merge: publish the partials, count arrivals; the last chunk merges.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        unsigned long long* ctr = p.counters + ((size_t)s * p.Hkv + hk) * p.nsub + sub;
        unsigned before = 0;
        if (lane == 0) before = arrive(ctr, p.epoch);
        before = (unsigned)uniform((int)before);
        if (before != (unsigned)(nc - 1)) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        for (int g = 0; g < G; ++g) merge_head<T, D>(p, s, hq0 + g, nc, lane);
        if (lane == 0) __hip_atomic_store(ctr, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void merge_kernel(DecodeParams p) {
    const int lane = threadIdx.x & (kWave - 1);
    const int w = uniform(blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6));
    if (w >= p.N * p.Hq) return;
    const int s = w / p.Hq, hq = w % p.Hq;
    int nc, j0, j1;
    chunk_range(p, s, 0, nc, j0, j1);
    if (nc <= 1) return;
    merge_head<T, D>(p, s, hq, nc, lane);
}

template <typename T, int D, int G>
int launch_split_mode(const DecodeLaunch& L, dim3 grid, hipStream_t st) {
    switch (L.mode) {
        case kContiguous:   hipLaunchKernelGGL((split_kernel<T, D, G, kContiguous>), grid, dim3(kThreads), 0, st, L.p); break;
        case kPagedUniform: hipLaunchKernelGGL((split_kernel<T, D, G, kPagedUniform>), grid, dim3(kThreads), 0, st, L.p); break;
        case kPagedPerLane: hipLaunchKernelGGL((split_kernel<T, D, G, kPagedPerLane>), grid, dim3(kThreads), 0, st, L.p); break;
        default: return set_error(KVC_ERR_ARG, "unknown decode mode");
    }
    return KVC_OK;
}

template <typename T, int D>
int launch_split_g(const DecodeLaunch& L, dim3 grid, hipStream_t st) {
    if constexpr (D == 64 || D == 128) {
        switch (L.G) {
            case 1: return launch_split_mode<T, D, 1>(L, grid, st);
            case 2: return launch_split_mode<T, D, 2>(L, grid, st);
            case 4: return launch_split_mode<T, D, 4>(L, grid, st);
            case 7: return launch_split_mode<T, D, 7>(L, grid, st);
            case 8: return launch_split_mode<T, D, 8>(L, grid, st);
            default: break;
        }
    } else {
        if (L.G == 1) return launch_split_mode<T, D, 1>(L, grid, st);
    }
    return set_error(KVC_ERR_UNSUPPORTED, "query heads per unit not instantiated");
}

template <typename T>
int launch_typed(const DecodeLaunch& L, hipStream_t st) {
    const long long units = (long long)L.p.max_chunks * L.p.N * L.p.Hkv * L.p.nsub;
    if (units <= 0) return KVC_OK;
    if (units > (long long)INT_MAX - kWavesPerBlock) return set_error(KVC_ERR_ARG, "decode grid too large");
    const dim3 grid((unsigned)((units + kWavesPerBlock - 1) / kWavesPerBlock));
    int rc;
    switch (L.D) {
        case 32:  rc = launch_split_g<T, 32>(L, grid, st); break;
        case 64:  rc = launch_split_g<T, 64>(L, grid, st); break;
        case 128: rc = launch_split_g<T, 128>(L, grid, st); break;
        case 256: rc = launch_split_g<T, 256>(L, grid, st); break;
        default: return set_error(KVC_ERR_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256");
    }
    if (rc != KVC_OK) return rc;
    rc = hip_check(hipGetLastError(), "decode split launch");
    if (rc != KVC_OK || !L.need_merge || L.p.counters != nullptr) return rc;
    const long long waves = (long long)L.p.N * L.p.Hq;
    const dim3 mgrid((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock));
    switch (L.D) {
        case 32:  hipLaunchKernelGGL((merge_kernel<T, 32>), mgrid, dim3(kThreads), 0, st, L.p); break;
        case 64:  hipLaunchKernelGGL((merge_kernel<T, 64>), mgrid, dim3(kThreads), 0, st, L.p); break;
        case 128: hipLaunchKernelGGL((merge_kernel<T, 128>), mgrid, dim3(kThreads), 0, st, L.p); break;
        case 256: hipLaunchKernelGGL((merge_kernel<T, 256>), mgrid, dim3(kThreads), 0, st, L.p); break;
    }
    return hip_check(hipGetLastError(), "decode merge launch");
}

}  // namespace

int launch_decode(const DecodeLaunch& L, hipStream_t stream) {
    if (L.dtype == KVC_F16) return launch_typed<_Float16>(L, stream);
    if (L.dtype == KVC_F32) return launch_typed<float>(L, stream);
    return set_error(KVC_ERR_ARG, "dtype must be KVC_F32 or KVC_F16");
}

}  // namespace kvc
