// decode_kernels.hpp -- gfx950 decode attention: split phase + log-sum-exp merge.
// Included by the decode_<type>_d<D>.hip translation units, each of which
// instantiates launch_decode_d<T, D> for one element type and head_dim.
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
#pragma once
#include "internal.hpp"
#include "kvc_abi.h"

#include <cfloat>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <climits>

namespace kvc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float shfl_xor(float x, int mask) {
    const int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

// Lane exchanges across the 16-lane rows and the 32-lane halves in registers
// (gfx950 v_permlane16_swap / v_permlane32_swap): swapping a value with itself
// leaves x[l] in one result and x[l ^ 16] (x[l ^ 32]) in the other, so the pair
// gives max / sum with that partner lane without an LDS round trip.
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
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
// Attended length of sequence s (device lengths, or the fixed/causal length).
__device__ __forceinline__ int seq_len(const DecodeParams& p, int s) {
    return p.cur_len ? p.cur_len[s] : (p.causal ? p.fixed_len + s + 1 : p.fixed_len);
}

// Chunk c of a sequence of L tokens.
__device__ __forceinline__ bool chunk_range_of(const DecodeParams& p, int L, int c, int& nc, int& j0, int& j1) {
    L = min(max(L, 0), p.cap);  // (longer sequences never get here: their units write NaN)
    if (p.num_splits > 0) {
        nc = p.num_splits;
        const int ch = (L + nc - 1) / nc;
        j0 = min(c * ch, L);
        j1 = min(j0 + ch, L);
        return (unsigned)c < (unsigned)nc;  // c in [0, nc)
    }
    const int ch = p.chunk_tokens;
    L = min(L, ch * p.max_chunks);  // lengths beyond cap stay inside grid and workspace
    nc = max(1, (L + ch - 1) / ch);
    j0 = c * ch;
    j1 = min(j0 + ch, L);
    return (unsigned)c < (unsigned)nc;  // c in [0, nc)
}

__device__ __forceinline__ bool chunk_range(const DecodeParams& p, int s, int c, int& nc, int& j0, int& j1) {
    return chunk_range_of(p, seq_len(p, s), c, nc, j0, j1);
}

// Log-sum-exp merge of the nc chunk partials of one query head: chunk c's
// record is rec0 + c*cstride (acc at record*D, (m, l) at record*2):
//   M = max_c m_c,  out = sum_c 2^(m_c-M) acc_c / sum_c 2^(m_c-M) l_c.
// One wave.  The chunk statistics (one chunk per lane) and the accumulators of
// the first eight chunks are read in one round of independent loads; the
// statistics are reduced across the wave, and lane d accumulates output dims d,
// d+64, ... with each chunk's weight taken from the lane that holds it (further
// chunks eight at a time).  COHERENT reads the
// partials with agent-scope atomic loads (partials written by other XCDs bypass
// stale L2 lines); otherwise plain loads after an acquire fence.
template <typename T, int D, bool COHERENT>
__device__ __forceinline__ void merge_head(const DecodeParams& p, size_t rec0, size_t cstride, int nc, T* ob,
                                           int lane) {
    constexpr int DPL = (D + kWave - 1) / kWave;
    constexpr int E = 8;  // chunk partials in flight per lane
    auto ld = [](const float* a) {
        if constexpr (COHERENT) return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else return *a;
    };
    auto rec_of = [&](int c) { return rec0 + (size_t)c * cstride; };
    // statistics of up to 64 chunks and the accumulators of the first E chunks in
    // one round of independent loads
    const bool in0 = lane < nc;
    const size_t r0 = rec_of(in0 ? lane : 0);
    const float m0 = in0 ? ld(p.part_ml + r0 * 2) : -FLT_MAX;
    const float l0 = in0 ? ld(p.part_ml + r0 * 2 + 1) : 0.f;
    float a0[E][DPL];
#pragma unroll
    for (int u = 0; u < E; ++u)
#pragma unroll
        for (int j = 0; j < DPL; ++j)
            a0[u][j] = u < nc ? ld(p.part_acc + rec_of(u) * D + min(lane + j * kWave, D - 1)) : 0.f;
    float M = m0;
    for (int c0 = kWave; c0 < nc; c0 += kWave) {
        const int c = c0 + lane;
        M = fmaxf(M, c < nc ? ld(p.part_ml + rec_of(c) * 2) : -FLT_MAX);
    }
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) M = fmaxf(M, shfl_xor(M, o));
    float l = 0.f, acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
    for (int c0 = 0; c0 < nc; c0 += kWave) {
        const int c = c0 + lane;
        const bool in = c < nc;
        float w;
        if (c0 == 0) {
            w = in ? fast_exp2(m0 - M) : 0.f;
            l += in ? w * l0 : 0.f;
        } else {
            const size_t rc = rec_of(in ? c : c0);
            w = in ? fast_exp2(ld(p.part_ml + rc * 2) - M) : 0.f;
            l += in ? w * ld(p.part_ml + rc * 2 + 1) : 0.f;
        }
        const int cn = min(kWave, nc - c0);
        int e = 0;
        if (c0 == 0) {
#pragma unroll
            for (int u = 0; u < E; ++u) {
                const float we = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc[j] = __builtin_fmaf(we, a0[u][j], acc[j]);  // 0 past nc
            }
            e = E;
        }
        for (; e + E <= cn; e += E) {
            float a[E][DPL], we[E];
#pragma unroll
            for (int u = 0; u < E; ++u) {
                we[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), e + u));
#pragma unroll
                for (int j = 0; j < DPL; ++j) a[u][j] = ld(p.part_acc + rec_of(c0 + e + u) * D + min(lane + j * kWave, D - 1));
            }
#pragma unroll
            for (int u = 0; u < E; ++u)
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc[j] = __builtin_fmaf(we[u], a[u][j], acc[j]);
        }
        for (; e < cn; ++e) {
            const float we = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), e));
#pragma unroll
            for (int j = 0; j < DPL; ++j)
                acc[j] = __builtin_fmaf(we, ld(p.part_acc + rec_of(c0 + e) * D + min(lane + j * kWave, D - 1)), acc[j]);
        }
    }
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) l += shfl_xor(l, o);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
        const int d = lane + j * kWave;
        if (d < D) ob[d] = (T)(acc[j] * inv);
    }
}

// Arrival count of a (sequence, KV head, head subgroup) before this unit, in a
// 64-bit counter holding the call's epoch in the low word and the count in the high
// word (counts never carry into the epoch): a counter from another call, reset, or
// never initialised counts as zero, and the last arriver resets it to zero, so
// neither fresh nor replayed workspaces need clearing.  An arrival is one
// fetch-and-add; only when that returns another call's tag (the first arrivals of a
// call) does the arriver adopt the counter with a compare-and-swap to (epoch, 1),
// which discards the additions made to the stale value -- each of their arrivers
// sees the stale tag too and comes through here.
__device__ __forceinline__ unsigned arrive(unsigned long long* ctr, unsigned epoch) {
    constexpr unsigned long long kOne = 1ull << 32;
    unsigned long long old = __hip_atomic_fetch_add(ctr, kOne, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((unsigned)old == epoch) return (unsigned)(old >> 32);
    old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        if ((unsigned)old == epoch)
            return (unsigned)(__hip_atomic_fetch_add(ctr, kOne, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32);
        if (__hip_atomic_compare_exchange_strong(ctr, &old, kOne | epoch, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return 0u;
    }
}

// The parameter block of a decode kernel (its third argument, at byte 16 of the
// kernarg segment after the work pointer and its int), read through a pointer the
// compiler cannot prove loop-invariant.  A persistent loop would otherwise keep
// every field it uses in scalar registers across all its iterations (some 60
// registers, spilled into vector lanes); a fresh copy per unit lives only as long
// as the unit that uses it.  The loads stay scalar (constant address space).
constexpr int kParamsKernargOffset = 16;
__device__ __forceinline__ DecodeParams fresh_params() {
    static_assert(alignof(DecodeParams) == 8 && sizeof(const int*) == 8, "kernarg layout");
#if defined(__HIP_DEVICE_COMPILE__)  // (the host pass only parses device functions)
    typedef __attribute__((address_space(4))) const char* KArg;
    typedef __attribute__((address_space(4))) const DecodeParams* KParams;
    KArg ka = (KArg)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ka));
    return *(KParams)(ka + kParamsKernargOffset);
#else
    return DecodeParams{};
#endif
}

// K/V registers of U wave-loads: the double-buffered unit of the inner loop.
template <int U>
struct Batch {
    u32x4 k[U], v[U];
    int k0;  // this wave's index of the batch's first wave-load
};

// Buffer descriptor over `bytes` bytes at `base` (raw, unswizzled, 32-bit data
// format).  Loads whose offset is >= bytes return 0 and touch no memory.
constexpr int kBufferWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kBufferWord3);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, int voffset) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0);
}

// The unit of a workgroup: from the planned work list or from the
// (chunk, sequence, KV head, subgroup) decomposition of the grid.
struct Unit {
    int s, hk, sub, c, nc, j0, j1, tab_start;
    int n_inline = 0;  // planned grouped-query units: block ids carried in the entry
    bool over_cap = false;  // device-length grid: the sequence is longer than the stated cap
    size_t rec0, cstride, ctr_idx;
};

// NaN in the output rows of `heads` query heads from hq0 of sequence s: what a
// sequence longer than the launch's stated cap gets instead of a silently
// truncated attention.
// The failure is also reported to the host: thread 0 stores `code` into the launch's
// error word (pinned host memory, a system-scope store), which the library returns as a
// status from kvc_check_device_errors and from the next device-length decode call.
__device__ __forceinline__ void report_device_error(const DecodeParams& p, int code) {
    if (p.err_word != nullptr && threadIdx.x == 0)
        __hip_atomic_store(p.err_word, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <typename T, int D, int NT>
__device__ void nan_rows(const DecodeParams& p, int s, int hq0, int heads) {
    T* ob = static_cast<T*>(p.out) + ((size_t)s * p.Hq + hq0) * D;
    for (int e = threadIdx.x; e < heads * D; e += NT) ob[e] = (T)__builtin_nanf("");
    report_device_error(p, kDevErrCap);
}

// The 8-int header of this workgroup's planned entry.  The kernels take the work
// list as their first, register-preloaded arguments and read the header before
// anything else, so it is in flight alongside the fetch of the parameter block; the
// grid never exceeds the entries allocated, so it is read before the device-count
// check.
__device__ __forceinline__ void read_header(const int* work, int work_ints, int (&h)[8]) {
    const int* w = work + (size_t)blockIdx.x * work_ints;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = w[i];
}

// Device-length decomposition: the length and table offset of this workgroup's
// sequence, read at kernel entry (h[0], h[1]) so both are in flight together
// with the rest of the parameter block.  Branch-free: s < N for every workgroup
// of the grid, and a missing array is a zero-size descriptor that reads 0.
template <bool PAGED>
__device__ __forceinline__ void read_seq(const DecodeParams& p, int (&h)[8]) {
    // the scalars load_unit needs come with the first fetch of the parameter block
    // (left to itself the compiler fetches them in a second round, after this one)
    asm volatile("" ::"s"(p.max_chunks), "s"(p.fixed_len), "s"(p.causal), "s"(p.cap), "s"(p.last_chunk_first));
    const int s = (int)(blockIdx.x / (unsigned)(p.max_chunks * p.nsub * p.Hkv));  // < N: load_unit's order
    h[0] = (int)__builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(p.cur_len, p.cur_len ? p.N * 4 : 0), s * 4, 0, 0);
    h[1] = (int)__builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(p.tab_off, PAGED && p.tab_off ? p.N * 4 : 0),
                                                     s * 4, 0, 0);
    // keep the scheduler from sinking the loads below work that waits for the
    // rest of the parameter block
    __builtin_amdgcn_sched_barrier(0);
}

// h: the planned entry's header, or read_seq's values for the device-length
// decomposition.
template <bool PLANNED, bool PAGED = true>
__device__ __forceinline__ bool load_unit(const DecodeParams& p, const int (&h)[8], int heads, Unit& u) {
    if constexpr (PLANNED) {
        int N = p.N, n_records = p.n_records;
        if (p.dev_counts) {  // fixed-capacity grid: the step's counts come from device memory
            if ((int)blockIdx.x >= p.dev_counts[1]) return false;
            N = min(p.dev_counts[0], p.N);
            n_records = min(p.dev_counts[2], p.n_records);
        }
        u.s = h[0];
        const int hks = h[1] & 0xFFFF;
        u.c = h[1] >> 16;
        u.hk = hks / p.nsub;
        u.sub = hks % p.nsub;
        u.j0 = max(h[2], 0);
        u.j1 = max(h[3], u.j0);
        u.nc = max(h[4] & 0xFFFF, 1);
        u.n_inline = (unsigned)h[4] >> 16;
        u.rec0 = ((size_t)(h[5] > 0 ? h[5] : 0) + (size_t)u.c) * heads;
        u.cstride = heads;
        u.ctr_idx = h[6] > 0 ? h[6] : 0;
        u.tab_start = h[7];
        // a unit outside the launch's shape (a stale or foreign plan) is skipped
        if (u.s < 0 || u.s >= N || u.hk < 0 || u.hk >= p.Hkv || u.c < 0 || u.c >= u.nc) return false;
        return u.nc == 1 || (h[5] >= 0 && (long long)h[5] + u.nc <= n_records && h[6] >= 0 && h[6] < n_records);
    } else {
        // chunk fastest: the hardware deals consecutive workgroups to the 8 XCDs in
        // turn, so every sequence's chunks spread evenly over the XCDs (with the
        // sequence fastest, blockIdx % 8 picked the (sequence, head) and an XCD holding
        // the long sequences streamed twice its share through its fabric link)
        int unit = blockIdx.x;
        const int cr = unit % p.max_chunks;  unit /= p.max_chunks;
        u.sub = unit % p.nsub;  unit /= p.nsub;
        u.hk = unit % p.Hkv;    unit /= p.Hkv;
        u.s = unit;
        u.c = p.last_chunk_first ? p.max_chunks - 1 - cr : cr;
        // length and table offset: read_seq (c >= max_chunks needs no test of its
        // own: nc <= max_chunks, so chunk_range_of rejects it)
        const int lu = uniform(h[0]);
        const int L = p.cur_len ? lu : (p.causal ? p.fixed_len + u.s + 1 : p.fixed_len);
        u.tab_start = uniform(h[1]);
        if (L > p.cap) {  // the grid and workspace do not cover it: chunk 0's unit writes NaN
            u.over_cap = u.c == 0;
            return false;
        }
        if (!chunk_range_of(p, L, u.c, u.nc, u.j0, u.j1)) return false;
        u.rec0 = ((size_t)u.s * p.max_chunks + u.c) * p.Hq + u.hk * p.group + u.sub * heads;
        u.cstride = p.Hq;
        u.ctr_idx = ((size_t)u.s * p.Hkv + u.hk) * p.nsub + u.sub;
        return true;
    }
}

#include "selfplan.hpp"

// Largest chunk, in blocks, the per-lane paged path stages in LDS.
constexpr int kMaxChunkBlocks = 4096;

// One workgroup of WPB waves per unit (sequence s, KV head hk, head subgroup,
// chunk c).  The chunk's wave-loads (TPW tokens each) are dealt round-robin to
// the waves; every wave keeps two batches of U wave-loads in flight (ping-pong)
// and its own online-softmax state per token slot.  Loads carry no control flow:
// contiguous and uniform-paged tiles are read with buffer loads whose descriptor
// covers exactly the tile's valid rows (rows past the chunk read as 0 and cost
// no memory traffic), so the compiler can count outstanding loads exactly and
// the next batch streams while the current one is consumed.  At the end the
// token slots are merged with lane shuffles, the waves through LDS, and wave 0
// writes either the normalised output (single-chunk sequence) or the chunk
// partial, optionally followed by the fused cross-chunk merge.
template <typename T, int D, int G, int MODE, int WPB, int U>
__global__ __launch_bounds__(WPB * kWave) void split_kernel(const int* __restrict__ work, int work_ints, DecodeParams p_arg) {
    const DecodeParams& p = p_arg;
    using Tr = Traits<T>;
    constexpr int EPL = Tr::EPL;
    constexpr int LPT = D / EPL;      // lanes per K/V row
    constexpr int TPW = kWave / LPT;  // rows (tokens) per wave-wide load
    constexpr int ROW = D * (int)sizeof(T);  // bytes per K/V row
    static_assert(LPT >= 1 && LPT <= kWave && D % EPL == 0, "unsupported head_dim");
    constexpr bool SELF = MODE == kSelfPlanned || MODE == kSelfContig;
    constexpr bool CONTIG = MODE == kContiguous || MODE == kSelfContig;
    constexpr bool PLANNED = MODE == kPlannedUniform || MODE == kPlannedPerLane || SELF;
    constexpr bool UNIFORM = MODE == kPagedUniform || MODE == kPlannedUniform || SELF;
    constexpr bool PER_LANE = MODE == kPagedPerLane || MODE == kPlannedPerLane;
    __shared__ float s_acc[WPB][G][D];
    __shared__ float s_m[WPB][G], s_l[WPB][G];
    __shared__ int s_tab[PER_LANE ? kMaxChunkBlocks : 1];
    __shared__ std::conditional_t<SELF, SelfPlanLds<kSelfMaxNValu, WPB, true>, char> s_plan;
    // self-planned short sequences: the partials of waves 1 .. WPB-1, kept until lead_finish
    constexpr int LW = SELF ? WPB - 1 : 1;
    __shared__ float s_lacc[LW][G][D];
    __shared__ float s_lm[LW][G], s_ll[LW][G];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = uniform(threadIdx.x >> 6);

    // One unit, given its entry header (hdr) and, on the host-planned path, the
    // entry's block ids (ev: one int per lane after the 8-int header).  LEAD: a short
    // sequence of a self-planned launch, whole, on waves 1 .. WPB-1 while wave 0 plans
    // (hdr = {sequence, head subgroup, length, first table entry}); its partials stay
    // in LDS (s_lacc) for lead_finish.
    auto body = [&](auto lead_tag, const int (&hdr)[8], const int ev) {
    constexpr bool LEAD = decltype(lead_tag)::value;
    constexpr int NW = LEAD ? WPB - 1 : WPB;  // waves that share the unit's wave-loads
    // self-planned (persistent) launches: the parameters and per-lane indices are
    // derived anew in every unit, not hoisted out of the loop and held across it
    const DecodeParams p = SELF ? fresh_params() : p_arg;
    int tid_u = threadIdx.x;
    if constexpr (SELF) asm volatile("" : "+v"(tid_u));
    const int lane = tid_u & (kWave - 1);
    const int tslot = lane / LPT;
    const int dl = lane % LPT;
    const int wv = LEAD ? wave - 1 : wave;
    Unit u;
    if constexpr (LEAD) {
        u.s = hdr[0];
        u.hk = hdr[1] / p.nsub;
        u.sub = hdr[1] - u.hk * p.nsub;
        u.c = 0;
        u.nc = 1;
        u.j0 = 0;
        u.j1 = min(max(hdr[2], 0), p.cap);  // (a length past the cap fails the plan: NaN rows)
        u.tab_start = hdr[3];
        u.rec0 = u.cstride = u.ctr_idx = 0;
    } else if (!load_unit<PLANNED, !CONTIG>(p, hdr, G, u)) {
        if (u.over_cap) nan_rows<T, D, WPB * kWave>(p, u.s, u.hk * p.group + u.sub * G, G);
        return;
    }
    const int s = u.s, hk = u.hk, sub = u.sub, c = u.c, nc = u.nc, j0 = u.j0, j1 = u.j1;
    const int tab_start = u.tab_start;
    const int n_inl = u.n_inline;  // block ids carried by the planned entry
    const size_t rec0 = u.rec0, cstride = u.cstride, ctr_idx = u.ctr_idx;
    const int hq0 = hk * p.group + sub * G;
    const int nwl = (j1 - j0 + TPW - 1) / TPW;                          // wave-loads in the chunk
    const int kmax = wv < nwl ? (nwl - wv + NW - 1) / NW : 0;           // this wave's share

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

    const char* kb = static_cast<const char*>(p.k);
    const char* vb = static_cast<const char*>(p.v);
    size_t cbase = 0;         // contiguous: byte offset of (s, hk, token 0)
    int tbl = 0;              // uniform paged: block ids of the chunk, one per lane
    const int b0 = j0 / p.block;
    // fused append: the new row's slice of this lane, used in place of the pool's
    // when the chunk holds its position (loads issued without waiting for wpos)
    int wp = -1;
    u32x4 knew = {0, 0, 0, 0}, vnew = {0, 0, 0, 0};
    if constexpr (PLANNED && !LEAD) {
        if (p.wpos != nullptr) {
            const size_t row = ((size_t)s * p.Hkv + hk) * ROW + dl * 16;
            knew = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.k_new) + row);
            vnew = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.v_new) + row);
            const int w = p.wpos[s];
            wp = (w >= j0 && w < j1) ? w : -1;
        }
    }
    if constexpr (CONTIG) {
        cbase = ((size_t)s * p.seq_stride + (size_t)hk * p.head_stride) * sizeof(T);
    } else {
        // blocks the chunk touches (0 for an empty chunk); the planner keeps this
        // within kMaxChunkBlocks, the min() only guards the LDS staging
        const int nblk = min(j1 > j0 ? (j1 - 1) / p.block - b0 + 1 : 0, kMaxChunkBlocks);
        // The block ids are read through a descriptor: on the planned path the
        // descriptor spans table_all (table_len ints), so any plan reads inside it;
        // otherwise it spans this chunk's nblk entries.
        // (a short sequence of a self-planned launch: its own entries)
        constexpr bool WHOLE_TABLE = PLANNED && !LEAD;
        const int first = tab_start + (PLANNED ? 0 : b0);
        const __amdgpu_buffer_rsrc_t trs =
            WHOLE_TABLE ? tile_rsrc(p.table_all, p.table_len * 4) : tile_rsrc(p.table_all + first, nblk * 4);
        const int tb = WHOLE_TABLE ? first * 4 : 0;  // byte offset of the chunk's first entry
        if constexpr (UNIFORM) {
            // unconditional: lanes past the chunk's blocks read a neighbour's id or 0 and
            // are never selected by the readlane below
            tbl = (int)__builtin_amdgcn_raw_buffer_load_b32(trs, tb + lane * 4, 0, 0);
        } else {
            for (int b = threadIdx.x; b < nblk; b += WPB * kWave)
                s_tab[b] = (int)__builtin_amdgcn_raw_buffer_load_b32(trs, tb + b * 4, 0, 0);
            __syncthreads();
        }
        // fused append: one unit per (sequence, KV head) stores the new row in the pool
        if (PLANNED && wp >= 0 && sub == 0 && wave == 0 && lane < LPT) {
            const int rel = wp / p.block - b0;
            int phys;
            if constexpr (UNIFORM) phys = __builtin_amdgcn_readlane(tbl, min(rel, kWave - 1));
            else phys = s_tab[min(rel, kMaxChunkBlocks - 1)];
            const size_t off = ((size_t)(phys * p.Hkv + hk) * p.block + wp % p.block) * ROW + lane * 16;
            *reinterpret_cast<u32x4*>(const_cast<char*>(kb) + off) = knew;
            *reinterpret_cast<u32x4*>(const_cast<char*>(vb) + off) = vnew;
        }
    }

    auto issue = [&](int k0, Batch<U>& b) {
        b.k0 = k0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = wv + NW * (k0 + u);      // wave-load index within the chunk
            const int t0 = j0 + i * TPW;
            if constexpr (PER_LANE) {
                int tt = t0 + tslot;
                const bool ok = tt < j1;
                tt = ok ? tt : j0;                     // a valid row; the value is discarded below
                const int bb = tt / p.block;
                const int phys = s_tab[bb - b0];
                const size_t off = ((size_t)(phys * p.Hkv + hk) * p.block + (tt - bb * p.block)) * ROW + dl * 16;
                const u32x4 kk = *reinterpret_cast<const u32x4*>(kb + off);
                const u32x4 vv = *reinterpret_cast<const u32x4*>(vb + off);
                b.k[u] = kk;
                b.v[u] = ok ? vv : u32x4{0, 0, 0, 0};
            } else {
                // valid rows of this wave-load, kept in scalar registers (the descriptor
                // lives in SGPRs; the empty asm stops the clamp from becoming a vector
                // med3, whose temporary could land on a register with a load in flight
                // and make the issue wait)
                int rows = max(j1 - t0, 0);
                asm("" : "+s"(rows));
                rows = min(rows, TPW);
                size_t tile;
                if constexpr (CONTIG) {
                    tile = cbase + (size_t)max(t0, 0) * ROW;
                } else {
                    const int rel = i >> p.lpb_shift;           // block of the chunk
                    int phys;
                    if (PLANNED && rel < n_inl) phys = __builtin_amdgcn_readlane(ev, 8 + min(rel, kWave - 9));
                    else phys = __builtin_amdgcn_readlane(tbl, min(rel, kWave - 1));
                    const int in = (i & ((1 << p.lpb_shift) - 1)) * TPW;
                    tile = ((size_t)(phys * p.Hkv + hk) * p.block + in) * ROW;
                }
                b.k[u] = buffer_load16(tile_rsrc(kb + tile, rows * ROW), lane * 16);
                b.v[u] = buffer_load16(tile_rsrc(vb + tile, rows * ROW), lane * 16);
            }
        }
    };

    auto consume = [&](const Batch<U>& b) {
        bool valid[U];
        float vf[U][EPL];
        u32x4 kq[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tok = j0 + (wv + NW * (b.k0 + u)) * TPW + tslot;
            valid[u] = tok < j1;
            kq[u] = tok == wp ? knew : b.k[u];
            Tr::to_float(tok == wp ? vnew : b.v[u], vf[u]);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sc[U];
            float mx = m[g];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                sc[u] = group_sum<LPT>(Tr::dot(qv[g], kq[u])) * p.scale_log2;
                mx = valid[u] ? fmaxf(mx, sc[u]) : mx;
            }
            const float corr = fast_exp2(m[g] - mx);
            float pu[U], ps = 0.f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                pu[u] = valid[u] ? fast_exp2(sc[u] - mx) : 0.f;
                ps += pu[u];
            }
            l[g] = __builtin_fmaf(l[g], corr, ps);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                float a = acc[g][e] * corr;
#pragma unroll
                for (int u = 0; u < U; ++u) a = __builtin_fmaf(pu[u], vf[u][e], a);
                acc[g][e] = a;
            }
            m[g] = mx;
        }
    };

    if (kmax > 0) {
        Batch<U> A, B;
        issue(0, A);
        for (int k = 0;; k += 2 * U) {
            issue(k + U, B);          // past the end it reads nothing (zero-size tiles)
            consume(A);
            if (k + U >= kmax) break;
            issue(k + 2 * U, A);
            consume(B);
            if (k + 2 * U >= kmax) break;
        }
    }

    // Merge the TPW token slots of the wave (lanes that differ in bits >= log2(LPT)).
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
    if constexpr (LEAD) {  // lead_finish combines the waves' partials
        if (tslot == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < EPL; ++e) s_lacc[wv][g][dl * EPL + e] = acc[g][e];
        }
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                s_lm[wv][g] = m[g];
                s_ll[wv][g] = l[g];
            }
        }
        return;
    }
    if (tslot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_acc[wave][g][dl * EPL + e] = acc[g][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            s_m[wave][g] = m[g];
            s_l[wave][g] = l[g];
        }
    }
    __syncthreads();
    if (wave != 0) return;

    // Wave 0 merges the WPB wave partials: lane handles (g, d) = divmod(idx, D).
    T* ob = static_cast<T*>(p.out) + ((size_t)s * p.Hq + hq0) * D;
    for (int idx = lane; idx < G * D; idx += kWave) {
        const int g = idx / D, d = idx % D;
        float M = -FLT_MAX;
#pragma unroll
        for (int w = 0; w < WPB; ++w) M = fmaxf(M, s_m[w][g]);
        float lt = 0.f, at = 0.f;
#pragma unroll
        for (int w = 0; w < WPB; ++w) {
            const float wt = fast_exp2(s_m[w][g] - M);
            lt = __builtin_fmaf(wt, s_l[w][g], lt);
            at = __builtin_fmaf(wt, s_acc[w][g][d], at);
        }
        if (nc == 1) {
            ob[(size_t)g * D + d] = (T)(lt > 0.f ? at * (1.0f / lt) : 0.f);
        } else if (p.merge_mode == kMergeAtomic) {
            __hip_atomic_store(p.part_acc + (rec0 + g) * D + d, at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(p.part_ml + (rec0 + g) * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(p.part_ml + (rec0 + g) * 2 + 1, lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            p.part_acc[(rec0 + g) * D + d] = at;
            if (d == 0) {
                p.part_ml[(rec0 + g) * 2] = M;
                p.part_ml[(rec0 + g) * 2 + 1] = lt;
            }
        }
    }
    if (nc == 1 || p.merge_mode == kMergeKernel) return;  // single chunk, or a merge kernel follows
    // Fused merge: publish the partials, count arrivals; the last chunk merges.
    if (p.merge_mode == kMergeAtomic) {
        // the partial stores were coherent; wait until this wave's stores completed
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    }
    unsigned long long* ctr = p.counters + ctr_slot(ctr_idx, p.ctr_shift);
    unsigned before = 0;
    if (lane == 0) before = arrive(ctr, p.epoch);
    before = (unsigned)uniform((int)before);
    if (before != (unsigned)(nc - 1)) return;
    const size_t first = rec0 - (size_t)c * cstride;  // record of chunk 0, head 0
    if (p.merge_mode == kMergeAtomic) {
        for (int g = 0; g < G; ++g) merge_head<T, D, true>(p, first + g, cstride, nc, ob + (size_t)g * D, lane);
    } else {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        for (int g = 0; g < G; ++g) merge_head<T, D, false>(p, first + g, cstride, nc, ob + (size_t)g * D, lane);
    }
    if (lane == 0) __hip_atomic_store(ctr, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };  // body
    auto run_unit = [&](const int (&hdr)[8], const int ev) { body(std::false_type{}, hdr, ev); };

    if constexpr (SELF) {
        // waves 1 ..: sequence b / hks, head subgroup b % hks, when it is short
        auto lead = [&]() -> bool {
            const DecodeParams p = fresh_params();
            const int hks = p.Hkv * p.nsub, b = (int)blockIdx.x;
            if (b >= p.N * hks) return false;
            const int s = b / hks;
            const int L = p.cur_len[s];
            if (L > p.sp_lead) return false;
            const int hdr[8] = {s, b - s * hks, L, p.tab_off ? p.tab_off[s] : 0, 0, 0, 0, 0};
            body(std::true_type{}, hdr, 0);
            return true;
        };
        // wave 1, once the plan (and the lengths) are in LDS: the output of that short
        // sequence from the lead waves' partials
        auto lead_finish = [&]() {
            if (wave != 1) return;
            const DecodeParams p = fresh_params();
            const int hks = p.Hkv * p.nsub, b = (int)blockIdx.x;
            if (b >= p.N * hks) return;
            const int s = b / hks, hh = b - s * hks;
            if (uniform(s_plan.len[s]) > p.sp_lead) return;
            const int hk = hh / p.nsub, sub = hh - hk * p.nsub;
            T* ob = static_cast<T*>(p.out) + ((size_t)s * p.Hq + hk * p.group + sub * G) * D;
            for (int idx = lane; idx < G * D; idx += kWave) {
                const int g = idx / D, d = idx % D;
                float M = -FLT_MAX;
#pragma unroll
                for (int w = 0; w < LW; ++w) M = fmaxf(M, s_lm[w][g]);
                float lt = 0.f, at = 0.f;
#pragma unroll
                for (int w = 0; w < LW; ++w) {
                    const float wt = fast_exp2(s_lm[w][g] - M);
                    lt = __builtin_fmaf(wt, s_ll[w][g], lt);
                    at = __builtin_fmaf(wt, s_lacc[w][g][d], at);
                }
                ob[(size_t)g * D + d] = (T)(lt > 0.f ? at * (1.0f / lt) : 0.f);
            }
        };
        // self-planned launches pass the device lengths as the (preloaded) first argument
        self_plan_loop<T, D, WPB * kWave>(work, work_ints, s_plan, G, [&](const int (&hdr)[8]) { run_unit(hdr, 0); },
                                          lead, lead_finish);
    } else {
        // planned entries may carry the chunk's first block ids after the 8-int
        // header (one int per lane, read together with the header), so the first
        // batch of loads does not wait for the table
        int ev = 0;
        if constexpr (PLANNED && UNIFORM) {
            if (work_ints > 8 && lane < work_ints) ev = work[(size_t)blockIdx.x * work_ints + lane];
        }
        int hdr[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (PLANNED) read_header(work, work_ints, hdr);
        else read_seq<!CONTIG>(p, hdr);
        run_unit(hdr, ev);
    }
}

// Standalone log-sum-exp merge: one 512-thread workgroup per (sequence, query
// head); MG = 512/D chunk groups x D dims.  The sequence's length and the first
// kMergeBatch records of every chunk group are loaded in ONE round: the record
// loads run ahead of the chunk count (indices clamped below max_chunks, inside
// the workspace) and records at or past the count are dropped by selects, so
// stale workspace contents never reach the sum.  Each thread reduces its records
// with its own maximum, later batches (more than kMergeBatch * MG chunks) are
// folded in with a rescale, and the groups combine through LDS:
//   M = max_g M_g,  out = sum_g 2^(M_g-M) acc_g / sum_g 2^(M_g-M) l_g.
// Sequences with a single chunk were finished by the split kernel.
constexpr int kMergeThreads = 512;
constexpr int kMergeBatch = 8;

template <typename T, int D>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(DecodeParams p) {
    constexpr int MG = kMergeThreads / D;  // chunk groups
    __shared__ float s_acc[MG][D];
    __shared__ float s_ml[MG][2];
    const int t = threadIdx.x;
    const int s = blockIdx.x / p.Hq, hq = blockIdx.x % p.Hq;
    const int cg = t / D, d = t % D;
    const size_t rec0 = (size_t)s * p.max_chunks * p.Hq + hq;
    const size_t cstride = (size_t)p.Hq;  // records between consecutive chunks
    const int cmax = p.max_chunks;

    float mm[kMergeBatch], ll[kMergeBatch], aa[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {  // unconditional loads: no branch waits between them
        const size_t rec = rec0 + (size_t)min(cg + u * MG, cmax - 1) * cstride;
        const float2 ml = *reinterpret_cast<const float2*>(p.part_ml + rec * 2);
        mm[u] = ml.x; ll[u] = ml.y;
        aa[u] = p.part_acc[rec * D + d];
    }
    int nc, j0, j1;
    chunk_range(p, s, 0, nc, j0, j1);
    if (nc <= 1 || seq_len(p, s) > p.cap) return;  // one chunk, or NaN rows from the split kernel

    float M = -FLT_MAX;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) M = cg + u * MG < nc ? fmaxf(M, mm[u]) : M;
    float at = 0.f, lt = 0.f;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
        const bool ok = cg + u * MG < nc;
        const float w = fast_exp2(mm[u] - M);
        lt = ok ? __builtin_fmaf(w, ll[u], lt) : lt;
        at = ok ? __builtin_fmaf(w, aa[u], at) : at;
    }
    for (int c0 = kMergeBatch * MG; c0 < nc; c0 += kMergeBatch * MG) {
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const size_t rec = rec0 + (size_t)min(c0 + cg + u * MG, nc - 1) * cstride;
            const float2 ml = *reinterpret_cast<const float2*>(p.part_ml + rec * 2);
            mm[u] = ml.x; ll[u] = ml.y;
            aa[u] = p.part_acc[rec * D + d];
        }
        float Mb = M;
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) Mb = c0 + cg + u * MG < nc ? fmaxf(Mb, mm[u]) : Mb;
        const float r = fast_exp2(M - Mb);
        at *= r;
        lt *= r;
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const bool ok = c0 + cg + u * MG < nc;
            const float w = fast_exp2(mm[u] - Mb);
            lt = ok ? __builtin_fmaf(w, ll[u], lt) : lt;
            at = ok ? __builtin_fmaf(w, aa[u], at) : at;
        }
        M = Mb;
    }
    s_acc[cg][d] = at;
    if (d == 0) {
        s_ml[cg][0] = M;
        s_ml[cg][1] = lt;
    }
    __syncthreads();
    if (t < D) {
        float Mx = s_ml[0][0];
#pragma unroll
        for (int g = 1; g < MG; ++g) Mx = fmaxf(Mx, s_ml[g][0]);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const float w = fast_exp2(s_ml[g][0] - Mx);
            a = __builtin_fmaf(w, s_acc[g][t], a);
            l = __builtin_fmaf(w, s_ml[g][1], l);
        }
        static_cast<T*>(p.out)[((size_t)s * p.Hq + hq) * D + t] = (T)(l > 0.f ? a * (1.0f / l) : 0.f);
    }
}

#include "gqa_mfma.hpp"

// Dynamic LDS that caps workgroups per CU (tuning "wg_per_cu"), from the
// kernel's static LDS (queried once per kernel).
inline unsigned lds_pad_for(const void* kernel, int wg_per_cu) {
    static std::mutex mu;
    static std::unordered_map<const void*, size_t> static_lds;
    size_t st = 0;
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = static_lds.find(kernel);
        if (it == static_lds.end()) {
            hipFuncAttributes a{};
            st = hipFuncGetAttributes(&a, kernel) == hipSuccess ? a.sharedSizeBytes : 0;
            static_lds.emplace(kernel, st);
        } else {
            st = it->second;
        }
    }
    return (unsigned)occupancy_lds(st, wg_per_cu);
}

template <typename K>
unsigned lds_pad(K kernel, int wg_per_cu) {
    return wg_per_cu > 0 ? lds_pad_for(reinterpret_cast<const void*>(kernel), wg_per_cu) : 0u;
}

// Workgroups of `kernel` resident on the whole device at once (block threads,
// `lds` bytes of dynamic LDS): the size of a persistent grid.
inline long long resident_blocks_for(const void* kernel, int block, unsigned lds) {
    static std::mutex mu;
    static std::unordered_map<const void*, std::unordered_map<unsigned, long long>> cache;
    std::lock_guard<std::mutex> lk(mu);
    auto& per = cache[kernel];
    auto it = per.find(lds);
    if (it != per.end()) return it->second;
    int dev = 0, cus = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, lds) != hipSuccess || n <= 0) n = 1;
    return per[lds] = (long long)n * cus;
}

// Grid of a self-planned launch: at most the units it can have, at most one
// workgroup per resident slot.
// Short sequences attended while the kernel plans need a workgroup per (sequence,
// head subgroup): with fewer, the launch plans every sequence.
template <typename K>
dim3 self_grid(K kernel, int block, unsigned lds, dim3 upper, DecodeParams& p) {
    const long long r = resident_blocks_for(reinterpret_cast<const void*>(kernel), block, lds);
    const dim3 g((unsigned)std::max(1LL, std::min((long long)upper.x, r)));
    if (p.sp_lead > 0 && (long long)p.N * p.Hkv * p.nsub > (long long)g.x) p.sp_lead = 0;
    return g;
}

template <typename T, int D, int G, int WPB, int U>
int launch_split_mode(DecodeLaunch L, dim3 grid, hipStream_t st) {
    const dim3 block(WPB * kWave);
    switch (L.mode) {
        case kContiguous:   L.lds_pad = lds_pad(split_kernel<T, D, G, kContiguous, WPB, U>, L.wg_per_cu); hipLaunchKernelGGL((split_kernel<T, D, G, kContiguous, WPB, U>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kPagedUniform: L.lds_pad = lds_pad(split_kernel<T, D, G, kPagedUniform, WPB, U>, L.wg_per_cu); hipLaunchKernelGGL((split_kernel<T, D, G, kPagedUniform, WPB, U>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kPagedPerLane: L.lds_pad = lds_pad(split_kernel<T, D, G, kPagedPerLane, WPB, U>, L.wg_per_cu); hipLaunchKernelGGL((split_kernel<T, D, G, kPagedPerLane, WPB, U>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kPlannedUniform: L.lds_pad = lds_pad(split_kernel<T, D, G, kPlannedUniform, WPB, U>, L.wg_per_cu); hipLaunchKernelGGL((split_kernel<T, D, G, kPlannedUniform, WPB, U>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kPlannedPerLane: L.lds_pad = lds_pad(split_kernel<T, D, G, kPlannedPerLane, WPB, U>, L.wg_per_cu); hipLaunchKernelGGL((split_kernel<T, D, G, kPlannedPerLane, WPB, U>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kSelfPlanned:
            L.lds_pad = lds_pad(split_kernel<T, D, G, kSelfPlanned, WPB, U>, L.wg_per_cu);
            grid = self_grid(split_kernel<T, D, G, kSelfPlanned, WPB, U>, block.x, L.lds_pad, grid, L.p);
            hipLaunchKernelGGL((split_kernel<T, D, G, kSelfPlanned, WPB, U>), grid, block, L.lds_pad, st, L.p.cur_len,
                               L.p.N, L.p);
            break;
        case kSelfContig:
            L.lds_pad = lds_pad(split_kernel<T, D, G, kSelfContig, WPB, U>, L.wg_per_cu);
            grid = self_grid(split_kernel<T, D, G, kSelfContig, WPB, U>, block.x, L.lds_pad, grid, L.p);
            hipLaunchKernelGGL((split_kernel<T, D, G, kSelfContig, WPB, U>), grid, block, L.lds_pad, st, L.p.cur_len,
                               L.p.N, L.p);
            break;
        default: return set_error(KVC_ERR_ARG, "unknown decode mode");
    }
    return KVC_OK;
}

// Wave-loads per double-buffered batch: 4 for one or two query heads per wave
// (2 and 8 selectable for D 64/128), 2 for larger head groups (register budget).
template <typename T, int D, int G, int WPB>
int launch_split_u(const DecodeLaunch& L, dim3 grid, hipStream_t st) {
    if constexpr (G <= 2) {
        if constexpr (D == 64 || D == 128) {
            if (L.batch == 2) return launch_split_mode<T, D, G, WPB, 2>(L, grid, st);
            if (L.batch == 8) return launch_split_mode<T, D, G, WPB, 8>(L, grid, st);
        }
        return launch_split_mode<T, D, G, WPB, 4>(L, grid, st);
    } else {
        return launch_split_mode<T, D, G, WPB, 2>(L, grid, st);
    }
}

template <typename T, int D, int G>
int launch_split_wpb(const DecodeLaunch& L, dim3 grid, hipStream_t st) {
    if (L.wpb == 8) return launch_split_u<T, D, G, 8>(L, grid, st);
    if (L.wpb == 4) return launch_split_u<T, D, G, 4>(L, grid, st);
    return set_error(KVC_ERR_ARG, "waves per block must be 4 or 8");
}

template <typename T, int D>
int launch_split_g(const DecodeLaunch& L, dim3 grid, hipStream_t st) {
    if constexpr (D == 64 || D == 128) {
        switch (L.G) {
            case 1: return launch_split_wpb<T, D, 1>(L, grid, st);
            case 2: return launch_split_wpb<T, D, 2>(L, grid, st);
            case 4: return launch_split_wpb<T, D, 4>(L, grid, st);
            case 7: return launch_split_wpb<T, D, 7>(L, grid, st);
            case 8: return launch_split_wpb<T, D, 8>(L, grid, st);
            default: break;
        }
    } else {
        if (L.G == 1) return launch_split_wpb<T, D, 1>(L, grid, st);
    }
    return set_error(KVC_ERR_UNSUPPORTED, "query heads per unit not instantiated");
}

template <int D, int WPB>
int launch_gqa_mode(DecodeLaunch L, dim3 grid, hipStream_t st) {
    const dim3 block(WPB * kWave);
    switch (L.mode) {
        case kContiguous:     L.lds_pad = lds_pad(gqa_mfma_kernel<D, kContiguous, WPB>, L.wg_per_cu); hipLaunchKernelGGL((gqa_mfma_kernel<D, kContiguous, WPB>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kPagedUniform:   L.lds_pad = lds_pad(gqa_mfma_kernel<D, kPagedUniform, WPB>, L.wg_per_cu); hipLaunchKernelGGL((gqa_mfma_kernel<D, kPagedUniform, WPB>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kPlannedUniform: L.lds_pad = lds_pad(gqa_mfma_kernel<D, kPlannedUniform, WPB>, L.wg_per_cu); hipLaunchKernelGGL((gqa_mfma_kernel<D, kPlannedUniform, WPB>), grid, block, L.lds_pad, st, L.p.work, L.p.work_ints, L.p); break;
        case kCausalTile:     hipLaunchKernelGGL((gqa_mfma_kernel<D, kCausalTile, WPB>), grid, block, 0, st, L.p.work, L.p.work_ints, L.p); break;
        case kSelfPlanned:
            L.lds_pad = lds_pad(gqa_mfma_kernel<D, kSelfPlanned, WPB>, L.wg_per_cu);
            grid = self_grid(gqa_mfma_kernel<D, kSelfPlanned, WPB>, block.x, L.lds_pad, grid, L.p);
            hipLaunchKernelGGL((gqa_mfma_kernel<D, kSelfPlanned, WPB>), grid, block, L.lds_pad, st, L.p.cur_len, L.p.N,
                               L.p);
            break;
        case kSelfContig:
            L.lds_pad = lds_pad(gqa_mfma_kernel<D, kSelfContig, WPB>, L.wg_per_cu);
            grid = self_grid(gqa_mfma_kernel<D, kSelfContig, WPB>, block.x, L.lds_pad, grid, L.p);
            hipLaunchKernelGGL((gqa_mfma_kernel<D, kSelfContig, WPB>), grid, block, L.lds_pad, st, L.p.cur_len, L.p.N,
                               L.p);
            break;
        default: return set_error(KVC_ERR_ARG, "matrix-core decode: unsupported addressing mode");
    }
    return KVC_OK;
}

template <typename T, int D>
int launch_gqa(const DecodeLaunch& L, dim3 grid, hipStream_t st) {
    if constexpr (std::is_same<T, _Float16>::value && (D == 64 || D == 128)) {
        if (L.mode != kCausalTile && (L.p.group > kMfmaMaxHeads || L.p.nsub != 1))
            return set_error(KVC_ERR_ARG, "matrix-core decode: bad group");
        if (L.wpb == 8) return launch_gqa_mode<D, 8>(L, grid, st);
        if (L.wpb == 4) return launch_gqa_mode<D, 4>(L, grid, st);
        return set_error(KVC_ERR_ARG, "waves per block must be 4 or 8");
    } else {
        return set_error(KVC_ERR_UNSUPPORTED, "matrix-core decode needs fp16 and head_dim 64 or 128");
    }
}

}  // namespace

template <typename T, int D>
int launch_decode_d(const DecodeLaunch& L, hipStream_t st) {
    // planned: the work list's units; self-planned: an upper bound of its units
    const bool planned = L.mode == kPlannedUniform || L.mode == kPlannedPerLane || L.mode == kSelfPlanned ||
                         L.mode == kSelfContig;
    const long long units = planned ? (long long)L.units
                          : L.mode == kCausalTile ? (long long)L.p.max_chunks * ((L.p.N + 15) / 16) * L.p.Hq
                                                  : (long long)L.p.max_chunks * L.p.N * L.p.Hkv * L.p.nsub;
    if (units <= 0) return KVC_OK;
    if (units > (long long)INT_MAX) return set_error(KVC_ERR_ARG, "decode grid too large");
    int rc = L.mfma ? launch_gqa<T, D>(L, dim3((unsigned)units), st) : launch_split_g<T, D>(L, dim3((unsigned)units), st);
    if (rc != KVC_OK) return rc;
    rc = hip_check(hipGetLastError(), "decode split launch");
    if (rc != KVC_OK || !L.need_merge || L.p.merge_mode != kMergeKernel) return rc;
    hipLaunchKernelGGL((merge_kernel<T, D>), dim3((unsigned)((long long)L.p.N * L.p.Hq)), dim3(kMergeThreads), 0, st,
                       L.p);
    return hip_check(hipGetLastError(), "decode merge launch");
}

}  // namespace kvc
