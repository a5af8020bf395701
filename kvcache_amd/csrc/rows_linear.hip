// rows_linear.hip -- the linear layers of one decode step (at most 32 rows, one per
// running sequence) as weight-streaming matrix-core kernels, with the operations
// around each layer fused in: the RMSNorm of the input rows as a prologue, and as
// epilogues the q/k/v bias plus rotary embedding, the residual add, SwiGLU, and the
// fp32 logits with per-row argmax candidates.  The reference runs each of these as a
// cuBLAS GEMM followed by one small kernel per elementwise op (qwen_serve.cu:127-175,
// qwen_kernels.cu:24-107, qwen_kernels.cu:229-247).
//
// y[M, N] = A[M, K] W[N, K]^T with M <= 32.  At so few rows a linear layer is a
// stream over its weights (N*K*2 bytes, read once from HBM) that all rows share, so
// the kernel is laid out for that stream:
//  * a column group = two 16-column tiles of W rows (32 outputs, or one SwiGLU
//    gate/up tile pair, or one rotary pair of q/k half-heads); one workgroup of
//    WAVES waves per (column group, K split);
//  * each wave owns a range of 32-wide k steps and issues every load of its range
//    at once (two weight tiles + the A rows, with buffer loads whose descriptors
//    bound the weight tile and the M valid rows, so the tail steps and the rows >= M
//    read as zero with no branches), then runs the 16x16x32 fp16 MFMAs: A lane l =
//    row l%16, B lane l = W row l%16, both with the 8 k values at 8*(l/16) of the
//    step.  That operand layout read straight from memory touches half of 16 cache
//    lines per load instruction, which streams at about half the rate of whole
//    lines when a launch occupies few CUs; so the loads read whole 128-byte lines
//    (a step pair of 8 rows per instruction) and each wave transposes them through
//    a 4 KiB LDS area, a step pair at a time, into the operand layout;
//  * waves are summed through LDS; when K is split across workgroups, each writes
//    its 32x32 partial and the last to arrive (agent-scope counter, reset by it)
//    sums the partials in split order -- deterministic -- and runs the epilogue.
//    Partials are written and read with agent-scope atomic stores and loads, which
//    go to the memory side past the per-XCD L2s; the writer waits for its stores
//    to complete before it counts itself in.  (An agent-scope fence instead writes
//    back / invalidates the whole L2 of the XCD for every workgroup, which costs
//    microseconds per split.)
// Every output rounds where the op-by-op path stores fp16 (GEMM result, then the
// bias/residual/activation), so results equal that path up to fp32 summation order.
#include "internal.hpp"
#include "kvc_abi.h"

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <utility>

namespace kvc {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 32;      // rows per call (two 16-row MFMA tiles)
constexpr int kCols = 32;      // outputs per column group (two 16-column tiles)
constexpr int kOob = 0x7FFFFFF0;  // buffer offset past every descriptor: loads return 0

enum RowsEpi { kEpiStore = 0, kEpiResidual = 1, kEpiQkv = 2, kEpiSwiglu = 3, kEpiLogits = 4 };

struct RowsParams {
    const _Float16* a;       // [M, K] input rows
    const _Float16* w;       // weight rows [*, K]
    const _Float16* norm_w;  // prologue RMSNorm weight [K]
    float eps;
    int M, N, K;             // N: outputs per row (kEpiSwiglu: I; W holds 2I rows, gate then up)
    int splits;              // workgroups per column group along K
    int gpw;                 // column groups per workgroup (splits == 1)
    int groups;              // column groups in all
    float* part;             // [groups * splits][kRows][kCols] split partials
    unsigned* ctr;           // arrival counters (zero between calls): group g's at ctr_word(g, ctr_shift)
    int ctr_shift;           // log2 of the 128-byte lines the counters are spread over
    _Float16* out;           // store: y; residual: x (+=); swiglu: act; qkv: q
    const _Float16* bias;    // qkv: [q_cols + 2 kv_cols]
    _Float16* k_out;
    _Float16* v_out;
    const int* pos;          // qkv: rotary position of each row
    float log2_theta;
    int q_cols, kv_cols, head_dim;
    const int* dev_rows;     // graph-safe launches: the step's row count in device memory (M is then a capacity)
    float* logits;           // logits: fp32 [M, N] or nullptr
    float* best_v;           // logits: [groups][kRows] per-group row maxima
    int* best_i;
};

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Atomics on one 128-byte line serialise (~10 ns each, whatever the address), so the
// groups' counters are spread over lines: group g's at line g mod L, word g / L
// (L = 2^shift lines of 32 words; one line per group up to 512 groups).
__host__ __device__ inline unsigned ctr_word(int g, int shift) {
    return ((unsigned)(g & ((1 << shift) - 1)) << 5) + ((unsigned)g >> shift);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ h8 as_h8(u4 v) { return __builtin_bit_cast(h8, v); }

// First W row of tile t (0/1) of column group g; output column = that + lane column.
template <int EPI>
__device__ __forceinline__ int tile_row(const RowsParams& p, int g, int t) {
    if constexpr (EPI == kEpiQkv) {
        const int gph = p.head_dim / 32;  // column groups per head: (d, d + D/2) rotary pairs
        return (g / gph) * p.head_dim + 16 * (g % gph) + t * (p.head_dim / 2);
    } else if constexpr (EPI == kEpiSwiglu) {
        return t * p.N + 16 * g;
    } else {
        return kCols * g + 16 * t;
    }
}

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// CP: cache-policy bits of a load or store (0, or kCoherent for data that other
// workgroups of the same launch produce or consume).
template <int CP>
__device__ __forceinline__ _Float16 ld_h(__amdgpu_buffer_rsrc_t r, int byte_ofs) {
    return __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, byte_ofs, 0, CP));
}
template <int CP>
__device__ __forceinline__ void st_h(__amdgpu_buffer_rsrc_t r, int byte_ofs, _Float16 v) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, byte_ofs, 0, CP);
}
template <int CP>
__device__ __forceinline__ void st_f(__amdgpu_buffer_rsrc_t r, int byte_ofs, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, byte_ofs, 0, CP);
}

// Epilogue inputs that depend only on the group, the row and the column pair (the
// residual row values; the q|k|v biases and the row's rotary position): loaded with
// the group's weights, so the epilogue needs no further memory round trip.
struct EpiIn {
    _Float16 a0, a1;
    int pos;
};

template <int EPI, int CP>
__device__ __forceinline__ EpiIn epi_load(const RowsParams& p, int M, int g, int m, int c, bool ok) {
    EpiIn e{};
    const int c0 = tile_row<EPI>(p, g, 0) + c, c1 = tile_row<EPI>(p, g, 1) + c;
    if constexpr (EPI == kEpiResidual) {
        const auto r = rsrc(p.out, M * p.N * 2);
        const int mm = ok ? m : kRows;
        e.a0 = ld_h<CP>(r, (mm * p.N + c0) * 2);
        e.a1 = ld_h<CP>(r, (mm * p.N + c1) * 2);
    } else if constexpr (EPI == kEpiQkv) {
        const auto rb = rsrc(p.bias, (p.q_cols + 2 * p.kv_cols) * 2);
        e.a0 = ld_h<0>(rb, c0 * 2);
        e.a1 = ld_h<0>(rb, c1 * 2);
        e.pos = (int)__builtin_amdgcn_raw_buffer_load_b32(rsrc(p.pos, M * 4), m * 4, 0, 0);
    }
    return e;
}

// Epilogue of one (row m, lane column c) pair: v0 from tile 0, v1 from tile 1.  All
// memory traffic goes through buffer descriptors bounded by the M valid rows, so
// rows >= M (and invalid groups, `ok` false) drop their stores without a branch:
// a branch around a store would make the compiler's load counters inexact and
// force a full wait on the weight loads in flight.
template <int EPI, int CP>
__device__ __forceinline__ void epilogue(const RowsParams& p, int M, int g, int m, int c, float v0, float v1, bool ok,
                                         const EpiIn& e, float& bv, int& bi) {
    const int c0 = tile_row<EPI>(p, g, 0) + c, c1 = tile_row<EPI>(p, g, 1) + c;
    const int mm = ok ? m : kRows;  // row index past the descriptors when the group is not valid
    if constexpr (EPI == kEpiStore) {
        const auto r = rsrc(p.out, M * p.N * 2);
        st_h<CP>(r, (mm * p.N + c0) * 2, (_Float16)v0);
        st_h<CP>(r, (mm * p.N + c1) * 2, (_Float16)v1);
    } else if constexpr (EPI == kEpiResidual) {
        const auto r = rsrc(p.out, M * p.N * 2);
        st_h<CP>(r, (mm * p.N + c0) * 2, (_Float16)((float)e.a0 + (float)(_Float16)v0));
        st_h<CP>(r, (mm * p.N + c1) * 2, (_Float16)((float)e.a1 + (float)(_Float16)v1));
    } else if constexpr (EPI == kEpiSwiglu) {
        const float gf = (float)(_Float16)v0, uf = (float)(_Float16)v1;
        st_h<CP>(rsrc(p.out, M * p.N * 2), (mm * p.N + 16 * g + c) * 2, (_Float16)(gf / (1.0f + expf(-gf)) * uf));
    } else if constexpr (EPI == kEpiQkv) {
        // q/k/v projection + bias (qwen_serve.cu:140-147), rotary on q and k (qwen_kernels.cu:64-79).
        // The group's columns lie in one head, so its region (q, k or v) is uniform.
        _Float16 y0 = (_Float16)((float)(_Float16)v0 + (float)e.a0);
        _Float16 y1 = (_Float16)((float)(_Float16)v1 + (float)e.a1);
        const int t = c0 % p.head_dim;  // < D/2: pair (t, t + D/2)
        const float inv = exp2f(-p.log2_theta * (2.0f * (float)t / (float)p.head_dim));
        float sn, co;
        sincosf((float)e.pos * inv, &sn, &co);
        const float x1 = (float)y0, x2 = (float)y1;
        // region of the group from its first column, wave-uniform (every column of the
        // group lies in one head), so the store descriptor is built once in scalars
        const int cg = uniform(tile_row<EPI>(p, g, 0));
        const bool rot = cg < p.q_cols + p.kv_cols;
        if (rot) {
            y0 = (_Float16)(x1 * co - x2 * sn);
            y1 = (_Float16)(x2 * co + x1 * sn);
        }
        const bool isq = cg < p.q_cols;
        _Float16* base = isq ? p.out : rot ? p.k_out : p.v_out;
        const int width = isq ? p.q_cols : p.kv_cols;
        const int col = c0 - (isq ? 0 : rot ? p.q_cols : p.q_cols + p.kv_cols);
        const auto r = rsrc(base, M * width * 2);
        st_h<CP>(r, (mm * width + col) * 2, y0);
        st_h<CP>(r, (mm * width + col + (c1 - c0)) * 2, y1);
    } else {  // kEpiLogits
        const auto r = rsrc(p.logits, p.logits ? M * p.N * 4 : 0);
        st_f<CP>(r, (mm * p.N + c0) * 4, v0);
        st_f<CP>(r, (mm * p.N + c1) * 4, v1);
        if (m < M) {  // (no memory access inside)
            better(bv, bi, v0, c0);
            better(bv, bi, v1, c1);
        }
    }
}

// ---- building blocks of the layer chain's phases (further below) ------------------
// The steps of rows_kernel's unit of work as functions, in the same order and
// arithmetic, so a chain phase computes exactly what the standalone kernel does.
// (rows_kernel keeps its own inline copy of these steps: written through these
// functions, the compiler gave its 4-wave shapes ~45 more VGPRs -- lm_head at 286
// instead of 236, one wave per SIMD instead of two -- so the standalone kernel is left
// as measured; the chain tests compare the two paths bit for bit.)
//
// LDS of a rows workgroup: per wave two 16-row x 128-byte staging blocks (a step
// pair of two A tiles or of the two weight tiles; 16-byte chunk c of row r at chunk
// c ^ (r & 7)), the double-buffered cross-wave reduction, the per-wave sums of
// squares of the prologue norm, and the split arrival flag.
template <int WAVES>
struct RowsLds {
    alignas(16) char stage[WAVES][2][16 * 128];
    float red[2][WAVES][kRows][kCols + 1];
    float ss[WAVES][kRows];
    unsigned last;
};

// Lane geometry of one wave of a rows workgroup over K split `sp` (S k steps per wave).
template <int WAVES, int S>
struct RowsLane {
    static constexpr int NP = (S + 1) / 2;  // step pairs
    int lane, wave, r16, q4, lrow, lch, first, nsteps, kbytes;
    __device__ __forceinline__ RowsLane(const RowsParams& p, int sp) {
        lane = threadIdx.x & 63;
        wave = uniform(threadIdx.x >> 6);
        first = (sp * WAVES + wave) * S;
        nsteps = max(0, min(S, p.K / 32 - first));
        r16 = lane & 15; q4 = lane >> 4;
        lrow = lane >> 3; lch = lane & 7;
        kbytes = p.K * 2;
    }
    // whole-line loads: step pair pp, half h = rows 8h .. 8h+7 of a 16-row tile; lane l
    // reads row 8h + l/8, 16-byte chunk l%8 of the 128 bytes at k step first + 2pp
    // (chunks 0-3 belong to the pair's first step, 4-7 to its second)
    // (the offset goes through an empty asm: with the chain's run-time validity flags
    // the compiler otherwise splits the load into branches with constant-offset copies)
    __device__ __forceinline__ int pair_ofs(int pp, int h, bool ok) const {
        int o = ok && 2 * pp + (lch >> 2) < nsteps ? (8 * h + lrow) * kbytes + (first + 2 * pp) * 64 + lch * 16 : kOob;
        asm("" : "+v"(o));
        return o;
    }
    static __device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }
    // block b (0/1) of the wave's staging area <- the lane's two whole-line chunks
    __device__ __forceinline__ void stage(char (*stg)[16 * 128], int b, u4 lo, u4 hi) const {
        *reinterpret_cast<u4*>(stg[b] + swz(lrow, lch)) = lo;
        *reinterpret_cast<u4*>(stg[b] + swz(8 + lrow, lch)) = hi;
    }
    // operand fragment of step j (0/1) of the pair in block b: row r16, chunk 4j + q4
    __device__ __forceinline__ u4 unstage(char (*stg)[16 * 128], int b, int j) const {
        return *reinterpret_cast<const u4*>(stg[b] + swz(r16, 4 * j + q4));
    }
};

__device__ __forceinline__ void lds_fence() {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

// A rows of this wave's k range (rows >= M and steps past K read as zero), loaded as
// whole lines; CP: cache-policy bits of the loads.
template <int CP, int MT, class Lane>
__device__ __forceinline__ void load_a(const Lane& ln, const RowsParams& p, int M, u4 (&al)[Lane::NP][MT][2]) {
    const auto ar = rsrc(p.a, M * ln.kbytes);
#pragma unroll
    for (int pp = 0; pp < Lane::NP; ++pp)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int o = ln.pair_ofs(pp, h, true);
                al[pp][mt][h] = __builtin_amdgcn_raw_buffer_load_b128(ar, o == kOob ? kOob : mt * 16 * ln.kbytes + o, 0, CP);
            }
}

// The norm weight values of this lane's k positions.
template <int S, class Lane>
__device__ __forceinline__ void load_norm_w(const Lane& ln, const RowsParams& p, u4 (&nw)[S]) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int kofs = (ln.first + i) * 64 + ln.q4 * 16;  // byte offset of the lane's 8 k values
        nw[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(p.norm_w, ln.kbytes), i < ln.nsteps ? kofs : kOob, 0, 0);
    }
}

// Weight tiles of group g: two 16-row tiles, S steps each.  Always issued (a group
// past the end reads zeros without touching memory), so the instruction stream has no
// branches and the compiler's load counters stay exact: the waits for one group leave
// the next group's loads in flight.
template <int EPI, class Lane>
__device__ __forceinline__ void load_w(const Lane& ln, const RowsParams& p, int g, bool valid, u4 (&b)[Lane::NP][2][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const auto br = rsrc(p.w + (size_t)tile_row<EPI>(p, g, t) * p.K, 16 * ln.kbytes);
#pragma unroll
        for (int pp = 0; pp < Lane::NP; ++pp)
#pragma unroll
            for (int h = 0; h < 2; ++h) b[pp][t][h] = __builtin_amdgcn_raw_buffer_load_b128(br, ln.pair_ofs(pp, h, valid), 0, 0);
    }
}

// The epilogue inputs of this thread's items of group g (g0 in place of a group that
// is not valid).
template <int EPI, int CP, int WAVES, int NI>
__device__ __forceinline__ void load_e(const RowsParams& p, int M, int g, int g0, bool valid, EpiIn (&e)[NI]) {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const int item = threadIdx.x + it * WAVES * 64;
        e[it] = epi_load<EPI, CP>(p, M, valid ? g : g0, item / 16, item % 16, valid);
    }
}

// A into the operand layout, a step pair at a time through the wave's staging area,
// then (NORM) the RMSNorm of the rows (qwen_kernels.cu:24-40): sum of squares over
// this wave's k range, summed over the waves in LDS, then A = fp16(x * inv_rms * w).
template <bool NORM, int MT, int S, int WAVES, class Lane>
__device__ __forceinline__ void prologue(const Lane& ln, const RowsParams& p, const u4 (&al)[Lane::NP][MT][2],
                                         const u4 (&nw)[NORM ? S : 1], u4 (&af)[S][MT], RowsLds<WAVES>& L) {
    char(*stg)[16 * 128] = L.stage[ln.wave];
#pragma unroll
    for (int pp = 0; pp < Lane::NP; ++pp) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) ln.stage(stg, mt, al[pp][mt][0], al[pp][mt][1]);
        lds_fence();
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (2 * pp + j < S) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) af[2 * pp + j][mt] = ln.unstage(stg, mt, j);
            }
        lds_fence();
    }
    if constexpr (NORM) {
        float ss[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            ss[mt] = 0.f;
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const h8 x = as_h8(af[i][mt]);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss[mt] = __builtin_fmaf((float)x[e], (float)x[e], ss[mt]);
            }
            ss[mt] += __shfl_xor(ss[mt], 16);
            ss[mt] += __shfl_xor(ss[mt], 32);
            L.ss[ln.wave][mt * 16 + ln.r16] = ss[mt];  // (the four lanes of a row write the same value)
        }
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) tot += L.ss[w][mt * 16 + ln.r16];
            const float inv = 1.0f / sqrtf(tot / (float)p.K + p.eps);
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const h8 x = as_h8(af[i][mt]), wv = as_h8(nw[i]);
                h8 y;
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = (_Float16)((float)x[e] * inv * (float)wv[e]);
                af[i][mt] = __builtin_bit_cast(u4, y);
            }
        }
    }
}

// One column group g = g0 + j: MFMAs over this wave's k range, sum over the waves,
// epilogue.  `ok` false (a group past the end) runs the same code with every store
// dropped.  SPLIT: the K range is split across workgroups (`sp` is this one's part);
// returns false when this workgroup is not the last of the group to arrive (it is
// done).
template <int EPI, int CP, bool SPLIT, int MT, int S, int WAVES, class Lane, int NI>
__device__ __forceinline__ bool run_group(const Lane& ln, const RowsParams& p, int M, int g0, int j, bool ok, int sp,
                                          const u4 (&af)[S][MT], const u4 (&b)[Lane::NP][2][2], const EpiIn (&e)[NI],
                                          RowsLds<WAVES>& L) {
    constexpr int kThreads = WAVES * 64;
    const int g = g0 + j;
    char(*stg)[16 * 128] = L.stage[ln.wave];
    f4 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[mt][t] = f4{0.f, 0.f, 0.f, 0.f};
    // (steps past this wave's range hold zeros: no guard, no branch); the weight tiles
    // go to the operand layout a step pair at a time through the staging area
#pragma unroll
    for (int pp = 0; pp < Lane::NP; ++pp) {
#pragma unroll
        for (int t = 0; t < 2; ++t) ln.stage(stg, t, b[pp][t][0], b[pp][t][1]);
        lds_fence();
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
            if (2 * pp + jj < S) {
                const int i = 2 * pp + jj;
                u4 bw[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) bw[t] = ln.unstage(stg, t, jj);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(af[i][mt]), as_h8(bw[t]), acc[mt][t],
                                                                            0, 0, 0);
            }
        lds_fence();
    }
    // C lane layout: rows 4*(l/16) + r of the 16-row tile, column l%16.
    float(*red)[kRows][kCols + 1] = L.red[j & 1];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[ln.wave][mt * 16 + 4 * ln.q4 + r][t * 16 + ln.r16] = acc[mt][t][r];
    __syncthreads();
    float v[NI][2];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
        const int mr = m < MT * 16 ? m : 0;  // rows of an unused tile: the sum is never stored
        v[it][0] = v[it][1] = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            v[it][0] += red[w][mr][c];
            v[it][1] += red[w][mr][c + 16];
        }
    }
    if constexpr (SPLIT) {  // one group per workgroup
        float* mine = p.part + ((size_t)g * p.splits + sp) * kRows * kCols;
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
            if (m < M) {
                __hip_atomic_store(mine + m * kCols + c, v[it][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(mine + m * kCols + c + 16, v[it][1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        // every store of this workgroup has completed before the arrival is counted
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (threadIdx.x == 0)
            L.last = __hip_atomic_fetch_add(p.ctr + ctr_word(g, p.ctr_shift), 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(p.splits - 1);
        __syncthreads();
        if (!L.last) return false;
        const float* all = p.part + (size_t)g * p.splits * kRows * kCols;
        auto ld = [](const float* a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
            if (m < M) {
                float a0 = 0.f, a1 = 0.f;
                for (int s2 = 0; s2 < p.splits; ++s2) {
                    a0 += ld(all + (size_t)s2 * kRows * kCols + m * kCols + c);
                    a1 += ld(all + (size_t)s2 * kRows * kCols + m * kCols + c + 16);
                }
                v[it][0] = a0;
                v[it][1] = a1;
            }
        }
        if (threadIdx.x == 0)
            __hip_atomic_store(p.ctr + ctr_word(g, p.ctr_shift), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
        float bv = -FLT_MAX;
        int bi = INT_MAX;
        epilogue<EPI, CP>(p, M, ok ? g : g0, m, c, v[it][0], v[it][1], ok, e[it], bv, bi);
        if constexpr (EPI == kEpiLogits) {
            // the 16 column pairs of row m sit in 16 consecutive lanes
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const float ov = __shfl_xor(bv, o);
                const int oi = __shfl_xor(bi, o);
                better(bv, bi, ov, oi);
            }
            // one lane per row stores the group's candidate (rows >= M are never read)
            const int o = ok && c == 0 ? (g * kRows + m) * 4 : kOob;
            st_f<0>(rsrc(p.best_v, p.groups * kRows * 4), o, bv);
            __builtin_amdgcn_raw_buffer_store_b32((unsigned)bi, rsrc(p.best_i, p.groups * kRows * 4), o, 0, 0);
        }
    }
    return true;
}

// MT: 16-row tiles of A in use (1 when M <= 16).  S: k steps per wave.  A
// workgroup runs `gpw` consecutive column groups: the A fragments of each wave's k
// range stay in registers (normalised once), and the weight loads of the next group
// are in flight while the current one is reduced across the waves (LDS, double
// buffered, one barrier per group) and stored.  SPLIT: the K range is split across
// workgroups (one group per workgroup) and the last to arrive finishes the group.
template <int EPI, bool NORM, int MT, int WAVES, int S, bool SPLIT>
__global__ __launch_bounds__(WAVES * 64) void rows_kernel(RowsParams p) {
    // the rows of this call (graph-safe launches read them from device memory);
    // p itself is never copied: a modified copy of the parameters ends up in scratch
    const int M = uniform(p.dev_rows ? min(max(*p.dev_rows, 0), p.M) : p.M);
    constexpr int kThreads = WAVES * 64;
    constexpr int kItems = kRows * 16 / kThreads;  // (row, column pair) items per thread
    __shared__ float s_red[2][WAVES][kRows][kCols + 1];
    __shared__ float s_ss[WAVES][kRows];
    __shared__ unsigned s_last;
    // per wave: two 16-row x 128-byte blocks (a step pair of two A tiles or of the
    // two weight tiles), 16-byte chunk c of row r at chunk c ^ (r & 7)
    __shared__ __attribute__((aligned(16))) char s_stage[WAVES][2][16 * 128];

    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int unit = uniform(blockIdx.x / p.splits), sp = uniform(blockIdx.x % p.splits);
    const int g0 = unit * p.gpw;
    const int ng = min(p.gpw, p.groups - g0);
    const int ksteps = p.K / 32;
    const int first = (sp * WAVES + wave) * S;
    const int nsteps = max(0, min(S, ksteps - first));
    const int r16 = lane & 15, q4 = lane >> 4;
    const int kbytes = p.K * 2;
    // whole-line loads: step pair pp, half h = rows 8h .. 8h+7 of a 16-row tile; lane l
    // reads row 8h + l/8, 16-byte chunk l%8 of the 128 bytes at k step first + 2pp
    // (chunks 0-3 belong to the pair's first step, 4-7 to its second)
    constexpr int NP = (S + 1) / 2;
    const int lrow = lane >> 3, lch = lane & 7;
    auto pair_ofs = [&](int pp, int h, bool ok) {
        return ok && 2 * pp + (lch >> 2) < nsteps ? (8 * h + lrow) * kbytes + (first + 2 * pp) * 64 + lch * 16 : kOob;
    };
    char(*stg)[16 * 128] = s_stage[wave];
    auto swz = [](int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); };
    // block b (0/1) of the wave's area <- the lane's two whole-line chunks
    auto stage = [&](int b, u4 lo, u4 hi) {
        *reinterpret_cast<u4*>(stg[b] + swz(lrow, lch)) = lo;
        *reinterpret_cast<u4*>(stg[b] + swz(8 + lrow, lch)) = hi;
    };
    // operand fragment of step j (0/1) of the pair in block b: row r16, chunk 4j + q4
    auto unstage = [&](int b, int j) { return *reinterpret_cast<const u4*>(stg[b] + swz(r16, 4 * j + q4)); };
    auto lds_fence = []() {
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };

    // A rows of this wave's k range (rows >= M and steps past K read as zero), loaded
    // as whole lines
    const auto ar = rsrc(p.a, M * kbytes);
    u4 al[NP][MT][2];
    u4 nw[NORM ? S : 1];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int o = pair_ofs(pp, h, true);
                al[pp][mt][h] = __builtin_amdgcn_raw_buffer_load_b128(ar, o == kOob ? kOob : mt * 16 * kbytes + o, 0, 0);
            }
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const int kofs = (first + i) * 64 + q4 * 16;  // byte offset of the lane's 8 k values
            nw[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(p.norm_w, kbytes), i < nsteps ? kofs : kOob, 0, 0);
        }
    }
    // Weight tiles of group g: two 16-row tiles, S steps each.  Always issued (a
    // group past the end reads zeros without touching memory), so the instruction
    // stream has no branches and the compiler's load counters stay exact: the waits
    // for one group leave the next group's loads in flight.
    auto load_b = [&](u4 (&b)[NP][2][2], EpiIn (&e)[kItems], int g, bool valid) {
#pragma unroll
        for (int it = 0; it < kItems; ++it) {
            const int item = threadIdx.x + it * kThreads;
            e[it] = epi_load<EPI, 0>(p, M, valid ? g : g0, item / 16, item % 16, valid);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const auto br = rsrc(p.w + (size_t)tile_row<EPI>(p, valid ? g : g0, t) * p.K, 16 * kbytes);
#pragma unroll
            for (int pp = 0; pp < NP; ++pp)
#pragma unroll
                for (int h = 0; h < 2; ++h) b[pp][t][h] = __builtin_amdgcn_raw_buffer_load_b128(br, pair_ofs(pp, h, valid), 0, 0);
        }
    };
    u4 b0[NP][2][2], b1[NP][2][2];
    EpiIn e0[kItems], e1[kItems];
    load_b(b0, e0, g0, true);

    // A into the operand layout, a step pair at a time through the wave's LDS area
    u4 af[S][MT];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) stage(mt, al[pp][mt][0], al[pp][mt][1]);
        lds_fence();
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (2 * pp + j < S) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) af[2 * pp + j][mt] = unstage(mt, j);
            }
        lds_fence();
    }

    if constexpr (NORM) {
        // RMSNorm of the rows (qwen_kernels.cu:24-40): sum of squares over this wave's
        // k range, summed over the waves in LDS, then A = fp16(x * inv_rms * w).
        float ss[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            ss[mt] = 0.f;
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const h8 x = as_h8(af[i][mt]);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss[mt] = __builtin_fmaf((float)x[e], (float)x[e], ss[mt]);
            }
            ss[mt] += __shfl_xor(ss[mt], 16);
            ss[mt] += __shfl_xor(ss[mt], 32);
            s_ss[wave][mt * 16 + r16] = ss[mt];  // (the four lanes of a row write the same value)
        }
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) tot += s_ss[w][mt * 16 + r16];
            const float inv = 1.0f / sqrtf(tot / (float)p.K + p.eps);
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const h8 x = as_h8(af[i][mt]), wv = as_h8(nw[i]);
                h8 y;
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = (_Float16)((float)x[e] * inv * (float)wv[e]);
                af[i][mt] = __builtin_bit_cast(u4, y);
            }
        }
    }

    // One column group: MFMAs over this wave's k range, sum over the waves, epilogue.
    // `ok` false (a group past the end) runs the same code with every store dropped.
    // Returns false when this workgroup is not the last of a split group (it is done).
    auto run_group = [&](const u4 (&b)[NP][2][2], const EpiIn (&e)[kItems], int j, bool ok) -> bool {
        const int g = g0 + j;
        f4 acc[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) acc[mt][t] = f4{0.f, 0.f, 0.f, 0.f};
        // (steps past this wave's range hold zeros: no guard, no branch); the weight
        // tiles go to the operand layout a step pair at a time through the LDS area
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
            for (int t = 0; t < 2; ++t) stage(t, b[pp][t][0], b[pp][t][1]);
            lds_fence();
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                if (2 * pp + jj < S) {
                    const int i = 2 * pp + jj;
                    u4 bw[2];
#pragma unroll
                    for (int t = 0; t < 2; ++t) bw[t] = unstage(t, jj);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int t = 0; t < 2; ++t)
                            acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(af[i][mt]), as_h8(bw[t]),
                                                                                acc[mt][t], 0, 0, 0);
                }
            lds_fence();
        }
        // C lane layout: rows 4*(l/16) + r of the 16-row tile, column l%16.
        float(*red)[kRows][kCols + 1] = s_red[j & 1];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[wave][mt * 16 + 4 * q4 + r][t * 16 + r16] = acc[mt][t][r];
        __syncthreads();
        float v[kItems][2];
#pragma unroll
        for (int it = 0; it < kItems; ++it) {
            const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
            const int mr = m < MT * 16 ? m : 0;  // rows of an unused tile: the sum is never stored
            v[it][0] = v[it][1] = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                v[it][0] += red[w][mr][c];
                v[it][1] += red[w][mr][c + 16];
            }
        }
        if constexpr (SPLIT) {  // one group per workgroup
            float* mine = p.part + ((size_t)g * p.splits + sp) * kRows * kCols;
#pragma unroll
            for (int it = 0; it < kItems; ++it) {
                const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
                if (m < M) {
                    __hip_atomic_store(mine + m * kCols + c, v[it][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(mine + m * kCols + c + 16, v[it][1], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            // every store of this workgroup has completed before the arrival is counted
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __syncthreads();
            if (threadIdx.x == 0)
                s_last = __hip_atomic_fetch_add(p.ctr + ctr_word(g, p.ctr_shift), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         (unsigned)(p.splits - 1);
            __syncthreads();
            if (!s_last) return false;
            const float* all = p.part + (size_t)g * p.splits * kRows * kCols;
            auto ld = [](const float* a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
#pragma unroll
            for (int it = 0; it < kItems; ++it) {
                const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
                if (m < M) {
                    float a0 = 0.f, a1 = 0.f;
                    for (int s2 = 0; s2 < p.splits; ++s2) {
                        a0 += ld(all + (size_t)s2 * kRows * kCols + m * kCols + c);
                        a1 += ld(all + (size_t)s2 * kRows * kCols + m * kCols + c + 16);
                    }
                    v[it][0] = a0;
                    v[it][1] = a1;
                }
            }
            if (threadIdx.x == 0) __hip_atomic_store(p.ctr + ctr_word(g, p.ctr_shift), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int it = 0; it < kItems; ++it) {
            const int item = threadIdx.x + it * kThreads, m = item / 16, c = item % 16;
            float bv = -FLT_MAX;
            int bi = INT_MAX;
            epilogue<EPI, 0>(p, M, ok ? g : g0, m, c, v[it][0], v[it][1], ok, e[it], bv, bi);
            if constexpr (EPI == kEpiLogits) {
                // the 16 column pairs of row m sit in 16 consecutive lanes
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {
                    const float ov = __shfl_xor(bv, o);
                    const int oi = __shfl_xor(bi, o);
                    better(bv, bi, ov, oi);
                }
                // one lane per row stores the group's candidate (rows >= M are never read)
                const int o = ok && c == 0 ? (g * kRows + m) * 4 : kOob;
                st_f<0>(rsrc(p.best_v, p.groups * kRows * 4), o, bv);
                __builtin_amdgcn_raw_buffer_store_b32((unsigned)bi, rsrc(p.best_i, p.groups * kRows * 4), o, 0, 0);
            }
        }
        return true;
    };

    if constexpr (SPLIT) {
        run_group(b0, e0, 0, true);
    } else {
        // two groups per iteration so the buffers swap roles without register copies
        for (int j = 0; j < ng; j += 2) {
            load_b(b1, e1, g0 + j + 1, j + 1 < ng);
            run_group(b0, e0, j, true);
            load_b(b0, e0, g0 + j + 2, j + 2 < ng);
            run_group(b1, e1, j + 1, j + 1 < ng);
        }
    }
}

// ---- the layer chain: the linear layers between two attention launches -----------
// One persistent launch runs, for the rows of a decode step, the previous layer's
// tail -- o_proj + residual, RMSNorm + gate|up + SwiGLU, down_proj + residual (K split)
// -- and the next layer's head -- RMSNorm + q|k|v + bias + rotary -- as phases
// separated by grid barriers, instead of one launch per layer (the reference runs one
// GEMM plus one kernel per elementwise op, qwen_serve.cu:127-175).  Each phase is the
// rows kernel's unit of work, in the same shapes and summation order, so the results
// equal the separate launches bit for bit.  What the chain gains: while a phase
// computes and waits at its barrier, every workgroup already holds its weights for the
// next phase in registers (issued right after the phase's own row loads), so a phase
// after a barrier only waits for its rows, not for a cold weight stream, and the
// launch and start-up of the separate kernels are gone.
//
// Within the launch, rows move between workgroups on different XCDs, whose L2 caches
// are not coherent with each other: every load and store of activations in the chain
// carries the sc1 cache policy (agent-coherent: past the XCD's L2 to the memory side),
// and a workgroup's stores have completed before it counts itself in at a barrier.
//
// Barrier k of a launch: 16 counters on 16 lines (k * 16 + i); workgroup b adds 1 to
// counter b % 16, and wave 0 of every workgroup polls the 16 counters until they sum
// to the grid (one counter line: 3.8 us per barrier on 256 workgroups, 16 lines 1.7 us,
// measured).  Counters reset themselves: workgroup 0 zeroes barriers 1 and 2 when the
// launch starts (nobody reaches them before it has counted itself in at barrier 0)
// and barrier 0 once it has passed barrier 1.  A wait gives up after `spin` polls
// (about a second at the default): it stores kDevErrBarrier into the device error
// word and the workgroup exits, so a grid that cannot be resident at once ends with an
// error, not a hang.  The grid is at most one workgroup per CU (the LDS of a rows
// workgroup is 99 KiB), checked on the host.
constexpr int kCoherent = 16;  // cache-policy bits: sc1
constexpr int kBarLines = 16;
constexpr int kBarriers = 3;
constexpr size_t kChainHdrBytes = 8192;  // barrier counters: 3 x 16 lines of 128 bytes, rounded up
constexpr int kChainWaves = 8, kChainSteps = 4;
enum ChainPhase { kPhO = 0, kPhG = 1, kPhD = 2, kPhQ = 3 };

struct ChainParams {
    RowsParams ph[4];  // o_proj + residual, norm + gate|up + SwiGLU, down_proj + residual, norm + q|k|v + rotary
    int units[4];      // workgroups each phase occupies
    int M;
    unsigned spin;     // polls before a barrier wait gives up
    unsigned* bar;     // kBarriers x kBarLines lines of 32 words
    int* err_word;     // pinned host word of the device (or nullptr)
};

using ChainLane = RowsLane<kChainWaves, kChainSteps>;
typedef u4 ChainW[2][ChainLane::NP][2][2];  // weights of up to two column groups

__device__ __forceinline__ bool chain_barrier(const ChainParams& cp, int k, RowsLds<kChainWaves>& L) {
    // this wave's stores (and loads) have completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x < 64) {
        unsigned* c = cp.bar + (size_t)k * kBarLines * 32;
        const int lane = threadIdx.x;
        if (lane == 0)
            __hip_atomic_fetch_add(c + (blockIdx.x % kBarLines) * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool done = false;
        for (unsigned it = 0; it < cp.spin; ++it) {
            unsigned v = lane < kBarLines ? __hip_atomic_load(c + lane * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                          : 0u;
#pragma unroll
            for (int o = 1; o < kBarLines; o <<= 1) v += __shfl_xor(v, o);
            if (uniform((int)v) >= (int)gridDim.x) {
                done = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) {
            if (!done && cp.err_word)
                __hip_atomic_store(cp.err_word, (int)kDevErrBarrier, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            L.last = done;
        }
    }
    __syncthreads();
    return L.last != 0;
}

// Weight loads of this workgroup's unit of a phase (GPW column groups; none, reading
// nothing, when the workgroup has no unit in it).
template <int EPI, int GPW>
__device__ __forceinline__ void chain_prefetch(const RowsParams& p, int units, ChainW& w) {
    const int blk = blockIdx.x;
    const bool act = blk < units;
    const int unit = uniform(act ? blk / p.splits : 0), sp = uniform(act ? blk % p.splits : 0);
    const ChainLane ln(p, sp);
    const int g0 = unit * p.gpw;
    const int ng = act ? min(p.gpw, p.groups - g0) : 0;
    load_w<EPI>(ln, p, g0, ng > 0, w[0]);
    if constexpr (GPW > 1) load_w<EPI>(ln, p, ng > 1 ? g0 + 1 : g0, ng > 1, w[1]);
}

// One phase of the chain for this workgroup: its unit's rows and epilogue inputs are
// loaded, then `next` issues the next phase's weight loads, then the unit runs on the
// weights `w` loaded before.
template <int EPI, bool NORM, bool SPLIT, int MT, int GPW, class Next>
__device__ __forceinline__ void chain_phase(const RowsParams& p, int M, int units, const ChainW& w,
                                            RowsLds<kChainWaves>& L, Next&& next) {
    constexpr int kItems = kRows * 16 / (kChainWaves * 64);
    const int blk = blockIdx.x;
    if (blk >= units) {  // (uniform)
        next();
        return;
    }
    const int unit = uniform(blk / p.splits), sp = uniform(blk % p.splits);
    const int g0 = unit * p.gpw;
    const int ng = min(p.gpw, p.groups - g0);
    const ChainLane ln(p, sp);
    u4 al[ChainLane::NP][MT][2];
    load_a<kCoherent>(ln, p, M, al);
    u4 nw[NORM ? kChainSteps : 1];
    if constexpr (NORM) load_norm_w(ln, p, nw);
    EpiIn e0[kItems], e1[kItems];
    load_e<EPI, kCoherent, kChainWaves>(p, M, g0, g0, true, e0);
    if constexpr (GPW > 1) load_e<EPI, kCoherent, kChainWaves>(p, M, g0 + 1, g0, ng > 1, e1);
    next();
    __builtin_amdgcn_sched_barrier(0);
    u4 af[kChainSteps][MT];
    prologue<NORM, MT, kChainSteps>(ln, p, al, nw, af, L);
    run_group<EPI, kCoherent, SPLIT>(ln, p, M, g0, 0, true, sp, af, w[0], e0, L);
    if constexpr (GPW > 1) {
        if (ng > 1) run_group<EPI, kCoherent, false>(ln, p, M, g0, 1, true, sp, af, w[1], e1, L);
    }
}

// TAIL: the previous layer's o_proj, gate|up, down_proj; HEAD: the next layer's q|k|v.
template <int MT, bool TAIL, bool HEAD>
__global__ __launch_bounds__(kChainWaves * 64) void chain_kernel(ChainParams cp) {
    __shared__ RowsLds<kChainWaves> L;
    const int M = cp.M;
    ChainW wa, wb;
    if constexpr (TAIL) {
        if (blockIdx.x == 0 && threadIdx.x < 2 * kBarLines)  // barriers 1 and 2
            __hip_atomic_store(cp.bar + (size_t)(kBarLines + threadIdx.x) * 32, 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        chain_prefetch<kEpiResidual, 1>(cp.ph[kPhO], cp.units[kPhO], wa);
        chain_phase<kEpiResidual, false, false, MT, 1>(cp.ph[kPhO], M, cp.units[kPhO], wa, L, [&] {
            chain_prefetch<kEpiSwiglu, 2>(cp.ph[kPhG], cp.units[kPhG], wb);
        });
        if (!chain_barrier(cp, 0, L)) return;
        chain_phase<kEpiSwiglu, true, false, MT, 2>(cp.ph[kPhG], M, cp.units[kPhG], wb, L, [&] {
            chain_prefetch<kEpiResidual, 1>(cp.ph[kPhD], cp.units[kPhD], wa);
        });
        if (!chain_barrier(cp, 1, L)) return;
        if (blockIdx.x == 0 && threadIdx.x < kBarLines)  // barrier 0: every workgroup is past it
            __hip_atomic_store(cp.bar + (size_t)threadIdx.x * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        chain_phase<kEpiResidual, false, true, MT, 1>(cp.ph[kPhD], M, cp.units[kPhD], wa, L, [&] {
            if constexpr (HEAD) chain_prefetch<kEpiQkv, 1>(cp.ph[kPhQ], cp.units[kPhQ], wb);
        });
        if constexpr (HEAD) {
            if (!chain_barrier(cp, 2, L)) return;
        }
    } else {
        chain_prefetch<kEpiQkv, 1>(cp.ph[kPhQ], cp.units[kPhQ], wb);
    }
    if constexpr (HEAD) chain_phase<kEpiQkv, true, false, MT, 1>(cp.ph[kPhQ], M, cp.units[kPhQ], wb, L, [] {});
}

// tokens[m] = the column of the largest candidate over the groups (first index on ties).
constexpr int kArgThreads = 256;
__global__ __launch_bounds__(kArgThreads) void group_argmax_kernel(const float* best_v, const int* best_i, int groups,
                                                                   int* tokens, const int* dev_rows) {
    __shared__ float sv[kArgThreads / 64];
    __shared__ int si[kArgThreads / 64];
    const int m = blockIdx.x;
    if (dev_rows && m >= *dev_rows) return;
    float bv = -FLT_MAX;
    int bi = INT_MAX;
    for (int gi = threadIdx.x; gi < groups; gi += kArgThreads)
        better(bv, bi, best_v[(size_t)gi * kRows + m], best_i[(size_t)gi * kRows + m]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        better(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kArgThreads / 64; ++k) better(bv, bi, sv[k], si[k]);
        tokens[m] = bi == INT_MAX ? 0 : bi;
    }
}

// ---- host side ------------------------------------------------------------------
// Kernel shapes: (waves, k steps per wave) = (4, 7) for K <= 896 with many groups,
// (8, 4) for K <= 1024 with few groups, (8, 4) or (4, 4) with the K range split
// across workgroups for larger K (no prologue norm then).
struct Shape {
    int groups, splits, waves, steps, gpw;
};

int g_tune_splits = -1, g_tune_gpw = -1, g_tune_shape = -1;  // tuning overrides (-1: automatic)

Shape plan_shape(int groups, int K, bool norm) {
    const int ks = K / 32;
    Shape s{groups, 1, 4, 7, 1};
    int shape = g_tune_shape;
    // automatic: 4x7 for very many groups (lm_head, 4748 groups: 49 us vs 51 us at
    // 8x4), 8x4 otherwise (gate|up at I 4864, 304 groups: 7.1 us vs 7.8 us at 4x7),
    // 8x4 with K split past 32 steps (down_proj K 4864 at 32 rows: 5 splits)
    if (shape < 0) shape = ks <= 28 && groups >= 1024 ? 0 : ks <= 32 ? 1 : 3;
    if (shape == 0 && ks > 28) shape = 1;
    if (shape == 1 && ks > 32) shape = 2;
    if (norm && shape >= 2) shape = 1;  // callers reject normalised K above 1024
    if (shape == 0) { s.waves = 4; s.steps = 7; }
    else if (shape == 1) { s.waves = 8; s.steps = 4; }
    else {
        // K split across workgroups: 4 or 8 waves of 4 steps each
        s.waves = shape == 3 ? 8 : 4; s.steps = 4;
        const int per_wg = s.waves * s.steps;
        const int min_splits = (ks + per_wg - 1) / per_wg;
        s.splits = std::max(min_splits, g_tune_splits > 0 ? std::min(g_tune_splits, std::max(1, ks / s.waves)) : 0);
    }
    if (s.splits == 1) {
        // groups per workgroup (measured at 32 rows): up to ~1024 groups, one workgroup
        // per CU (256) running its groups back to back with the next one's loads in
        // flight beats two co-resident single-group workgroups (gate/up, 304 groups:
        // 8.7 vs 12.5 us); for many groups, about two workgroups per CU (lm_head, 4748
        // groups: 10 per workgroup, 67-69 us, vs 78-88 us at 5-8 or 12-16)
        const int per = groups <= 1024 ? 256 : 512;
        s.gpw = g_tune_gpw > 0 ? g_tune_gpw : std::max(1, (groups + per - 1) / per);
    }
    return s;
}

size_t part_bytes(const Shape& s) { return s.splits > 1 ? (size_t)s.groups * s.splits * kRows * kCols * 4 : 0; }

template <int EPI, bool NORM>
int launch_rows(RowsParams p, const Shape& s, hipStream_t st) {
    p.splits = s.splits;
    p.gpw = s.gpw;
    p.groups = s.groups;
    const dim3 grid((s.groups + s.gpw - 1) / s.gpw * s.splits);
    const bool two = p.M > 16;
#define KVC_ROWS_LAUNCH(W, S, SPLIT)                                                                            \
    do {                                                                                                       \
        if (two) hipLaunchKernelGGL((rows_kernel<EPI, NORM, 2, W, S, SPLIT>), grid, dim3(W * 64), 0, st, p);   \
        else hipLaunchKernelGGL((rows_kernel<EPI, NORM, 1, W, S, SPLIT>), grid, dim3(W * 64), 0, st, p);       \
    } while (0)
    if (s.waves == 8 && s.splits > 1) KVC_ROWS_LAUNCH(8, 4, true);
    else if (s.waves == 8) KVC_ROWS_LAUNCH(8, 4, false);
    else if (s.steps == 7) KVC_ROWS_LAUNCH(4, 7, false);
    else if (s.splits > 1) KVC_ROWS_LAUNCH(4, 4, true);
    else KVC_ROWS_LAUNCH(4, 4, false);
#undef KVC_ROWS_LAUNCH
    return hip_check(hipGetLastError(), "rows linear launch");
}

// Workspace layout: [counters: 64 KiB = 512 lines of 32 counters][argmax candidates][split partials]
constexpr size_t kCtrBytes = 64 << 10;

int check_rows(int M, int K, const void* a, const void* w) {
    if (M < 1 || M > kRows) return set_error(KVC_ERR_ARG, "rows linear: 1 <= M <= 32 rows");
    if (K <= 0 || K % 32) return set_error(KVC_ERR_ARG, "rows linear: K must be a positive multiple of 32");
    if ((size_t)K * 2 * kRows > (size_t)INT_MAX) return set_error(KVC_ERR_ARG, "rows linear: K too large");
    if (!a || !w || ((uintptr_t)a & 15) || ((uintptr_t)w & 15))
        return set_error(KVC_ERR_ARG, "rows linear: null or misaligned input");
    return KVC_OK;
}

int check_norm(const void* norm_w, float eps, int K) {
    if (!norm_w) return KVC_OK;
    if (((uintptr_t)norm_w & 15) || !(eps >= 0.f)) return set_error(KVC_ERR_ARG, "rows linear: bad norm weight or eps");
    if (K > 1024) return set_error(KVC_ERR_UNSUPPORTED, "rows linear: normalised K above 1024");
    return KVC_OK;
}

int check_weight_span(size_t rows, int K) {
    // each 16-row weight tile is addressed with 32-bit offsets
    if ((size_t)16 * K * 2 > (size_t)INT_MAX || rows == 0) return set_error(KVC_ERR_ARG, "rows linear: bad weight shape");
    return KVC_OK;
}

// Workgroups of a chain kernel resident on the device at once (at most one per CU).
long long chain_resident(const void* kernel) {
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, long long> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find({dev, kernel});
    if (it != cache.end()) return it->second;
    int cus = 0, n = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kChainWaves * 64, 0) != hipSuccess || n <= 0) n = 0;
    return cache[{dev, kernel}] = (long long)n * cus;
}

size_t chain_ws_bytes(int H, int I) {
    const Shape d = plan_shape(H / kCols, I, false);
    return kChainHdrBytes + kCtrBytes + part_bytes(d);
}

template <int MT>
const void* chain_kernel_for(bool tail, bool head) {
    if (tail && head) return reinterpret_cast<const void*>(&chain_kernel<MT, true, true>);
    if (tail) return reinterpret_cast<const void*>(&chain_kernel<MT, true, false>);
    return reinterpret_cast<const void*>(&chain_kernel<MT, false, true>);
}

template <int MT>
void launch_chain(bool tail, bool head, const ChainParams& cp, int grid, hipStream_t st) {
    if (tail && head) hipLaunchKernelGGL((chain_kernel<MT, true, true>), dim3(grid), dim3(kChainWaves * 64), 0, st, cp);
    else if (tail) hipLaunchKernelGGL((chain_kernel<MT, true, false>), dim3(grid), dim3(kChainWaves * 64), 0, st, cp);
    else hipLaunchKernelGGL((chain_kernel<MT, false, true>), dim3(grid), dim3(kChainWaves * 64), 0, st, cp);
}

bool aligned16(const void* q) { return q && ((uintptr_t)q & 15) == 0; }

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" {

size_t kvc_rows_workspace_size(int N, int K) {
    if (N <= 0 || K <= 0 || N % kCols || K % 32) return 0;
    const Shape s = plan_shape(N / kCols, K, false);
    const size_t cand = (size_t)(N / kCols) * kRows * 8;
    return kCtrBytes + (cand + 255) / 256 * 256 + part_bytes(s);
}

int kvc_rows_linear(void* y, const void* x, const void* w, int M, int N, int K, const void* norm_w, float eps,
                    int residual, const int* dev_rows, void* ws, size_t ws_bytes, kvc_stream_t st) {
    try {
        int rc = check_rows(M, K, x, w);
        if (!rc) rc = check_norm(norm_w, eps, K);
        if (!rc) rc = check_weight_span((size_t)N, K);
        if (rc) return rc;
        if (N <= 0 || N % kCols || !y || ((uintptr_t)y & 15))
            return set_error(KVC_ERR_ARG, "rows linear: N must be a positive multiple of 32, y aligned");
        if (y == x) return set_error(KVC_ERR_ARG, "rows linear: y must not alias x");
        const int groups = N / kCols;
        const Shape s = plan_shape(groups, K, norm_w != nullptr);
        if (s.splits > 1) {
            if ((size_t)groups * 4 > kCtrBytes) return set_error(KVC_ERR_ARG, "rows linear: N too large to split");
            if (!ws || ((uintptr_t)ws & 255) || ws_bytes < kCtrBytes + part_bytes(s))
                return set_error(KVC_ERR_ARG, "rows linear: workspace too small (kvc_rows_workspace_size)");
        }
        RowsParams p{};
        p.a = (const _Float16*)x; p.w = (const _Float16*)w; p.norm_w = (const _Float16*)norm_w; p.eps = eps;
        p.M = M; p.N = N; p.K = K;
        p.out = (_Float16*)y;
        p.dev_rows = dev_rows;
        p.ctr = (unsigned*)ws;
        while ((1 << p.ctr_shift) < std::min(groups, (int)(kCtrBytes / 128))) ++p.ctr_shift;
        p.part = ws ? (float*)((char*)ws + kCtrBytes) : nullptr;
        const hipStream_t hs = (hipStream_t)st;
        if (norm_w) return residual ? launch_rows<kEpiResidual, true>(p, s, hs) : launch_rows<kEpiStore, true>(p, s, hs);
        return residual ? launch_rows<kEpiResidual, false>(p, s, hs) : launch_rows<kEpiStore, false>(p, s, hs);
    } catch (...) {
        return set_error(KVC_ERR_STATE, "unexpected exception");
    }
}

int kvc_rows_qkv(void* q, void* k, void* v, const void* x, const void* norm_w, float eps, const void* w_qkv,
                 const void* b_qkv, const int* pos, int M, int H, int Hq, int Hkv, int D, float theta,
                 const int* dev_rows, kvc_stream_t st) {
    try {
        int rc = check_rows(M, H, x, w_qkv);
        if (!rc) rc = check_norm(norm_w, eps, H);
        if (rc) return rc;
        if (Hq <= 0 || Hkv <= 0 || D <= 0 || D % 32 || !(theta > 1.f))
            return set_error(KVC_ERR_ARG, "rows qkv: heads > 0, D a multiple of 32, theta > 1");
        const int n = (Hq + 2 * Hkv) * D;
        if ((rc = check_weight_span((size_t)n, H))) return rc;
        if (!q || !k || !v || !b_qkv || !pos) return set_error(KVC_ERR_ARG, "rows qkv: null pointer");
        RowsParams p{};
        p.a = (const _Float16*)x; p.w = (const _Float16*)w_qkv; p.norm_w = (const _Float16*)norm_w; p.eps = eps;
        p.M = M; p.N = n; p.K = H;
        p.out = (_Float16*)q; p.k_out = (_Float16*)k; p.v_out = (_Float16*)v;
        p.bias = (const _Float16*)b_qkv; p.pos = pos; p.log2_theta = log2f(theta);
        p.dev_rows = dev_rows;
        p.q_cols = Hq * D; p.kv_cols = Hkv * D; p.head_dim = D;
        const Shape s = plan_shape(n / kCols, H, norm_w != nullptr);
        if (s.splits > 1) return set_error(KVC_ERR_UNSUPPORTED, "rows qkv: K too large for one workgroup");
        return norm_w ? launch_rows<kEpiQkv, true>(p, s, (hipStream_t)st)
                      : launch_rows<kEpiQkv, false>(p, s, (hipStream_t)st);
    } catch (...) {
        return set_error(KVC_ERR_STATE, "unexpected exception");
    }
}

int kvc_rows_swiglu(void* act, const void* x, const void* norm_w, float eps, const void* w_gate_up, int M, int I,
                    int H, const int* dev_rows, kvc_stream_t st) {
    try {
        int rc = check_rows(M, H, x, w_gate_up);
        if (!rc) rc = check_norm(norm_w, eps, H);
        if (!rc) rc = check_weight_span((size_t)2 * I, H);
        if (rc) return rc;
        if (I <= 0 || I % 16 || !act || ((uintptr_t)act & 15))
            return set_error(KVC_ERR_ARG, "rows swiglu: I a positive multiple of 16, act aligned");
        if ((size_t)2 * I * H * 2 > (size_t)UINT32_MAX * 4) return set_error(KVC_ERR_ARG, "rows swiglu: too large");
        RowsParams p{};
        p.a = (const _Float16*)x; p.w = (const _Float16*)w_gate_up; p.norm_w = (const _Float16*)norm_w; p.eps = eps;
        p.M = M; p.N = I; p.K = H;
        p.out = (_Float16*)act;
        p.dev_rows = dev_rows;
        const Shape s = plan_shape(I / 16, H, norm_w != nullptr);
        if (s.splits > 1) return set_error(KVC_ERR_UNSUPPORTED, "rows swiglu: K too large for one workgroup");
        return norm_w ? launch_rows<kEpiSwiglu, true>(p, s, (hipStream_t)st)
                      : launch_rows<kEpiSwiglu, false>(p, s, (hipStream_t)st);
    } catch (...) {
        return set_error(KVC_ERR_STATE, "unexpected exception");
    }
}

int kvc_rows_lm_head(float* logits, int* tokens, const void* x, const void* norm_w, float eps, const void* w, int M,
                     int V, int H, const int* dev_rows, void* ws, size_t ws_bytes, kvc_stream_t st) {
    try {
        int rc = check_rows(M, H, x, w);
        if (!rc) rc = check_norm(norm_w, eps, H);
        if (!rc) rc = check_weight_span((size_t)V, H);
        if (rc) return rc;
        if (V <= 0 || V % kCols) return set_error(KVC_ERR_ARG, "rows lm_head: V must be a positive multiple of 32");
        if (!tokens) return set_error(KVC_ERR_ARG, "rows lm_head: null tokens");
        const int groups = V / kCols;
        const size_t cand = (size_t)groups * kRows * 8;
        if (!ws || ((uintptr_t)ws & 255) || ws_bytes < kCtrBytes + cand)
            return set_error(KVC_ERR_ARG, "rows lm_head: workspace too small (kvc_rows_workspace_size)");
        RowsParams p{};
        p.a = (const _Float16*)x; p.w = (const _Float16*)w; p.norm_w = (const _Float16*)norm_w; p.eps = eps;
        p.M = M; p.N = V; p.K = H;
        p.logits = logits;
        p.dev_rows = dev_rows;
        p.best_v = (float*)((char*)ws + kCtrBytes);
        p.best_i = (int*)((char*)ws + kCtrBytes + (size_t)groups * kRows * 4);
        const Shape one = plan_shape(groups, H, true);  // candidates need whole rows: no K split
        if (one.splits > 1 || H > 1024) return set_error(KVC_ERR_UNSUPPORTED, "rows lm_head: K above 1024");
        rc = norm_w ? launch_rows<kEpiLogits, true>(p, one, (hipStream_t)st)
                    : launch_rows<kEpiLogits, false>(p, one, (hipStream_t)st);
        if (rc) return rc;
        hipLaunchKernelGGL(group_argmax_kernel, dim3(M), dim3(kArgThreads), 0, (hipStream_t)st, p.best_v, p.best_i,
                           groups, tokens, dev_rows);
        return hip_check(hipGetLastError(), "argmax launch");
    } catch (...) {
        return set_error(KVC_ERR_STATE, "unexpected exception");
    }
}

size_t kvc_rows_chain_workspace_size(int H, int I) {
    if (H <= 0 || I <= 0 || H % kCols || I % 32) return 0;
    return chain_ws_bytes(H, I);
}

int kvc_rows_chain(const kvc_layer_chain* c, void* ws, size_t ws_bytes, kvc_stream_t st) {
    try {
        if (!c) return set_error(KVC_ERR_ARG, "rows chain: null description");
        const bool tail = c->w_o != nullptr, head = c->w_qkv != nullptr;
        if (!tail && !head) return set_error(KVC_ERR_ARG, "rows chain: neither w_o nor w_qkv given");
        const int M = c->M, H = c->H, I = c->I, D = c->D, QD = c->Hq * c->D, KD = c->Hkv * c->D;
        int rc = check_rows(M, H, c->x, head ? c->w_qkv : c->w_o);
        if (rc) return rc;
        if (H % kCols || H > 1024) return set_error(KVC_ERR_UNSUPPORTED, "rows chain: H a multiple of 32, at most 1024");
        if (c->Hq <= 0 || c->Hkv <= 0 || D <= 0 || D % 32 || !(c->eps >= 0.f))
            return set_error(KVC_ERR_ARG, "rows chain: heads > 0, D a multiple of 32, eps >= 0");
        if (tail) {
            if (I <= 0 || I % 32) return set_error(KVC_ERR_ARG, "rows chain: I a positive multiple of 32");
            if (!aligned16(c->att) || !aligned16(c->w_o) || !aligned16(c->ln2) || !aligned16(c->w_gate_up) ||
                !aligned16(c->act) || !aligned16(c->w_down))
                return set_error(KVC_ERR_ARG, "rows chain: null or misaligned tail pointer");
            if (c->att == c->x || c->act == c->x) return set_error(KVC_ERR_ARG, "rows chain: x must not alias att or act");
            if ((rc = check_weight_span((size_t)H, QD)) || (rc = check_weight_span((size_t)2 * I, H)) ||
                (rc = check_weight_span((size_t)H, I)))
                return rc;
            if ((size_t)2 * I * H * 2 > (size_t)UINT32_MAX * 4) return set_error(KVC_ERR_ARG, "rows chain: I too large");
        }
        if (head) {
            if (!(c->theta > 1.f)) return set_error(KVC_ERR_ARG, "rows chain: theta > 1");
            if (!aligned16(c->ln1) || !c->b_qkv || !c->pos || !c->q || !c->k || !c->v)
                return set_error(KVC_ERR_ARG, "rows chain: null or misaligned head pointer");
            if ((rc = check_weight_span((size_t)QD + 2 * KD, H))) return rc;
        }
        const hipStream_t hs = (hipStream_t)st;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        const bool capturing = hs && hipStreamIsCapturing(hs, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
        if (tail) {
            if (!ws || ((uintptr_t)ws & 255) || ws_bytes < chain_ws_bytes(H, I))
                return set_error(KVC_ERR_ARG, "rows chain: workspace too small (kvc_rows_chain_workspace_size)");
            // a barrier that gave up left its counters part-way -- the barriers' and the
            // down_proj split's (workgroups past the barrier may have counted in without
            // the one that gave up): clear both, report once
            if (take_device_error_code(kDevErrBarrier)) {
                if (!capturing) (void)hipMemsetAsync(ws, 0, kChainHdrBytes + kCtrBytes, hs);
                return device_error_status(kDevErrBarrier);
            }
        }
        ChainParams cp{};
        cp.M = M;
        cp.spin = (unsigned)tuning().chain_spin;
        cp.bar = (unsigned*)ws;
        cp.err_word = device_error_word(hs, !capturing);
        Shape sh[4] = {};
        bool used[4] = {tail, tail, tail, head};
        if (tail) {
            RowsParams& o = cp.ph[kPhO];
            o.a = (const _Float16*)c->att; o.w = (const _Float16*)c->w_o; o.M = M; o.N = H; o.K = QD;
            o.out = (_Float16*)c->x;
            sh[kPhO] = plan_shape(H / kCols, QD, false);
            RowsParams& g = cp.ph[kPhG];
            g.a = (const _Float16*)c->x; g.w = (const _Float16*)c->w_gate_up; g.norm_w = (const _Float16*)c->ln2;
            g.eps = c->eps; g.M = M; g.N = I; g.K = H; g.out = (_Float16*)c->act;
            sh[kPhG] = plan_shape(I / 16, H, true);
            RowsParams& d = cp.ph[kPhD];
            d.a = (const _Float16*)c->act; d.w = (const _Float16*)c->w_down; d.M = M; d.N = H; d.K = I;
            d.out = (_Float16*)c->x;
            d.ctr = (unsigned*)((char*)ws + kChainHdrBytes);
            while ((1 << d.ctr_shift) < std::min(H / kCols, (int)(kCtrBytes / 128))) ++d.ctr_shift;
            d.part = (float*)((char*)ws + kChainHdrBytes + kCtrBytes);
            sh[kPhD] = plan_shape(H / kCols, I, false);
        }
        if (head) {
            RowsParams& q = cp.ph[kPhQ];
            q.a = (const _Float16*)c->x; q.w = (const _Float16*)c->w_qkv; q.norm_w = (const _Float16*)c->ln1;
            q.eps = c->eps; q.M = M; q.N = QD + 2 * KD; q.K = H;
            q.out = (_Float16*)c->q; q.k_out = (_Float16*)c->k; q.v_out = (_Float16*)c->v;
            q.bias = (const _Float16*)c->b_qkv; q.pos = c->pos; q.log2_theta = log2f(c->theta);
            q.q_cols = QD; q.kv_cols = KD; q.head_dim = D;
            sh[kPhQ] = plan_shape((QD + 2 * KD) / kCols, H, true);
        }
        int grid = 1;
        for (int i = 0; i < 4; ++i) {
            if (!used[i]) continue;
            const Shape& s = sh[i];
            const int max_gpw = i == kPhG ? 2 : 1;
            if (s.waves != kChainWaves || s.steps != kChainSteps || (i != kPhD && s.splits != 1) || s.gpw > max_gpw)
                return set_error(KVC_ERR_UNSUPPORTED, "rows chain: a layer shape outside the chain's kernel shapes");
            cp.ph[i].splits = s.splits;
            cp.ph[i].gpw = s.gpw;
            cp.ph[i].groups = s.groups;
            cp.units[i] = (s.groups + s.gpw - 1) / s.gpw * s.splits;
            grid = std::max(grid, cp.units[i]);
        }
        if (tail && (size_t)(H / kCols) * 4 > kCtrBytes) return set_error(KVC_ERR_ARG, "rows chain: H too large");
        const bool two = M > 16;
        const void* kern = two ? chain_kernel_for<2>(tail, head) : chain_kernel_for<1>(tail, head);
        if (chain_resident(kern) < grid)
            return set_error(KVC_ERR_UNSUPPORTED, "rows chain: the grid (" + std::to_string(grid) +
                                                      " workgroups) cannot be resident at once on this device");
        if (two) launch_chain<2>(tail, head, cp, grid, hs);
        else launch_chain<1>(tail, head, cp, grid, hs);
        return hip_check(hipGetLastError(), "rows chain launch");
    } catch (...) {
        return set_error(KVC_ERR_STATE, "unexpected exception");
    }
}

int kvc_rows_set_tuning(int splits, int groups_per_wg, int shape) {
    if (splits < -1 || splits == 0 || groups_per_wg < -1 || groups_per_wg == 0 || shape < -1 || shape > 3)
        return set_error(KVC_ERR_ARG, "rows tuning: splits, groups_per_wg -1 or >= 1; shape -1..3");
    g_tune_splits = splits;
    g_tune_gpw = groups_per_wg;
    g_tune_shape = shape;
    return KVC_OK;
}

}  // extern "C"
