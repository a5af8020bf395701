// internal.hpp -- declarations shared by the translation units of libkvcache_amd.so.
// Not installed; the public surface is include/kvc_abi.h (C) and include/kvc/*.h (C++).
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <string>

#include "status.hpp"

namespace kvc {

// Checks a HIP return code; on failure records it and returns KVC_ERR_HIP.
int hip_check(hipError_t e, const char* what);

// ---------------------------------------------------------------------------
// Decode launch description (host side).  One "unit" = (sequence s, KV head hk,
// query-head subgroup sub, chunk c); each unit is one workgroup of `wpb` waves.
// ---------------------------------------------------------------------------
// kPlanned*: the grid is a host-built work list (kvc_decode_plan) instead of a
// (chunk, sequence, head) decomposition; otherwise as kPaged*.
// kCausalTile (matrix-core kernel only): prompt attention, a unit is 16 consecutive
// queries of one query head over one chunk of keys of the shared block table.
// kSelfPlanned: lengths in device memory; every workgroup of a persistent grid
// derives the host planner's units itself (selfplan.hpp) and serves ranks
// blockIdx.x, blockIdx.x + gridDim.x, ... (uniform paging, as kPlannedUniform).
// kSelfContig: the same over contiguous caches [N, Hkv, MAXS, D], with chunks cut at
// the paged path's 16-token block granularity, so paged and contiguous batches run
// the same chunks and agree bit for bit.
enum DecodeMode { kContiguous = 0, kPagedUniform = 1, kPagedPerLane = 2, kPlannedUniform = 3, kPlannedPerLane = 4,
                  kCausalTile = 5, kSelfPlanned = 6, kSelfContig = 7 };

struct DecodeParams {
    // scalars first: everything a workgroup needs to locate its unit lies in the
    // first lines of the parameter block, fetched in one round at wave start
    int N, Hq, Hkv, block;
    int group;                // Hq / Hkv
    int nsub;                 // query-head subgroups per KV head (group / G)
    int chunk_tokens;         // >0: fixed chunk size (tokens); else num_splits mode
    int num_splits;           // >0: chunk = ceil(L / num_splits) per sequence
    int max_chunks;           // chunks per sequence covered by the grid
    int fixed_len;            // length used when cur_len == nullptr
    int causal;               // 1: sequence s has length fixed_len + s + 1 (prompt queries, causal mask)
    int cap;                  // the caller's stated maximum length: a longer sequence gets NaN outputs
    int lpb_shift;            // kPagedUniform: log2(wave-loads per block)
    float scale_log2;         // softmax scale * log2(e)
    unsigned epoch;           // per-call tag of the arrival counters
    int merge_mode;           // MergeMode
    int last_chunk_first;     // 1: dispatch the highest chunk index first
    const void* q;
    const void* k;
    const void* v;
    void* out;
    const int* table_all;     // paged only
    const int* tab_off;       // paged only (nullptr: single table starting at table_all)
    const int* cur_len;       // device lengths (nullptr: use fixed_len)
    float* part_acc;          // [N*max_chunks*Hq, D] fp32 partial accumulators
    float* part_ml;           // [N*max_chunks*Hq, 2] (running max in log2 units, running sum)
    unsigned long long* counters;  // arrival counters (fused merge), or nullptr; counter i lives at
                                   // ctr_slot(i, ctr_shift): consecutive counters on separate lines
    int ctr_shift;            // log2 of the 128-byte lines of the counter region
    long long seq_stride;     // contiguous: elements between sequences
    long long head_stride;    // contiguous: elements between KV heads
    const int* work;          // planned units (work_ints ints each, see kvc_decode_plan), or nullptr
    int work_ints;            // planned: ints per unit (8, or 64 with inline block ids)
    int table_len;            // planned: ints in table_all (bounds every block-id read)
    int n_records;            // planned: record groups of the plan (bounds partials and counters)
    const int* dev_counts;    // planned, graph-safe launches: {N, units, records} of this step in device
                              // memory (each clamped to the launch's N / grid / n_records capacities)
    // planned launches with a fused append: the step's new K/V rows [N][Hkv][D] and
    // their positions wpos[N]; the unit whose chunk holds wpos[s] uses the new row in
    // place of the pool's and (first head subgroup) writes it to the pool
    const void* k_new;
    const void* v_new;
    const int* wpos;
    // kSelfPlanned: the planner's shape (plan_shape in abi.hip) and, for prompt
    // queries whose first position lives in device memory, that position (query s
    // then attends to *dev_base + s + 1 keys; causal must be 1)
    int sp_slots, sp_min_chunk, sp_max_chunk, sp_target_cap;
    int sp_nc_max;            // chunks per sequence the merge can combine (0: any)
    int sp_records;           // partial records per (sequence, head) in the workspace
    int sp_pf_blocks;         // blocks of every sequence read ahead while the plan is made (0: none)
    int sp_pf_min_len;        // shortest sequence read ahead
    int sp_pf_xcd;            // 1: each KV head's slice is read ahead on the XCD of its units (self_prefetch)
    // short sequences (VALU self-planned decode): a sequence of at most sp_lead tokens
    // is attended whole, while wave 0 plans, by waves 1.. of workgroup s * hks + h (one
    // per head subgroup h); the plan leaves it out (0: none; a multiple of the block)
    int sp_lead;
    const int* dev_base;
    // where a launch reports a length it could not attend (the rows get NaN as well):
    // a pinned host word per device (device_error_word in abi.hip), or nullptr
    int* err_word;
};

// Codes the kernels store into DecodeParams::err_word.
enum DeviceError {
    kDevErrNone = 0,
    kDevErrCap = 1,      // a sequence longer than the launch's stated cap (explicit-split grid)
    kDevErrBudget = 2,   // a self-planned batch past its planning budget, or a contiguous
                         // length past its cache (MAXS)
    kDevErrBarrier = 3   // a layer-chain launch gave up waiting at a grid barrier
};

// Device-side failure reports (abi.hip): the per-device pinned host word the kernels
// store a DeviceError into (made on first use when may_alloc, never under capture;
// nullptr if none); take_device_error_code clears the word if it holds `code` and says
// whether it did; device_error_status turns a code into a status + message.
int* device_error_word(hipStream_t st, bool may_alloc);
bool take_device_error_code(int code);
int device_error_status(int code);

// Arrival counters.  Atomics that land on one 128-byte line serialise (about 10 ns
// each on MI355X, whether or not they hit the same address), so counters that are
// hot together must not share a line: counter i goes to line i mod L, word i / L
// (L = 2^ctr_shift lines of 16 words).  L is at least min(count, 1024), so up to
// 1024 counters each own a line.
constexpr int kCtrWordsPerLine = 16;
inline int ctr_shift_for(size_t count) {
    size_t lines = count < 1024 ? count : 1024;
    const size_t need = (count + kCtrWordsPerLine - 1) / kCtrWordsPerLine;
    if (need > lines) lines = need;
    int sh = 0;
    while (((size_t)1 << sh) < lines) ++sh;
    return sh;
}
inline size_t ctr_region_bytes(size_t count) {
    return count ? ((size_t)kCtrWordsPerLine * sizeof(unsigned long long)) << ctr_shift_for(count) : 0;
}
__host__ __device__ inline size_t ctr_slot(size_t i, int shift) {
    return ((i & (((size_t)1 << shift) - 1)) * kCtrWordsPerLine) + (i >> shift);
}

// How the chunk partials of a split sequence are combined.
enum MergeMode {
    kMergeKernel = 0,   // separate merge kernel after the split kernel
    kMergeFence = 1,    // last-arriving chunk merges; agent-scope release/acquire fences
    kMergeAtomic = 2    // last-arriving chunk merges; partials written and read with
                        // coherent (agent-scope atomic) accesses, ordered by a wave-local wait
};

struct DecodeLaunch {
    DecodeParams p;
    int dtype;   // KVC_F32 / KVC_F16
    int D;
    int G;       // query heads per unit
    int mode;    // DecodeMode
    int wpb;     // waves per workgroup (4 or 8); one workgroup per unit
    int batch;   // wave-loads per double-buffered batch (2, 4 or 8; used for G <= 2)
    int units;   // planned launches: number of work-list units (the grid); else 0
    bool need_merge;
    bool mfma;   // grouped-query matrix-core kernel (fp16, head_dim 64/128, G = group <= 16)
    unsigned lds_pad;  // dynamic LDS bytes reserved per workgroup (occupancy cap)
    int wg_per_cu;     // >0: at most this many workgroups per CU (through lds_pad)
};

// Launches the split kernel and, when needed and not fused, the merge kernel.
int launch_decode(const DecodeLaunch& L, hipStream_t stream);
// The same for one element type and head_dim; each (T, D) pair is instantiated
// in its own translation unit (decode_<type>_d<D>.hip).
template <typename T, int D>
int launch_decode_d(const DecodeLaunch& L, hipStream_t stream);

// Tuning knobs (kvc_set_tuning).
struct Tuning {
    int fused_merge = -1;       // MergeMode, or -1: automatic (kMergeAtomic when a sequence
                                // has at most 8 chunks, else kMergeKernel)
    int target_units = 4096;    // automatic split: workgroups to aim for (about 16 per CU: the
                                // device-length grid is not ordered by length, so smaller chunks
                                // balance it; N=128 ragged MHA: 45.6 -> 39.3 us)
    int min_chunk_bytes = 32768;// automatic split: least K+V bytes per workgroup
    int waves_per_block = 0;    // 0: automatic (8 for small grids, else 4)
    int batch = 4;              // wave-loads per batch for <= 2 query heads per wave
    int last_chunk_first = 1;   // dispatch order of chunks
    int mfma = -1;              // grouped-query heads on the matrix cores: -1 automatic, 0 off, 1 on
    int wg_per_cu = -1;         // >0: reserve LDS so at most this many decode workgroups share a CU;
                                // 0: no cap; -1: automatic (4 on the planned one/two-head path)
    int split_first = 1;        // planner: chunks of split sequences before whole sequences
    int mfma_min_chunk = 1024;  // planner, grouped-query path: tokens below which a sequence stays in one unit
    int self_plan = 1;          // device-length decode with an automatic split: 1 the kernel plans its own
                                // units (selfplan.hpp), 0 the chunk x sequence x head grid
    int self_grid = 0;          // self-planned launches: 0 automatic (resident workgroups), n: at most n
                                // workgroups (each then serves several ranks, in rounds)
    int self_prefetch_kib = 32768;  // self-planned paged launches: K+V bytes (KiB) read ahead while the
                                    // kernel plans (the first blocks of every sequence; 0: none)
    int self_prefetch_min_len = 256;  // ... of the sequences of at least this many tokens
    int self_prefetch_xcd = 1;  // 1: read each KV head's slice ahead on the XCD whose units use it
                                // (whole-KV-head units and a multiple of 8 KV heads only)
    int self_lead_tokens = 320; // self-planned VALU decode: sequences of at most this many tokens are
                                // attended while the kernel plans the others (0: none)
    int chain_spin = 1 << 20;   // layer chain (kvc_rows_chain): polls before a grid-barrier wait gives
                                // up and reports kDevErrBarrier (about a second at the default)
};
// Dynamic LDS that caps decode workgroups per CU at wg_per_cu (0: none).
size_t occupancy_lds(size_t static_lds, int wg_per_cu);
Tuning& tuning();

// ---------------------------------------------------------------------------
// K/V row writes.
// ---------------------------------------------------------------------------
enum WriteMode { kWriteAppend = 0, kWriteTable = 1, kWriteBatched = 2, kWriteSlots = 3 };
struct WriteParams {
    const void* k;
    const void* v;
    void* kd;
    void* vd;
    const int* table;    // kWriteTable: block table; kWriteBatched: table_all
    const int* tab_off;  // kWriteBatched
    const int* idx;      // kWriteBatched: wpos[rows]; kWriteSlots: slot_map[rows]
    int rows, heads, D, block, start_pos, S, mode;
    const int* dev_start = nullptr;  // kWriteTable: start position read from device memory
};
int launch_write(const WriteParams& p, int dtype, hipStream_t stream);

// Deterministic N(0,1) fill (Box-Muller over a counter hash), fp32 or fp16.
int launch_fill_normal(void* dst, size_t n, int dtype, uint64_t seed, float stddev, hipStream_t stream);

// Read-only pass over the K/V bytes of a planned decode work list (probe.hip).
struct ProbeParams {
    const void* k;
    const void* v;
    const int* table_all;
    int table_len;
    int Hkv, block, nsub;
    int row_bytes;    // D * element size (at most 1024)
    int tpw_shift;    // log2(rows per 1 KiB wave-load)
    int lpb_shift;    // log2(wave-loads per block)
    int* sink;        // [n_units]; written only when a unit's xor equals a fixed value
};
int launch_read_probe(const ProbeParams& p, const int* work, int work_ints, int n_units, hipStream_t stream);
// One launch of an empty kernel of `blocks` one-wave workgroups (probe.hip).
int launch_empty(int blocks, hipStream_t stream);

}  // namespace kvc
