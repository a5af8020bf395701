// abi.hip -- the extern "C" boundary of libkvcache_amd.so (declared in include/kvc_abi.h).
//
// Validates shapes, plans each decode launch (query heads per wave, split size,
// addressing mode, workspace carve-up) and forwards to the kernels in decode.hip
// and append.hip.  Nothing here throws across the boundary; every entry point
// returns a kvc_status and records a message for kvc_last_error().
#include "internal.hpp"
#include "kvc_abi.h"

#include <algorithm>
#include <climits>
#include <atomic>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace kvc {

namespace {
thread_local std::string g_last_error;
}

int set_error(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

Tuning& tuning() {
    static Tuning t;
    return t;
}

size_t occupancy_lds(size_t static_lds, int n) {
    constexpr size_t kLdsPerCu = 160 * 1024;
    if (n <= 0) return 0;
    const size_t per = kLdsPerCu / (size_t)n;
    return per > static_lds + 256 ? per - static_lds - 256 : 0;
}

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return KVC_OK;
    return set_error(KVC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
inline int esize(int dtype) { return dtype == KVC_F16 ? 2 : 4; }
inline bool dtype_ok(int dtype) { return dtype == KVC_F16 || dtype == KVC_F32; }
inline bool d_ok(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Query heads one wave serves from the same K/V registers (a divisor of the GQA group).
inline bool g_instantiated(int D, int G) {
    if (D == 64 || D == 128) return G == 1 || G == 2 || G == 4 || G == 7 || G == 8;
    return G == 1;
}
int choose_g(int group, int D) {
    static const int cands[] = {8, 7, 4, 2, 1};
    for (int c : cands)
        if (group % c == 0 && g_instantiated(D, c)) return c;
    return 1;
}
// Grouped-query decode on the matrix cores (gqa_mfma.hpp): fp16 K/V, head_dim 64
// or 128, groups of 3..16 query heads per KV head (automatic: 4..16), blocks that
// hold whole 16-token subtiles.
constexpr int kMfmaMaxChunkBlocksHost = 1024;
constexpr int kMfmaMaxFusedChunks = 64;
inline bool mfma_path(int group, int D, int dtype, int BLOCK, bool paged) {
    const int t = tuning().mfma;
    if (t == 0 || dtype != KVC_F16 || (D != 64 && D != 128) || group > 16 || group < (t == 1 ? 3 : 4)) return false;
    // paged: 16-token subtiles inside one block, block index and offset by shift and mask
    return !paged || (BLOCK % 16 == 0 && (BLOCK & (BLOCK - 1)) == 0);
}

// Tokens covered by one wave-wide 16-byte load.
inline int tokens_per_wave_load(int D, int dtype) { return 64 / (D * esize(dtype) / 16); }

int auto_split(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int dtype) {
    const int group = Hq / Hkv;
    const int nsub = group / choose_g(group, D);
    const long long per_chunk_units = (long long)N * Hkv * nsub;
    // Enough workgroups to keep all 256 CUs streaming, but never less than
    // min_chunk_bytes of K+V per workgroup so the partial traffic stays small.
    const long long target_units = std::max(1, tuning().target_units);
    long long ch = per_chunk_units > 0 ? ((long long)std::max(cap, 1) * per_chunk_units + target_units - 1) / target_units : 1;
    const long long min_ch = std::max<long long>(16, tuning().min_chunk_bytes / (2LL * D * esize(dtype)));
    ch = std::max(ch, min_ch);
    long long p2 = 1;
    while (p2 < ch) p2 <<= 1;
    ch = p2;
    if (BLOCK > 0 && ch % BLOCK) ch = (ch + BLOCK - 1) / BLOCK * BLOCK;
    if (ch > (1 << 24)) ch = 1 << 24;
    return (int)ch;
}

struct Plan {
    int G = 1, nsub = 1, mode = kContiguous, chunk = 1, max_chunks = 1, wpb = 4, lpb_shift = 0;
    bool mfma = false;
    bool chunk_blocks_ok = true;  // the per-lane path stages at most 4096 block ids per chunk
    size_t acc_bytes = 0, ml_bytes = 0, ws_bytes = 0;
    size_t n_ctr = 0;  // arrival counters
};

inline int ilog2_exact(int x) {  // log2 of a power of two, else -1
    if (x <= 0 || (x & (x - 1))) return -1;
    int r = 0;
    while ((1 << r) < x) ++r;
    return r;
}

// Waves per workgroup: 8 when the grid is small (long contexts, few sequences),
// so each chunk still streams with many loads in flight; 4 otherwise.
int choose_wpb(long long units) {
    const int t = tuning().waves_per_block;
    if (t == 4 || t == 8) return t;
    return units < 1024 ? 8 : 4;
}

// Workspace: [part_acc | part_ml | arrival counters (one per seq x KV head x subgroup, ctr_slot layout)].
void size_workspace(Plan& pl, int N, int Hq, int Hkv, int D) {
    if (pl.max_chunks <= 1) return;
    const size_t recs = (size_t)N * pl.max_chunks * Hq;
    pl.acc_bytes = align_up(recs * D * sizeof(float), kAlign);
    pl.ml_bytes = align_up(recs * 2 * sizeof(float), kAlign);
    pl.n_ctr = (size_t)N * Hkv * pl.nsub;
    pl.ws_bytes = pl.acc_bytes + pl.ml_bytes + align_up(ctr_region_bytes(pl.n_ctr), kAlign);
}

// Matrix-core path: all heads of the group per unit, 8 waves per unit, chunks of
// at least two 32-token tiles per wave, about 512 units over the longest length.
Plan plan_batched_mfma(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int split, bool paged) {
    Plan pl;
    pl.mfma = true;
    pl.G = Hq / Hkv;
    pl.nsub = 1;
    long long ch = split;
    if (ch <= 0) {
        const long long units = (long long)N * Hkv;
        ch = std::max<long long>(512, ((long long)std::max(cap, 1) * units + 511) / 512);
        long long p2 = 1;
        while (p2 < ch) p2 <<= 1;
        ch = p2;
        if (paged) ch = std::min<long long>(ch, (long long)kMfmaMaxChunkBlocksHost * BLOCK);
    }
    if (paged && ch % BLOCK) ch = (ch + BLOCK - 1) / BLOCK * BLOCK;
    pl.chunk = (int)std::min<long long>(ch, 1 << 24);
    pl.max_chunks = std::max(1, (std::max(cap, 0) + pl.chunk - 1) / pl.chunk);
    // 4 waves per unit once there are enough units to fill the CUs, else 8
    const int t = tuning().waves_per_block;
    pl.wpb = (t == 4 || t == 8) ? t : ((long long)pl.max_chunks * N * Hkv >= 256 ? 4 : 8);
    pl.mode = paged ? kPagedUniform : kContiguous;
    pl.chunk_blocks_ok = !paged || pl.chunk / BLOCK <= kMfmaMaxChunkBlocksHost;
    size_workspace(pl, N, Hq, Hkv, D);
    return pl;
}

Plan plan_batched(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int dtype, int split, bool paged) {
    const int group = Hq / Hkv;
    if (mfma_path(group, D, dtype, BLOCK, paged)) {
        Plan pm = plan_batched_mfma(N, Hq, Hkv, D, BLOCK, cap, split, paged);
        if (pm.chunk_blocks_ok) return pm;  // else the chunk is too long for the staged table
    }
    Plan pl;
    pl.G = choose_g(group, D);
    pl.nsub = group / pl.G;
    pl.chunk = split > 0 ? split : auto_split(N, Hq, Hkv, D, paged ? BLOCK : 0, cap, dtype);
    pl.max_chunks = std::max(1, (std::max(cap, 0) + pl.chunk - 1) / pl.chunk);
    const int tpw = tokens_per_wave_load(D, dtype);
    if (paged) {
        // scalar block ids need whole wave-loads per block (a power of two of them)
        // and at most 64 blocks per chunk (one table entry per lane)
        const int lpb = BLOCK % tpw == 0 ? ilog2_exact(BLOCK / tpw) : -1;
        const bool uniform = lpb >= 0 && pl.chunk % BLOCK == 0 && pl.chunk / BLOCK <= 64;
        pl.mode = uniform ? kPagedUniform : kPagedPerLane;
        pl.lpb_shift = uniform ? lpb : 0;
        // per-lane path: block ids of a chunk are staged in LDS (at most 4096)
        const int span = (pl.chunk + BLOCK - 1) / BLOCK + (pl.chunk % BLOCK ? 1 : 0);
        pl.chunk_blocks_ok = uniform || span <= 4096;
    }
    pl.wpb = choose_wpb((long long)pl.max_chunks * N * Hkv * pl.nsub);
    size_workspace(pl, N, Hq, Hkv, D);
    return pl;
}

// Call tag for the fused-merge arrival counters; never 0 (0 is the reset value).
std::atomic<unsigned> g_epoch{0x9e3779b9u};
unsigned next_epoch() {
    unsigned e = g_epoch.fetch_add(1u, std::memory_order_relaxed) + 1u;
    return e ? e : g_epoch.fetch_add(1u, std::memory_order_relaxed) + 1u;
}

// Library-owned grow-only workspace per (device, stream), used when the caller passes
// none.  Launches on one stream run in order, so they can share a buffer; launches on
// different streams get different buffers, so overlapping split-K calls never write
// each other's partials or arrival counters.  Refused under stream capture: a graph
// would keep the address of a buffer that a later growth frees.
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> g_ws;

int default_workspace(size_t bytes, hipStream_t st, void** out) {
    if (st != nullptr) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        int rc = hip_check(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
        if (rc) return rc;
        if (cs != hipStreamCaptureStatusNone)
            return set_error(KVC_ERR_STATE, "a launch under stream capture must pass its own workspace");
    }
    std::lock_guard<std::mutex> lk(g_ws_mu);
    int dev = 0;
    int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    auto& slot = g_ws[{dev, st}];
    if (slot.second < bytes) {
        if (slot.first) {
            // kernels queued on this stream may still read the old buffer
            rc = hip_check(hipStreamSynchronize(st), "hipStreamSynchronize (workspace growth)");
            if (rc) return rc;
            (void)hipFree(slot.first);
            slot = {nullptr, 0};
        }
        const size_t sz = align_up(std::max(bytes, (size_t)1 << 20), (size_t)1 << 20);
        void* p = nullptr;
        if (hipMalloc(&p, sz) != hipSuccess) return set_error(KVC_ERR_NOMEM, "workspace allocation failed");
        slot = {p, sz};
    }
    *out = slot.first;
    return KVC_OK;
}

bool stream_capturing(hipStream_t st) {
    if (st == nullptr) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Device-side failure reports.  A launch that cannot attend a sequence whole (a length
// past its stated cap or its contiguous cache, a batch past the self-planned budget)
// writes NaN rows and stores a DeviceError code into this per-device word of pinned
// host memory (kernels store with system scope; the host reads it without a device
// synchronisation).  The word is made on the first decode call on a device that may
// allocate (never under stream capture, never by the allocation-free entry point,
// which then reports through NaN rows only) and lives until the process ends.
std::mutex g_err_mu;
std::vector<int*> g_err_words;

}  // namespace

int* device_error_word(hipStream_t st, bool may_alloc) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_err_mu);
    if ((int)g_err_words.size() <= dev) g_err_words.resize(dev + 1, nullptr);
    if (!g_err_words[dev] && may_alloc && !stream_capturing(st)) {
        void* w = nullptr;
        if (hipHostMalloc(&w, 64, hipHostMallocDefault) == hipSuccess) {
            __atomic_store_n(static_cast<int*>(w), 0, __ATOMIC_RELAXED);
            g_err_words[dev] = static_cast<int*>(w);
        }
    }
    return g_err_words[dev];
}

// Takes (reads and clears) the current device's reported code; 0 when none.
int take_device_error() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lk(g_err_mu);
    if ((int)g_err_words.size() <= dev || !g_err_words[dev]) return 0;
    return __atomic_exchange_n(g_err_words[dev], 0, __ATOMIC_ACQ_REL);
}

bool take_device_error_code(int code) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    std::lock_guard<std::mutex> lk(g_err_mu);
    if ((int)g_err_words.size() <= dev || !g_err_words[dev]) return false;
    int expected = code;
    return __atomic_compare_exchange_n(g_err_words[dev], &expected, 0, false, __ATOMIC_ACQ_REL, __ATOMIC_ACQUIRE);
}

int device_error_status(int code) {
    switch (code) {
        case kDevErrNone: return KVC_OK;
        case kDevErrCap:
            return set_error(KVC_ERR_ARG, "an earlier decode launch on this device had a sequence longer than its "
                                          "stated cap; its rows were written as NaN");
        case kDevErrBarrier:
            return set_error(KVC_ERR_STATE, "an earlier layer-chain launch on this device gave up waiting at a grid "
                                            "barrier (its workgroups were not all resident); its outputs are "
                                            "incomplete");
        default:
            return set_error(KVC_ERR_ARG, "an earlier decode launch on this device had a batch past its planning "
                                          "budget or a length past its contiguous cache; its rows were written as NaN");
    }
}

// Entry check of the device-length decode calls: an earlier launch's report (as far as
// it has reached the host) fails this call before it launches, and is cleared.
int pending_device_error() { return device_error_status(take_device_error()); }

namespace {

int resolve_workspace(const Plan& pl, void* ws, size_t ws_bytes, DecodeParams& p, hipStream_t st) {
    if (pl.max_chunks <= 1) return KVC_OK;
    if (!ws) {
        int rc = default_workspace(pl.ws_bytes, st, &ws);
        if (rc) return rc;
    } else if (ws_bytes < pl.ws_bytes) {
        return set_error(KVC_ERR_WORKSPACE, "workspace too small: need " + std::to_string(pl.ws_bytes) +
                                                " bytes, got " + std::to_string(ws_bytes));
    } else if (((uintptr_t)ws & 15u) != 0) {
        return set_error(KVC_ERR_ARG, "workspace must be 16-byte aligned");
    }
    p.part_acc = static_cast<float*>(ws);
    p.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + pl.acc_bytes);
    p.counters = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + pl.acc_bytes + pl.ml_bytes);
    p.ctr_shift = ctr_shift_for(pl.n_ctr);
    p.epoch = next_epoch();
    const int t = tuning().fused_merge;
    p.merge_mode = t >= 0 ? t : (pl.max_chunks <= 8 ? kMergeAtomic : kMergeKernel);
    // the matrix-core kernel's fused merge holds one chunk per lane
    if (pl.mfma && pl.max_chunks > kMfmaMaxFusedChunks) p.merge_mode = kMergeKernel;
    return KVC_OK;
}

int check_common(int N, int Hq, int Hkv, int D, int dtype, const void* q, const void* k, const void* v,
                 const void* out) {
    if (!dtype_ok(dtype)) return set_error(KVC_ERR_ARG, "dtype must be KVC_F32 (0) or KVC_F16 (1)");
    if (N < 0 || Hq <= 0 || Hkv <= 0) return set_error(KVC_ERR_ARG, "N must be >= 0 and head counts > 0");
    // the kernels read lengths and table offsets through 32-bit byte-sized descriptors
    if (N >= (1 << 28)) return set_error(KVC_ERR_UNSUPPORTED, "N must be below 2^28 sequences per launch");
    if (Hq % Hkv) return set_error(KVC_ERR_ARG, "Hq must be a multiple of Hkv");
    if (!d_ok(D)) return set_error(KVC_ERR_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256");
    if (N == 0) return KVC_OK;
    if (!q || !k || !v || !out) return set_error(KVC_ERR_ARG, "null q/k/v/out pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return set_error(KVC_ERR_ARG, "q, k, v and out must be 16-byte aligned");
    return KVC_OK;
}

int run_batched(const void* q, const void* k, const void* v, const int* table_all, const int* tab_off,
                const int* cur_len, int fixed_len, void* out, int N, int Hq, int Hkv, int D, int BLOCK,
                long long seq_stride, long long head_stride, int cap, float scale, int dtype, int split,
                bool paged, void* ws, size_t ws_bytes, hipStream_t st, int causal = 0) {
    int rc = check_common(N, Hq, Hkv, D, dtype, q, k, v, out);
    if (rc || N == 0) return rc;
    if (paged && (BLOCK <= 0 || !table_all)) return set_error(KVC_ERR_ARG, "paged decode needs BLOCK > 0 and a block table");
    if (cap < 0) return set_error(KVC_ERR_ARG, "cap must be >= 0");
    if (split < 0) return set_error(KVC_ERR_ARG, "split_tokens must be >= 0");
    if (paged && split > 0 && split % BLOCK) return set_error(KVC_ERR_ARG, "split_tokens must be a multiple of BLOCK");
    if (!std::isfinite(scale)) return set_error(KVC_ERR_ARG, "scale must be finite");
    const Plan pl = plan_batched(N, Hq, Hkv, D, BLOCK, cap, dtype, split, paged);
    if (!pl.chunk_blocks_ok)
        return set_error(KVC_ERR_UNSUPPORTED, "split_tokens spans more than 4096 blocks of this block size");
    DecodeLaunch L{};
    DecodeParams& p = L.p;
    p.q = q; p.k = k; p.v = v; p.out = out;
    p.table_all = table_all; p.tab_off = tab_off; p.cur_len = cur_len; p.fixed_len = fixed_len; p.cap = cap;
    p.causal = causal;
    p.seq_stride = seq_stride; p.head_stride = head_stride;
    p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.block = paged ? BLOCK : 1;
    p.group = Hq / Hkv; p.nsub = pl.nsub;
    p.chunk_tokens = pl.chunk; p.num_splits = 0; p.max_chunks = pl.max_chunks;
    p.scale_log2 = scale * 1.4426950408889634f;
    p.err_word = device_error_word(st, true);
    rc = resolve_workspace(pl, ws, ws_bytes, p, st);
    if (rc) return rc;
    p.lpb_shift = pl.lpb_shift;
    p.last_chunk_first = tuning().last_chunk_first;
    L.dtype = dtype; L.D = D; L.G = pl.G; L.mode = pl.mode; L.wpb = pl.wpb; L.batch = tuning().batch;
    L.need_merge = pl.max_chunks > 1;
    L.mfma = pl.mfma;
    L.wg_per_cu = std::max(tuning().wg_per_cu, 0);
    return launch_decode(L, st);
}

// ---- planned decode (host-known lengths) ----------------------------------
// A unit = {s, hk*nsub + sub, j0, j1, c, nc, record group, counter}.  Every
// sequence is cut into nc near-equal chunks (multiples of BLOCK, at most 64
// blocks so the uniform paged path applies) sized so the whole batch fills the
// resident workgroup slots about once; units are sorted longest first so the
// hardware dispatcher fills the machine greedily (longest-processing-time order).
constexpr int kPlanInts = 8;          // header ints of a unit
constexpr int kPlanIntsInline = 64;   // grouped-query units: header + up to 56 block ids

struct PlanShape {
    int G, nsub, hks, tpw, wpb, min_chunk, max_chunk, slots, entry_ints;
    int target_cap = INT_MAX;  // largest automatic chunk target (tokens)
    bool uniform, mfma;
};

PlanShape plan_shape(int Hq, int Hkv, int D, int BLOCK, int dtype) {
    PlanShape ps{};
    const int group = Hq / Hkv;
    if (mfma_path(group, D, dtype, BLOCK, true)) {
        // all heads of the group per unit; 8 waves; at least two 32-token tiles per
        // wave; about 0.7 units per CU: each unit streams ~1000 tokens, which keeps
        // the chunks of long sequences few (their fused merge is the tail)
        ps.mfma = true;
        ps.uniform = true;
        ps.G = group;
        ps.nsub = 1;
        ps.hks = Hkv;
        ps.tpw = 32;
        const int t = tuning().waves_per_block;
        ps.wpb = (t == 4 || t == 8) ? t : 8;
        // a split costs the chunk tail a store, an arrival and a merge: below ~1024
        // tokens a sequence stays in one unit
        ps.min_chunk = ((tuning().mfma_min_chunk + BLOCK - 1) / BLOCK) * BLOCK;
        ps.max_chunk = kMfmaMaxChunkBlocksHost * BLOCK;
        ps.slots = 176;
        // the unit's first block ids travel in its entry: the kernel reads entry and
        // ids in one round instead of entry, then table
        ps.entry_ints = kPlanIntsInline;
        return ps;
    }
    ps.G = choose_g(group, D);
    ps.nsub = group / ps.G;
    ps.hks = Hkv * ps.nsub;
    ps.tpw = tokens_per_wave_load(D, dtype);
    const int lpb = BLOCK % ps.tpw == 0 ? ilog2_exact(BLOCK / ps.tpw) : -1;
    ps.uniform = lpb >= 0;
    ps.wpb = 4;
    // each wave should stream at least two batches of 4 wave-loads
    ps.min_chunk = ((ps.wpb * ps.tpw * 8 + BLOCK - 1) / BLOCK) * BLOCK;
    ps.max_chunk = ps.uniform ? 64 * BLOCK : std::max(BLOCK, 4095 * BLOCK);
    // units to aim for per CU: ~3.5 for one or two heads per wave (about 1.3 rounds
    // of the 4 units a CU runs at once), ~3 for larger groups
    ps.slots = ps.G <= 2 ? 256 * 7 / 2 : 256 * 3;
    // and, for one or two heads, chunks of at most 640 tokens: on config 2 (N=128 ragged
    // MHA) 640 beat the 752 the slot count gives (33.9 vs 34.5 us), and 576-640 was the
    // best range for log-uniform lengths as well
    if (ps.G <= 2) ps.target_cap = 640;
    // uniform paging: the first 8 block ids ride in the entry (the first batch of
    // every wave of a 4-wave unit touches at most 8 blocks for 16-token blocks)
    ps.entry_ints = ps.uniform ? kPlanInts + 8 : kPlanInts;
    return ps;
}

// Order key of a unit of `len` tokens at chunk target T: with split_first, chunks of
// split sequences above whole sequences; then 64 length buckets, longer above
// shorter.  The kernel's own planner (selfplan.hpp) orders units by the same keys.
inline int plan_key(bool split, long long len, int T, bool split_first) {
    const int b = (int)std::min<long long>(63, len * 42 / T);
    return (split && split_first ? 64 : 0) + b;
}

// Two passes, no sort: the first cuts every sequence into chunks and counts the
// units per order key (all a size query needs), the second writes each unit at its
// key's next slot (a counting sort; within a key in generation order: sequence, then
// chunks 0..nc-2 of every head, then the last chunk of every head).
// The chunk target (tokens) of a plan: `target`, or automatically enough units to
// fill the machine's slots about once, at least min_chunk, a multiple of BLOCK.
int plan_chunk_target(const int* lens, int N, const PlanShape& ps, int BLOCK, int target) {
    long long total = 0;
    for (int i = 0; i < N; ++i) total += std::max(lens[i], 1);
    total *= ps.hks;
    if (target <= 0)
        target = (int)std::min<long long>(std::min<long long>((total + ps.slots - 1) / ps.slots, ps.target_cap),
                                          INT_MAX / 2);
    int T = std::max(target, ps.min_chunk);
    T = (T + BLOCK - 1) / BLOCK * BLOCK;
    return std::min(T, ps.max_chunk);
}

int make_plan(const int* lens, const int* tab_off, const int* table, int table_len, int N, int Hq, int Hkv, int D,
              int BLOCK, int dtype, int target, int* work, int capacity, int* n_units, int* n_records) {
    const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
    if (ps.hks > 0xFFFF) return set_error(KVC_ERR_UNSUPPORTED, "too many KV heads for the plan encoding");
    const int T = plan_chunk_target(lens, N, ps, BLOCK, target);
    const bool split_first = tuning().split_first != 0;
    // pass 1: chunks per sequence, units per key
    thread_local std::vector<int> s_nc, s_chunk;
    s_nc.resize(N);
    s_chunk.resize(N);
    long long count[128] = {0};
    long long units = 0, rec = 0;
    long long off = 0;  // table start of sequence i when tab_off is not given: tables packed in order
    for (int i = 0; i < N; ++i) {
        const int L = std::max(lens[i], 0);
        const long long t0 = tab_off ? tab_off[i] : off;
        off += (L + BLOCK - 1) / BLOCK;
        if (t0 > INT_MAX - (L + BLOCK - 1) / BLOCK) return set_error(KVC_ERR_ARG, "block tables too long");
        int nc = 1, chunk = std::max(L, 1);
        if (L > ps.max_chunk || L > T + T / 2) {
            long long n = std::max(2LL, ((long long)L + T / 2) / T);  // nearest whole number of chunks
            n = std::max(n, ((long long)L + ps.max_chunk - 1) / ps.max_chunk);
            if (ps.mfma) n = std::min<long long>(n, kMfmaMaxFusedChunks);  // the fused merge holds 64 chunks
            chunk = (int)(((long long)L + n - 1) / n);
            chunk = (chunk + BLOCK - 1) / BLOCK * BLOCK;  // block-aligned chunk starts
            nc = (int)(((long long)L + chunk - 1) / chunk);
        }
        if (nc > 0x7FFF) return set_error(KVC_ERR_UNSUPPORTED, "too many chunks per sequence for the plan encoding");
        if (ps.mfma && (nc > kMfmaMaxFusedChunks || (chunk + BLOCK - 1) / BLOCK + 1 > kMfmaMaxChunkBlocksHost))
            return set_error(KVC_ERR_UNSUPPORTED, "sequence too long for the grouped-query planned path");
        s_nc[i] = nc;
        s_chunk[i] = chunk;
        if (nc > 1) {
            count[plan_key(true, chunk, T, split_first)] += (long long)ps.hks * (nc - 1);
            count[plan_key(true, L - (long long)(nc - 1) * chunk, T, split_first)] += ps.hks;
            rec += (long long)nc * ps.hks;
        } else {
            count[plan_key(false, L, T, split_first)] += ps.hks;
        }
        units += (long long)ps.hks * nc;
    }
    if (units > INT_MAX / 2 || rec > INT_MAX / 2) return set_error(KVC_ERR_UNSUPPORTED, "plan too large");
    *n_units = (int)units;
    *n_records = (int)rec;
    if (!work) return KVC_OK;  // size query
    if (capacity < units)
        return set_error(KVC_ERR_WORKSPACE, "plan capacity " + std::to_string(capacity) + " < " +
                                                std::to_string(units) + " units");
    // pass 2: each unit at its key's next slot, keys in descending order
    long long next[128];
    long long acc = 0;
    for (int k = 127; k >= 0; --k) {
        next[k] = acc;
        acc += count[k];
    }
    const int inline_max = ps.entry_ints - kPlanInts;
    auto put = [&](int key, int s, int h, int c, int j0, int j1, int nc, int r, int k, int tab) {
        int* w = work + next[key]++ * (size_t)ps.entry_ints;
        int n_inl = 0;
        if (inline_max > 0) {
            const int nblk = j1 > j0 ? (j1 - 1) / BLOCK - j0 / BLOCK + 1 : 0;
            if (table && tab >= 0 && (long long)tab + std::min(nblk, inline_max) <= table_len)
                n_inl = std::min(nblk, inline_max);
            for (int b = 0; b < n_inl; ++b) w[kPlanInts + b] = table[tab + b];
            for (int b = n_inl; b < inline_max; ++b) w[kPlanInts + b] = 0;
        }
        w[0] = s; w[1] = h | (c << 16); w[2] = j0; w[3] = j1;
        w[4] = nc | (n_inl << 16); w[5] = r; w[6] = k; w[7] = tab;
    };
    int r0 = 0, k0 = 0;
    off = 0;
    for (int i = 0; i < N; ++i) {
        const int L = std::max(lens[i], 0), nc = s_nc[i], chunk = s_chunk[i];
        const int t0 = tab_off ? tab_off[i] : (int)off;
        off += (L + BLOCK - 1) / BLOCK;
        if (nc > 1) {
            const int ka = plan_key(true, chunk, T, split_first);
            const int kb = plan_key(true, L - (long long)(nc - 1) * chunk, T, split_first);
            for (int h = 0; h < ps.hks; ++h)
                for (int c = 0; c < nc - 1; ++c)
                    put(ka, i, h, c, c * chunk, c * chunk + chunk, nc, r0 + h * nc, k0 + h, t0 + c * chunk / BLOCK);
            const int jl = (nc - 1) * chunk;
            for (int h = 0; h < ps.hks; ++h)
                put(kb, i, h, nc - 1, jl, L, nc, r0 + h * nc, k0 + h, t0 + jl / BLOCK);
            r0 += nc * ps.hks;
            k0 += ps.hks;
        } else {
            const int kb = plan_key(false, L, T, split_first);
            for (int h = 0; h < ps.hks; ++h) put(kb, i, h, 0, 0, L, 1, -1, -1, t0);
        }
    }
    return KVC_OK;
}

size_t planned_workspace(int Hq, int Hkv, int D, int BLOCK, int dtype, int n_records) {
    if (n_records <= 0) return 0;
    Plan pl;
    pl.G = plan_shape(Hq, Hkv, D, BLOCK, dtype).G;
    const size_t recs = (size_t)n_records * pl.G;
    pl.acc_bytes = align_up(recs * D * sizeof(float), kAlign);
    pl.ml_bytes = align_up(recs * 2 * sizeof(float), kAlign);
    return pl.acc_bytes + pl.ml_bytes + align_up(ctr_region_bytes((size_t)n_records), kAlign);
}

template <class F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        return set_error(KVC_ERR_ARG, std::string("internal error: ") + e.what());
    } catch (...) {
        return set_error(KVC_ERR_ARG, "internal error");
    }
}

inline hipStream_t S(kvc_stream_t s) { return static_cast<hipStream_t>(s); }

// ---- prompt attention on the matrix cores: 16 queries of one head per unit ----
bool causal_tile_path(int Nq, int Hq, int Hkv, int D, int BLOCK, int dtype) {
    if (tuning().mfma == 0 || dtype != KVC_F16 || (D != 64 && D != 128) || BLOCK <= 0 || BLOCK % 16 ||
        (BLOCK & (BLOCK - 1)))
        return false;
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv) return false;
    return (long long)Nq * Hq * D * 2 < (1LL << 31);  // the q descriptor spans all queries
}

// Key chunks: enough units (query tiles x heads x chunks) to fill the CUs about
// twice, chunks of at least 512 tokens and at most 1024 blocks.
Plan plan_causal_tile(int base, int Nq, int Hq, int Hkv, int D, int BLOCK) {
    Plan pl;
    pl.mfma = true;
    pl.G = Hq / Hkv;
    pl.nsub = 1;
    pl.mode = kCausalTile;
    const long long lmax = std::max(1LL, (long long)base + Nq);
    const long long tiles = (long long)((Nq + 15) / 16) * Hq;
    const long long want = std::max(1LL, (512 + tiles - 1) / std::max(tiles, 1LL));
    long long ch = std::max<long long>(512, (lmax + want - 1) / want);
    long long p2 = 1;
    while (p2 < ch) p2 <<= 1;
    ch = std::min<long long>(p2, (long long)kMfmaMaxChunkBlocksHost * BLOCK);
    ch = (ch + BLOCK - 1) / BLOCK * BLOCK;
    pl.chunk = (int)ch;
    pl.max_chunks = (int)((lmax + ch - 1) / ch);
    const int t = tuning().waves_per_block;
    pl.wpb = (t == 4 || t == 8) ? t : (tiles * pl.max_chunks >= 512 ? 4 : 8);
    size_workspace(pl, Nq, Hq, Hkv, D);
    return pl;
}

int run_causal_tile(const void* q, void* out, const void* k, const void* v, const int* table, int base, int Nq, int Hq,
                    int Hkv, int D, int BLOCK, float scale, void* ws, size_t ws_bytes, hipStream_t st) {
    int rc = check_common(Nq, Hq, Hkv, D, KVC_F16, q, k, v, out);
    if (rc || Nq == 0) return rc;
    if (!table) return set_error(KVC_ERR_ARG, "null block table");
    if (!std::isfinite(scale)) return set_error(KVC_ERR_ARG, "scale must be finite");
    const Plan pl = plan_causal_tile(base, Nq, Hq, Hkv, D, BLOCK);
    DecodeLaunch L{};
    DecodeParams& p = L.p;
    p.q = q; p.k = k; p.v = v; p.out = out;
    p.table_all = table;
    p.N = Nq; p.Hq = Hq; p.Hkv = Hkv; p.block = BLOCK;
    p.group = Hq / Hkv; p.nsub = 1;
    p.chunk_tokens = pl.chunk; p.max_chunks = pl.max_chunks;
    p.fixed_len = base; p.cap = base + Nq; p.causal = 1;
    p.scale_log2 = scale * 1.4426950408889634f;
    rc = resolve_workspace(pl, ws, ws_bytes, p, st);
    if (rc) return rc;
    p.merge_mode = kMergeKernel;
    L.dtype = KVC_F16; L.D = D; L.G = pl.G; L.mode = kCausalTile; L.wpb = pl.wpb; L.batch = tuning().batch;
    L.need_merge = pl.max_chunks > 1;
    L.mfma = true;
    return launch_decode(L, st);
}

int run_planned(const void* q, const void* k_new, const void* v_new, const int* wpos, const void* k_pool,
                const void* v_pool, const int* table_all, int table_len, void* out, int N, int Hq, int Hkv, int D,
                int BLOCK, float scale, int dtype, const int* work, int n_units, int n_records, void* ws,
                size_t ws_bytes, hipStream_t st, const int* dev_counts = nullptr) {
    {
        int rc = check_common(N, Hq, Hkv, D, dtype, q, k_pool, v_pool, out);
        if (rc || N == 0 || n_units == 0) return rc;
        if (BLOCK <= 0 || !table_all || table_len <= 0 || !work || n_units < 0 || n_records < 0)
            return set_error(KVC_ERR_ARG, "planned decode needs BLOCK > 0, a block table and a work list");
        if (!std::isfinite(scale)) return set_error(KVC_ERR_ARG, "scale must be finite");
        const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
        DecodeLaunch L{};
        DecodeParams& p = L.p;
        p.q = q; p.k = k_pool; p.v = v_pool; p.out = out;
        p.table_all = table_all; p.table_len = table_len;
        p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.block = BLOCK;
        p.group = Hq / Hkv; p.nsub = ps.nsub;
        p.chunk_tokens = 1; p.max_chunks = 1; p.cap = INT_MAX;
        p.scale_log2 = scale * 1.4426950408889634f;
        p.work = work;
        p.work_ints = ps.entry_ints;
        p.n_records = n_records;
        p.lpb_shift = ps.uniform ? ilog2_exact(BLOCK / ps.tpw) : 0;
        if (n_records > 0) {
            const size_t need = planned_workspace(Hq, Hkv, D, BLOCK, dtype, n_records);
            if (!ws) {
                rc = default_workspace(need, st, &ws);
                if (rc) return rc;
            } else if (ws_bytes < need) {
                return set_error(KVC_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                                        " bytes, got " + std::to_string(ws_bytes));
            } else if (((uintptr_t)ws & 15u) != 0) {
                return set_error(KVC_ERR_ARG, "workspace must be 16-byte aligned");
            }
            const size_t recs = (size_t)n_records * ps.G;
            const size_t acc = align_up(recs * D * sizeof(float), kAlign), ml = align_up(recs * 2 * sizeof(float), kAlign);
            p.part_acc = static_cast<float*>(ws);
            p.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + acc);
            p.counters = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + acc + ml);
            p.ctr_shift = ctr_shift_for((size_t)n_records);
        }
        p.epoch = next_epoch();
        p.merge_mode = tuning().fused_merge == kMergeFence ? kMergeFence : kMergeAtomic;  // planned: always fused
        // the grid is the unit list; chunk_range is not used on this path
        L.dtype = dtype; L.D = D; L.G = ps.G; L.mode = ps.uniform ? kPlannedUniform : kPlannedPerLane;
        L.mfma = ps.mfma;
        // a cap on co-resident units lets the longest-first order work as a queue
        L.wg_per_cu = tuning().wg_per_cu >= 0 ? tuning().wg_per_cu : (!ps.mfma && ps.G <= 2 ? 6 : 0);
        L.wpb = tuning().waves_per_block ? tuning().waves_per_block : ps.wpb;
        L.batch = tuning().batch;
        L.need_merge = false;
        L.units = n_units;
        p.k_new = k_new; p.v_new = v_new; p.wpos = wpos;
        p.dev_counts = dev_counts;  // (n_units, N, n_records are then capacities)
        return launch_decode(L, st);
    }
}

// ---- self-planned decode (device lengths, no host plan) -------------------
// Every workgroup of a persistent grid derives the host planner's units from the
// lengths in device memory (selfplan.hpp).  Available when the planner's shape pages
// uniformly and the batch's lengths fit in LDS.
constexpr int kSelfMaxNValuHost = 1024, kSelfMaxNMfmaHost = 512, kSelfRecordsPerHeadHost = 64;

// Partial records per (sequence, head) of a self-planned launch: 64, or enough for
// a mean length of `bound` tokens (the caller's cap) at the largest chunk, so a
// batch within its stated bound never overflows the record budget.
int self_plan_budget(const PlanShape& ps, long long bound) {
    long long r = kSelfRecordsPerHeadHost;
    if (bound > 0) r = std::max(r, (bound + ps.max_chunk - 1) / ps.max_chunk + 1);
    return (int)std::min<long long>(r, 1 << 24);
}

bool self_plan_ok(int N, int Hq, int Hkv, int D, int BLOCK, int dtype, long long bound = 0) {
    if (N <= 0 || BLOCK <= 0 || (BLOCK & (BLOCK - 1)) || Hq <= 0 || Hkv <= 0 || Hq % Hkv || !d_ok(D) ||
        !dtype_ok(dtype))
        return false;
    const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
    if (!ps.uniform || ps.hks > 0xFFFF) return false;
    if (N > (ps.mfma ? kSelfMaxNMfmaHost : kSelfMaxNValuHost)) return false;
    // the units' record numbering stays inside int
    return (long long)self_plan_budget(ps, bound) * ps.hks * N + 1 < (1LL << 30);
}

// Records of a self-planned launch (the budget per sequence and head).
long long self_plan_records(int N, int Hq, int Hkv, int D, int BLOCK, int dtype, long long bound = 0) {
    const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
    return (long long)self_plan_budget(ps, bound) * ps.hks * N;
}

size_t self_plan_workspace(int N, int Hq, int Hkv, int D, int BLOCK, int dtype, long long bound = 0) {
    return planned_workspace(Hq, Hkv, D, BLOCK, dtype, (int)self_plan_records(N, Hq, Hkv, D, BLOCK, dtype, bound));
}

// Sequences per launch when a batch has more than one self-planned launch plans (it
// then runs as consecutive groups); 0 when the shape has no self-planned path at all.
int self_plan_group(int N, int Hq, int Hkv, int D, int BLOCK, int dtype, long long bound = 0) {
    if (N <= 0 || !self_plan_ok(1, Hq, Hkv, D, BLOCK, dtype, bound)) return 0;
    const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
    int g = std::min(N, ps.mfma ? kSelfMaxNMfmaHost : kSelfMaxNValuHost);
    while (g > 1 && !self_plan_ok(g, Hq, Hkv, D, BLOCK, dtype, bound)) g /= 2;
    return g;
}

// Contiguous caches are planned with chunks cut at this granularity, the paged
// path's usual block, so a paged batch with 16-token blocks and the same batch in
// contiguous caches run the same chunks (bit-identical outputs).
constexpr int kSelfContigBlock = 16;

// cur_len: device lengths; or (cur_len == NULL) causal prompt queries, query s
// attending to *dev_base + s + 1 keys of the one table at table_all.  cap > 0 only
// sizes the grid (the units of lengths up to cap); 0: unknown.  contig: caches
// [N, Hkv, MAXS, D] addressed by seq_stride / head_stride (BLOCK ignored).
int run_self_planned(const void* q, const void* k, const void* v, const int* table_all, const int* tab_off,
                     const int* cur_len, const int* dev_base, void* out, int N, int Hq, int Hkv, int D, int BLOCK,
                     int cap, float scale, int dtype, void* ws, size_t ws_bytes, hipStream_t st, bool contig = false,
                     long long seq_stride = 0, long long head_stride = 0, bool no_alloc = false) {
    int rc = check_common(N, Hq, Hkv, D, dtype, q, k, v, out);
    if (rc || N == 0) return rc;
    if (contig) BLOCK = kSelfContigBlock;
    if (!contig && !table_all) return set_error(KVC_ERR_ARG, "null block table");
    if (!std::isfinite(scale)) return set_error(KVC_ERR_ARG, "scale must be finite");
    const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
    const long long bound = cap;  // the record budget follows the caller's stated bound
    const long long recs = self_plan_records(N, Hq, Hkv, D, BLOCK, dtype, bound);
    const size_t need = self_plan_workspace(N, Hq, Hkv, D, BLOCK, dtype, bound);
    if (!ws) {
        rc = default_workspace(need, st, &ws);
        if (rc) return rc;
    } else if (ws_bytes < need) {
        return set_error(KVC_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) + " bytes, got " +
                                                std::to_string(ws_bytes));
    } else if (((uintptr_t)ws & 15u) != 0) {
        return set_error(KVC_ERR_ARG, "workspace must be 16-byte aligned");
    }
    DecodeLaunch L{};
    DecodeParams& p = L.p;
    p.q = q; p.k = k; p.v = v; p.out = out;
    p.table_all = contig ? nullptr : table_all; p.tab_off = contig ? nullptr : tab_off;
    p.cur_len = cur_len; p.dev_base = dev_base;
    p.causal = cur_len ? 0 : 1;
    p.seq_stride = seq_stride; p.head_stride = head_stride;
    p.table_len = 0x1FFFFFFF;  // the reference's signature carries no table length
    p.N = N; p.Hq = Hq; p.Hkv = Hkv; p.block = BLOCK;
    p.group = Hq / Hkv; p.nsub = ps.nsub;
    p.chunk_tokens = 1; p.max_chunks = 1;
    p.cap = contig ? (int)(head_stride / D) : INT_MAX;  // contiguous: a longer sequence would leave its cache
    p.scale_log2 = scale * 1.4426950408889634f;
    p.work = nullptr; p.work_ints = kPlanInts;
    p.n_records = (int)recs;
    p.lpb_shift = ilog2_exact(BLOCK / ps.tpw);  // uniform paging (self_plan_ok)
    p.sp_slots = ps.slots; p.sp_min_chunk = ps.min_chunk; p.sp_max_chunk = ps.max_chunk;
    p.sp_target_cap = ps.target_cap; p.sp_nc_max = ps.mfma ? kMfmaMaxFusedChunks : 0;
    p.sp_records = self_plan_budget(ps, bound);
    if (!contig && cur_len && tab_off && tuning().self_prefetch_kib > 0) {
        // the first blocks of every sequence, about self_prefetch_kib KiB of K and V
        const long long kvb = 2LL * Hkv * BLOCK * D * (dtype == KVC_F16 ? 2 : 4);
        if (kvb <= (4LL << 20))  // a block of both pools (every KV head) addressed with 32-bit offsets
            p.sp_pf_blocks = (int)std::min<long long>(((long long)tuning().self_prefetch_kib << 10) / ((long long)N * kvb), 4096);
        p.sp_pf_min_len = std::max(tuning().self_prefetch_min_len, 1);
        p.sp_pf_xcd = tuning().self_prefetch_xcd != 0 && ps.nsub == 1 && Hkv % 8 == 0;
    }
    // short sequences attended while the kernel plans the others (VALU decodes whose
    // table offsets, if paged, are given; at most the largest chunk: a chunk's block
    // ids are one per lane)
    if (!ps.mfma && cur_len && (contig || tab_off) && tuning().self_lead_tokens > 0)
        p.sp_lead = std::min(tuning().self_lead_tokens, ps.max_chunk);
    const size_t rall = (size_t)recs;
    const size_t acc = align_up(rall * ps.G * D * sizeof(float), kAlign), ml = align_up(rall * ps.G * 2 * sizeof(float), kAlign);
    p.part_acc = static_cast<float*>(ws);
    p.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + acc);
    p.counters = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + acc + ml);
    p.ctr_shift = ctr_shift_for(rall);
    p.epoch = next_epoch();
    p.merge_mode = kMergeAtomic;
    p.err_word = device_error_word(st, !no_alloc);
    L.dtype = dtype; L.D = D; L.G = ps.G; L.mode = contig ? kSelfContig : kSelfPlanned; L.mfma = ps.mfma;
    L.wg_per_cu = tuning().wg_per_cu >= 0 ? tuning().wg_per_cu : (!ps.mfma && ps.G <= 2 ? 6 : 0);
    L.wpb = tuning().waves_per_block ? tuning().waves_per_block : ps.wpb;
    L.batch = tuning().batch;
    L.need_merge = false;
    // grid: the units lengths up to cap can need (the planner's bound), else the
    // record budget; the launch caps it at the resident workgroups
    long long upper = recs;
    if (cap > 0) upper = std::min(upper, (long long)ps.hks * N * ((long long)cap / std::max(ps.min_chunk, 1) + 2));
    if (tuning().self_grid > 0) upper = std::min(upper, (long long)tuning().self_grid);
    L.units = (int)std::min<long long>(std::max(upper, 1LL), INT_MAX);
    return launch_decode(L, st);
}

// ---- allocation-free prompt attention (graph capture, callers that cannot allocate) ----
// kvc_paged_causal_attn_dev_noalloc keeps its split-K partials and arrival counters
// in this file-scope device array instead of a workspace.  Each GPU holds its own
// copy at its own address, resolved once per device with hipGetSymbolAddress (the
// array's name is only a host-side stand-in); every call on a GPU shares that GPU's
// copy, so calls that overlap on one GPU race.  Nothing in it needs clearing: the
// arrival counters carry each call's epoch and partials are written before they are
// read.
constexpr size_t kScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch;  // device address of `scratch`, per GPU

int scratch_address(void** out) {
    int dev = 0;
    int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1, nullptr);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (rc) return rc;
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return KVC_OK;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" {

int kvc_version(void) { return 100; }

const char* kvc_status_string(int s) {
    switch (s) {
        case KVC_OK: return "ok";
        case KVC_ERR_ARG: return "invalid argument";
        case KVC_ERR_UNSUPPORTED: return "unsupported shape";
        case KVC_ERR_HIP: return "HIP runtime error";
        case KVC_ERR_NOMEM: return "out of memory";
        case KVC_ERR_WORKSPACE: return "workspace too small";
        case KVC_ERR_STATE: return "invalid state";
        default: return "unknown status";
    }
}

const char* kvc_last_error(void) { return g_last_error.c_str(); }

int kvc_device_count(int* count) {
    if (!count) return set_error(KVC_ERR_ARG, "null count");
    *count = 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return KVC_OK;  // no device: count 0
    *count = n;
    return KVC_OK;
}

int kvc_malloc(void** dptr, size_t bytes) {
    if (!dptr) return set_error(KVC_ERR_ARG, "null out pointer");
    *dptr = nullptr;
    if (bytes == 0) return KVC_OK;
    if (hipMalloc(dptr, bytes) != hipSuccess) {
        *dptr = nullptr;
        return set_error(KVC_ERR_NOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    return KVC_OK;
}
int kvc_free(void* dptr) { return dptr ? hip_check(hipFree(dptr), "hipFree") : KVC_OK; }
int kvc_host_alloc(void** hptr, size_t bytes) {
    if (!hptr) return set_error(KVC_ERR_ARG, "null out pointer");
    *hptr = nullptr;
    if (bytes == 0) return KVC_OK;
    if (hipHostMalloc(hptr, bytes, hipHostMallocDefault) != hipSuccess) {
        *hptr = nullptr;
        return set_error(KVC_ERR_NOMEM, "hipHostMalloc failed");
    }
    return KVC_OK;
}
int kvc_host_free(void* hptr) { return hptr ? hip_check(hipHostFree(hptr), "hipHostFree") : KVC_OK; }
int kvc_memcpy_h2d(void* dst, const void* src, size_t bytes, kvc_stream_t st) {
    if (!bytes) return KVC_OK;
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(st)), "hipMemcpyAsync H2D");
}
int kvc_memcpy_d2h(void* dst, const void* src, size_t bytes, kvc_stream_t st) {
    if (!bytes) return KVC_OK;
    int rc = hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(st)), "hipMemcpyAsync D2H");
    return rc ? rc : hip_check(hipStreamSynchronize(S(st)), "hipStreamSynchronize");
}
int kvc_memcpy_d2d(void* dst, const void* src, size_t bytes, kvc_stream_t st) {
    if (!bytes) return KVC_OK;
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(st)), "hipMemcpyAsync D2D");
}
int kvc_memset(void* dst, int value, size_t bytes, kvc_stream_t st) {
    if (!bytes) return KVC_OK;
    return hip_check(hipMemsetAsync(dst, value, bytes, S(st)), "hipMemsetAsync");
}
int kvc_stream_create(kvc_stream_t* st) {
    if (!st) return set_error(KVC_ERR_ARG, "null out pointer");
    hipStream_t s = nullptr;
    int rc = hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *st = s;
    return rc;
}
int kvc_stream_destroy(kvc_stream_t st) { return st ? hip_check(hipStreamDestroy(S(st)), "hipStreamDestroy") : KVC_OK; }
int kvc_stream_synchronize(kvc_stream_t st) { return hip_check(hipStreamSynchronize(S(st)), "hipStreamSynchronize"); }
int kvc_device_synchronize(void) { return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
int kvc_event_create(void** ev) {
    if (!ev) return set_error(KVC_ERR_ARG, "null out pointer");
    hipEvent_t e = nullptr;
    int rc = hip_check(hipEventCreate(&e), "hipEventCreate");
    *ev = e;
    return rc;
}
int kvc_read_probe_planned(const void* k_pool, const void* v_pool, const int* table_all, int table_len,
                           const int* work, int n_units, int Hq, int Hkv, int D, int BLOCK, int dtype, int* sink,
                           kvc_stream_t st) {
    return guarded([&]() -> int {
        if (n_units < 0 || table_len < 0) return set_error(KVC_ERR_ARG, "n_units and table_len must be >= 0");
        if (n_units == 0) return KVC_OK;
        if (!k_pool || !v_pool || !table_all || !work || !sink) return set_error(KVC_ERR_ARG, "null pointer");
        if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || BLOCK <= 0 || !d_ok(D) || !dtype_ok(dtype))
            return set_error(KVC_ERR_ARG, "bad shape");
        const PlanShape ps = plan_shape(Hq, Hkv, D, BLOCK, dtype);
        const int row = D * esize(dtype);
        const int tpw = 1024 / row;
        const int lpb = BLOCK % tpw == 0 ? ilog2_exact(BLOCK / tpw) : -1;
        if (row > 1024 || lpb < 0 || ilog2_exact(tpw) < 0)
            return set_error(KVC_ERR_UNSUPPORTED, "the read probe needs blocks of a power-of-two number of 1 KiB loads");
        if (!aligned16(k_pool) || !aligned16(v_pool)) return set_error(KVC_ERR_ARG, "pools must be 16-byte aligned");
        ProbeParams p{};
        p.k = k_pool; p.v = v_pool; p.table_all = table_all; p.table_len = table_len;
        p.Hkv = Hkv; p.block = BLOCK; p.nsub = ps.mfma ? 1 : ps.nsub;
        p.row_bytes = row; p.tpw_shift = ilog2_exact(tpw); p.lpb_shift = lpb; p.sink = sink;
        return launch_read_probe(p, work, ps.entry_ints, n_units, S(st));
    });
}
int kvc_empty_launch(int blocks, kvc_stream_t st) {
    if (blocks < 1 || blocks > 65535) return set_error(KVC_ERR_ARG, "blocks must be in 1..65535");
    return launch_empty(blocks, S(st));
}
int kvc_stream_is_capturing(kvc_stream_t st, int* capturing) {
    if (!capturing) return set_error(KVC_ERR_ARG, "null out pointer");
    *capturing = 0;
    if (st == nullptr) return KVC_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    int rc = hip_check(hipStreamIsCapturing(S(st), &cs), "hipStreamIsCapturing");
    if (rc == KVC_OK) *capturing = cs != hipStreamCaptureStatusNone ? 1 : 0;
    return rc;
}
int kvc_check_device_errors(kvc_stream_t st) {
    return guarded([&]() -> int {
        if (stream_capturing(S(st)))
            return set_error(KVC_ERR_STATE, "kvc_check_device_errors synchronizes: not under stream capture");
        int rc = hip_check(hipStreamSynchronize(S(st)), "hipStreamSynchronize");
        if (rc) return rc;
        return device_error_status(take_device_error());
    });
}
int kvc_graph_begin(kvc_stream_t st) {
    return hip_check(hipStreamBeginCapture(S(st), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}
int kvc_graph_end(kvc_stream_t st, void** exec) {
    if (!exec) return set_error(KVC_ERR_ARG, "null out pointer");
    *exec = nullptr;
    hipGraph_t g = nullptr;
    int rc = hip_check(hipStreamEndCapture(S(st), &g), "hipStreamEndCapture");
    if (rc) return rc;
    hipGraphExec_t e = nullptr;
    rc = hip_check(hipGraphInstantiate(&e, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc == KVC_OK) *exec = e;
    return rc;
}
int kvc_graph_launch(void* exec, kvc_stream_t st) {
    if (!exec) return set_error(KVC_ERR_ARG, "null graph");
    return hip_check(hipGraphLaunch((hipGraphExec_t)exec, S(st)), "hipGraphLaunch");
}
int kvc_graph_destroy(void* exec) {
    return exec ? hip_check(hipGraphExecDestroy((hipGraphExec_t)exec), "hipGraphExecDestroy") : KVC_OK;
}
int kvc_event_destroy(void* ev) { return ev ? hip_check(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy") : KVC_OK; }
int kvc_event_record(void* ev, kvc_stream_t st) { return hip_check(hipEventRecord((hipEvent_t)ev, S(st)), "hipEventRecord"); }
int kvc_event_synchronize(void* ev) { return hip_check(hipEventSynchronize((hipEvent_t)ev), "hipEventSynchronize"); }
int kvc_stream_wait_event(kvc_stream_t st, void* ev) {
    return hip_check(hipStreamWaitEvent(S(st), (hipEvent_t)ev, 0), "hipStreamWaitEvent");
}
int kvc_event_elapsed_ms(float* ms, void* a, void* b) {
    if (!ms) return set_error(KVC_ERR_ARG, "null out pointer");
    int rc = hip_check(hipEventSynchronize((hipEvent_t)b), "hipEventSynchronize");
    if (rc) return rc;
    return hip_check(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime");
}

int kvc_step_upload(void* dst, const void* src, size_t bytes, kvc_stream_t st) {
    if (!bytes) return KVC_OK;
    if (!dst || !src) return set_error(KVC_ERR_ARG, "null upload pointer");
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(st)), "step upload");
}

int kvc_fill_normal(void* dst, size_t n, int dtype, uint64_t seed, float stddev, kvc_stream_t st) {
    if (!dtype_ok(dtype)) return set_error(KVC_ERR_ARG, "bad dtype");
    if (n && !dst) return set_error(KVC_ERR_ARG, "null fill pointer");
    return launch_fill_normal(dst, n, dtype, seed, stddev, S(st));
}

// ---- K/V writes ------------------------------------------------------------
static int write_common(int dtype, int heads, int D, const void* k, const void* v, void* kd, void* vd) {
    if (!dtype_ok(dtype)) return set_error(KVC_ERR_ARG, "bad dtype");
    if (heads <= 0 || D <= 0) return set_error(KVC_ERR_ARG, "heads and D must be > 0");
    if (!k || !v || !kd || !vd) return set_error(KVC_ERR_ARG, "null K/V pointer");
    return KVC_OK;
}

int kvc_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache, int pos, int H, int D,
               int S_, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        int rc = write_common(dtype, H, D, k_new, v_new, k_cache, v_cache);
        if (rc) return rc;
        if (pos < 0 || pos >= S_) return set_error(KVC_ERR_ARG, "pos must be in [0, S)");
        WriteParams p{k_new, v_new, k_cache, v_cache, nullptr, nullptr, nullptr, 1, H, D, 1, pos, S_, kWriteAppend};
        return launch_write(p, dtype, S(st));
    });
}

int kvc_write_kv(const void* k, const void* v, void* k_pool, void* v_pool, const int* block_table, int start_pos,
                 int L, int Hkv, int D, int BLOCK, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        int rc = write_common(dtype, Hkv, D, k, v, k_pool, v_pool);
        if (rc) return rc;
        if (L < 0 || start_pos < 0 || BLOCK <= 0) return set_error(KVC_ERR_ARG, "bad L / start_pos / BLOCK");
        if (L > 0 && !block_table) return set_error(KVC_ERR_ARG, "null block table");
        WriteParams p{k, v, k_pool, v_pool, block_table, nullptr, nullptr, L, Hkv, D, BLOCK, start_pos, 0, kWriteTable};
        return launch_write(p, dtype, S(st));
    });
}

int kvc_write_kv_dev(const void* k, const void* v, void* k_pool, void* v_pool, const int* block_table,
                     const int* dev_start_pos, int L, int Hkv, int D, int BLOCK, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        int rc = write_common(dtype, Hkv, D, k, v, k_pool, v_pool);
        if (rc) return rc;
        if (L < 0 || BLOCK <= 0) return set_error(KVC_ERR_ARG, "bad L / BLOCK");
        if (L > 0 && (!block_table || !dev_start_pos)) return set_error(KVC_ERR_ARG, "null block table / start");
        WriteParams p{k, v, k_pool, v_pool, block_table, nullptr, nullptr, L, Hkv, D, BLOCK, 0, 0, kWriteTable,
                      dev_start_pos};
        return launch_write(p, dtype, S(st));
    });
}

int kvc_batched_write_kv(const void* k, const void* v, void* k_pool, void* v_pool, const int* table_all,
                         const int* tab_off, const int* wpos, int N, int Hkv, int D, int BLOCK, int dtype,
                         kvc_stream_t st) {
    return guarded([&]() -> int {
        int rc = write_common(dtype, Hkv, D, k, v, k_pool, v_pool);
        if (rc) return rc;
        if (N < 0 || BLOCK <= 0) return set_error(KVC_ERR_ARG, "bad N / BLOCK");
        if (N > 0 && (!table_all || !tab_off || !wpos)) return set_error(KVC_ERR_ARG, "null table / offsets / wpos");
        WriteParams p{k, v, k_pool, v_pool, table_all, tab_off, wpos, N, Hkv, D, BLOCK, 0, 0, kWriteBatched};
        return launch_write(p, dtype, S(st));
    });
}

int kvc_write_kv_slots(const void* k, const void* v, void* k_pool, void* v_pool, const int* slot_map, int rows,
                       int Hkv, int D, int BLOCK, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        int rc = write_common(dtype, Hkv, D, k, v, k_pool, v_pool);
        if (rc) return rc;
        if (rows < 0 || BLOCK <= 0) return set_error(KVC_ERR_ARG, "bad rows / BLOCK");
        if (rows > 0 && !slot_map) return set_error(KVC_ERR_ARG, "null slot map");
        WriteParams p{k, v, k_pool, v_pool, nullptr, nullptr, slot_map, rows, Hkv, D, BLOCK, 0, 0, kWriteSlots};
        return launch_write(p, dtype, S(st));
    });
}

// ---- decode ------------------------------------------------------------------
int kvc_decode(const void* q, const void* k_cache, const void* v_cache, void* out, int cur_len, int H, int D,
               int S_, float scale, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (S_ < 0 || cur_len > S_) return set_error(KVC_ERR_ARG, "cur_len must be <= S");
        return run_batched(q, k_cache, v_cache, nullptr, nullptr, nullptr, cur_len, out, 1, H, H, D, 0, 0,
                           (long long)S_ * D, std::max(cur_len, 0), scale, dtype, 0, false, nullptr, 0, S(st));
    });
}

int kvc_paged_decode(const void* q, const void* k_pool, const void* v_pool, const int* block_table, void* out,
                     int cur_len, int H, int D, int BLOCK, float scale, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        return run_batched(q, k_pool, v_pool, block_table, nullptr, nullptr, cur_len, out, 1, H, H, D, BLOCK, 0, 0,
                           std::max(cur_len, 0), scale, dtype, 0, true, nullptr, 0, S(st));
    });
}

int kvc_batched_decode(const void* q, const void* k_cache, const void* v_cache, const int* cur_len, void* out, int N,
                       int Hq, int Hkv, int D, int MAXS, int cap, float scale, int dtype, void* ws, size_t ws_bytes,
                       kvc_stream_t st) {
    return kvc_batched_decode_split(q, k_cache, v_cache, cur_len, out, N, Hq, Hkv, D, MAXS, cap, scale, dtype, 0, ws,
                                    ws_bytes, st);
}

int kvc_batched_decode_split(const void* q, const void* k_cache, const void* v_cache, const int* cur_len, void* out,
                             int N, int Hq, int Hkv, int D, int MAXS, int cap, float scale, int dtype, int split,
                             void* ws, size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (MAXS < 0 || cap < 0 || cap > MAXS) return set_error(KVC_ERR_ARG, "cap must be in [0, MAXS]");
        if (N > 0 && !cur_len) return set_error(KVC_ERR_ARG, "null cur_len");
        int rc = check_common(N, Hq, Hkv, D, dtype, q, k_cache, v_cache, out);
        if (rc || N == 0) return rc;
        rc = pending_device_error();
        if (rc) return rc;
        // automatic split: the kernel plans from the device lengths, with the chunks of
        // the paged path (so paged and contiguous batches agree bit for bit)
        if (split == 0 && tuning().self_plan != 0 && self_plan_ok(N, Hq, Hkv, D, kSelfContigBlock, dtype, cap))
            return run_self_planned(q, k_cache, v_cache, nullptr, nullptr, cur_len, nullptr, out, N, Hq, Hkv, D, 0,
                                    cap, scale, dtype, ws, ws_bytes, S(st), true, (long long)Hkv * MAXS * D,
                                    (long long)MAXS * D);
        // every length is at most MAXS (the cache's extent): cap 0 means that bound
        return run_batched(q, k_cache, v_cache, nullptr, nullptr, cur_len, 0, out, N, Hq, Hkv, D, 0,
                           (long long)Hkv * MAXS * D, (long long)MAXS * D, cap > 0 ? cap : MAXS, scale, dtype, split,
                           false, ws, ws_bytes, S(st));
    });
}

int kvc_batched_paged_decode(const void* q, const void* k_pool, const void* v_pool, const int* table_all,
                             const int* tab_off, const int* cur_len, void* out, int N, int Hq, int Hkv, int D,
                             int BLOCK, int cap, float scale, int dtype, void* ws, size_t ws_bytes, kvc_stream_t st) {
    return kvc_batched_paged_decode_split(q, k_pool, v_pool, table_all, tab_off, cur_len, out, N, Hq, Hkv, D, BLOCK,
                                          cap, scale, dtype, 0, ws, ws_bytes, st);
}

int kvc_batched_paged_decode_split(const void* q, const void* k_pool, const void* v_pool, const int* table_all,
                                   const int* tab_off, const int* cur_len, void* out, int N, int Hq, int Hkv, int D,
                                   int BLOCK, int cap, float scale, int dtype, int split, void* ws, size_t ws_bytes,
                                   kvc_stream_t st) {
    return guarded([&]() -> int {
        if (N > 0 && (!tab_off || !cur_len)) return set_error(KVC_ERR_ARG, "null tab_off / cur_len");
        if (cap < 0) return set_error(KVC_ERR_ARG, "cap must be >= 0");
        int rc = check_common(N, Hq, Hkv, D, dtype, q, k_pool, v_pool, out);
        if (rc || N == 0) return rc;
        if (BLOCK <= 0 || !table_all) return set_error(KVC_ERR_ARG, "paged decode needs BLOCK > 0 and a block table");
        rc = pending_device_error();
        if (rc) return rc;
        if (split == 0 && tuning().self_plan != 0) {
            // automatic split: the kernel plans from the device lengths (cap only a hint)
            if (self_plan_ok(N, Hq, Hkv, D, BLOCK, dtype, cap))
                return run_self_planned(q, k_pool, v_pool, table_all, tab_off, cur_len, nullptr, out, N, Hq, Hkv, D,
                                        BLOCK, cap, scale, dtype, ws, ws_bytes, S(st));
            // more sequences than one self-planned launch plans: consecutive groups of
            // them, one launch each (the launches share the workspace in stream order)
            const int group = self_plan_group(N, Hq, Hkv, D, BLOCK, dtype, cap);
            if (group > 0) {
                const size_t qrow = (size_t)Hq * D * esize(dtype);
                for (int g0 = 0; g0 < N; g0 += group) {
                    const int n = std::min(group, N - g0);
                    rc = run_self_planned(static_cast<const char*>(q) + g0 * qrow, k_pool, v_pool, table_all,
                                          tab_off + g0, cur_len + g0, nullptr, static_cast<char*>(out) + g0 * qrow, n,
                                          Hq, Hkv, D, BLOCK, cap, scale, dtype, ws, ws_bytes, S(st));
                    if (rc) return rc;
                }
                return KVC_OK;
            }
        }
        if (cap == 0 && N > 0) {
            // no self-planned path and no bound stated: the longest length is read from the
            // device (a synchronisation; refused under stream capture) and sizes the grid
            if (stream_capturing(S(st)))
                return set_error(KVC_ERR_STATE, "this shape has no self-planned path: under stream capture it needs "
                                                "cap, the longest length");
            std::vector<int> h(N);
            rc = hip_check(hipMemcpyAsync(h.data(), cur_len, (size_t)N * sizeof(int), hipMemcpyDeviceToHost, S(st)),
                           "hipMemcpyAsync (lengths)");
            if (rc) return rc;
            rc = hip_check(hipStreamSynchronize(S(st)), "hipStreamSynchronize (lengths)");
            if (rc) return rc;
            cap = std::max(1, *std::max_element(h.begin(), h.end()));
        }
        return run_batched(q, k_pool, v_pool, table_all, tab_off, cur_len, 0, out, N, Hq, Hkv, D, BLOCK, 0, 0, cap,
                           scale, dtype, split, true, ws, ws_bytes, S(st));
    });
}

int kvc_paged_causal_attn(const void* q, void* out, const void* k_pool, const void* v_pool, const int* block_table,
                          int q_pos_base, int Nq, int Hq, int Hkv, int D, int BLOCK, float scale, int dtype, void* ws,
                          size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (q_pos_base < 0 || Nq < 0) return set_error(KVC_ERR_ARG, "q_pos_base and Nq must be >= 0");
        if ((long long)q_pos_base + Nq > INT_MAX) return set_error(KVC_ERR_ARG, "q_pos_base + Nq overflows");
        if (causal_tile_path(Nq, Hq, Hkv, D, BLOCK, dtype))
            return run_causal_tile(q, out, k_pool, v_pool, block_table, q_pos_base, Nq, Hq, Hkv, D, BLOCK, scale, ws,
                                   ws_bytes, S(st));
        // query i is a sequence of length q_pos_base + i + 1 over the one block table
        return run_batched(q, k_pool, v_pool, block_table, nullptr, nullptr, q_pos_base, out, Nq, Hq, Hkv, D, BLOCK,
                           0, 0, q_pos_base + Nq, scale, dtype, 0, true, ws, ws_bytes, S(st), 1);
    });
}

int kvc_paged_causal_attn_dev(const void* q, void* out, const void* k_pool, const void* v_pool, const int* block_table,
                              const int* dev_q_pos_base, int Nq, int Hq, int Hkv, int D, int BLOCK, float scale,
                              int dtype, void* ws, size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (Nq < 0) return set_error(KVC_ERR_ARG, "Nq must be >= 0");
        if (Nq > 0 && !dev_q_pos_base) return set_error(KVC_ERR_ARG, "null q_pos_base pointer");
        int rc = pending_device_error();
        if (rc) return rc;
        if (Nq > 0 && !self_plan_ok(Nq, Hq, Hkv, D, BLOCK, dtype))
            return set_error(KVC_ERR_UNSUPPORTED, "device-position prompt attention needs a power-of-two BLOCK the "
                                                  "kernels page uniformly and at most 512 queries");
        return run_self_planned(q, k_pool, v_pool, block_table, nullptr, nullptr, dev_q_pos_base, out, Nq, Hq, Hkv,
                                D, BLOCK, 0, scale, dtype, ws, ws_bytes, S(st));
    });
}

size_t kvc_paged_causal_attn_dev_workspace_size(int Nq, int Hq, int Hkv, int D, int BLOCK, int dtype) {
    if (!self_plan_ok(Nq, Hq, Hkv, D, BLOCK, dtype)) return 0;
    return self_plan_workspace(Nq, Hq, Hkv, D, BLOCK, dtype);
}

int kvc_paged_causal_attn_dev_noalloc(const void* q, void* out, const void* k_pool, const void* v_pool,
                                      const int* block_table, const int* dev_q_pos_base, int Nq, int Hq, int Hkv,
                                      int D, int BLOCK, float scale, int dtype, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (Nq < 0) return set_error(KVC_ERR_ARG, "Nq must be >= 0");
        if (Nq == 0) return KVC_OK;
        if (!dev_q_pos_base) return set_error(KVC_ERR_ARG, "null q_pos_base pointer");
        if (!self_plan_ok(Nq, Hq, Hkv, D, BLOCK, dtype))
            return set_error(KVC_ERR_UNSUPPORTED, "device-position prompt attention needs a power-of-two BLOCK the "
                                                  "kernels page uniformly and at most 512 queries");
        const size_t need = self_plan_workspace(Nq, Hq, Hkv, D, BLOCK, dtype);
        if (need > kScratchBytes)
            return set_error(KVC_ERR_UNSUPPORTED, "allocation-free prompt attention of " + std::to_string(Nq) +
                                                      " queries needs " + std::to_string(need) +
                                                      " bytes of scratch; the static scratch holds " +
                                                      std::to_string(kScratchBytes));
        void* ws = nullptr;
        int rc = scratch_address(&ws);
        if (rc) return rc;
        return run_self_planned(q, k_pool, v_pool, block_table, nullptr, nullptr, dev_q_pos_base, out, Nq, Hq, Hkv,
                                D, BLOCK, 0, scale, dtype, ws, kScratchBytes, S(st), false, 0, 0, true);
    });
}

size_t kvc_paged_causal_attn_workspace_size(int q_pos_base, int Nq, int Hq, int Hkv, int D, int BLOCK, int dtype) {
    if (q_pos_base < 0 || Nq < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || !d_ok(D) || BLOCK <= 0) return 0;
    if (causal_tile_path(Nq, Hq, Hkv, D, BLOCK, dtype)) return plan_causal_tile(q_pos_base, Nq, Hq, Hkv, D, BLOCK).ws_bytes;
    return plan_batched(Nq, Hq, Hkv, D, BLOCK, q_pos_base + Nq, dtype, 0, true).ws_bytes;
}

int kvc_decode_plan_entry_ints(int Hq, int Hkv, int D, int BLOCK, int dtype) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || BLOCK <= 0 || !d_ok(D) || !dtype_ok(dtype)) return 0;
    return plan_shape(Hq, Hkv, D, BLOCK, dtype).entry_ints;
}

int kvc_decode_plan(const int* host_lens, const int* host_tab_off, const int* host_table_all, int host_table_len,
                    int N, int Hq, int Hkv, int D, int BLOCK, int dtype, int target_tokens, int* work, int capacity,
                    int* n_units, int* n_records) {
    return guarded([&]() -> int {
        if (!n_units || !n_records) return set_error(KVC_ERR_ARG, "null output pointer");
        if (N < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || BLOCK <= 0) return set_error(KVC_ERR_ARG, "bad shape");
        if (!d_ok(D)) return set_error(KVC_ERR_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256");
        if (!dtype_ok(dtype)) return set_error(KVC_ERR_ARG, "bad dtype");
        if (N > 0 && !host_lens) return set_error(KVC_ERR_ARG, "null lengths");
        if (host_table_all && host_table_len < 0) return set_error(KVC_ERR_ARG, "negative table length");
        return make_plan(host_lens, host_tab_off, host_table_all, host_table_all ? host_table_len : 0, N, Hq, Hkv, D,
                         BLOCK, dtype, target_tokens, work, capacity, n_units, n_records);
    });
}

size_t kvc_decode_planned_workspace_size(int Hq, int Hkv, int D, int BLOCK, int dtype, int n_records) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || !d_ok(D) || n_records < 0) return 0;
    return planned_workspace(Hq, Hkv, D, BLOCK, dtype, n_records);
}


int kvc_batched_paged_decode_planned(const void* q, const void* k_pool, const void* v_pool, const int* table_all,
                                     int table_len, void* out, int N, int Hq, int Hkv, int D, int BLOCK,
                                     float scale, int dtype, const int* work, int n_units, int n_records, void* ws,
                                     size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        return kvc::run_planned(q, nullptr, nullptr, nullptr, k_pool, v_pool, table_all, table_len, out, N, Hq, Hkv,
                                D, BLOCK, scale, dtype, work, n_units, n_records, ws, ws_bytes, S(st));
    });
}

int kvc_batched_paged_append_decode_planned(const void* q, const void* k_new, const void* v_new, const int* wpos,
                                            void* k_pool, void* v_pool, const int* table_all, int table_len,
                                            void* out, int N, int Hq, int Hkv, int D, int BLOCK, float scale,
                                            int dtype, const int* work, int n_units, int n_records, void* ws,
                                            size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (N > 0 && (!k_new || !v_new || !wpos)) return set_error(KVC_ERR_ARG, "null k_new / v_new / wpos");
        if (N > 0 && (!aligned16(k_new) || !aligned16(v_new)))
            return set_error(KVC_ERR_ARG, "k_new and v_new must be 16-byte aligned");
        return kvc::run_planned(q, k_new, v_new, wpos, k_pool, v_pool, table_all, table_len, out, N, Hq, Hkv, D,
                                BLOCK, scale, dtype, work, n_units, n_records, ws, ws_bytes, S(st));
    });
}

int kvc_batched_paged_decode_planned_dev(const void* q, const void* k_new, const void* v_new, const int* wpos,
                                        void* k_pool, void* v_pool, const int* table_all, int table_len, void* out,
                                        int N_cap, int Hq, int Hkv, int D, int BLOCK, float scale, int dtype,
                                        const int* work, int units_cap, int records_cap, const int* dev_counts,
                                        void* ws, size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        if (!dev_counts) return set_error(KVC_ERR_ARG, "null dev_counts");
        const bool append = k_new != nullptr;
        if (append && (!v_new || !wpos)) return set_error(KVC_ERR_ARG, "append needs k_new, v_new and wpos");
        if (append && (!aligned16(k_new) || !aligned16(v_new)))
            return set_error(KVC_ERR_ARG, "k_new and v_new must be 16-byte aligned");
        if (records_cap > 0 && !ws) return set_error(KVC_ERR_ARG, "a graph-safe launch needs its workspace");
        return kvc::run_planned(q, append ? k_new : nullptr, append ? v_new : nullptr, append ? wpos : nullptr,
                                k_pool, v_pool, table_all, table_len, out, N_cap, Hq, Hkv, D, BLOCK, scale, dtype,
                                work, units_cap, records_cap, ws, ws_bytes, S(st), dev_counts);
    });
}

int kvc_decode_plan_chunk(const int* host_lens, int N, int Hq, int Hkv, int D, int BLOCK, int dtype,
                          int target_tokens, int* chunk_tokens) {
    return guarded([&]() -> int {
        if (!chunk_tokens) return set_error(KVC_ERR_ARG, "null out pointer");
        *chunk_tokens = 0;
        if (N < 0 || (N > 0 && !host_lens) || Hq <= 0 || Hkv <= 0 || Hq % Hkv || BLOCK <= 0 || !d_ok(D) ||
            !dtype_ok(dtype))
            return set_error(KVC_ERR_ARG, "bad plan arguments");
        *chunk_tokens = kvc::plan_chunk_target(host_lens, N, kvc::plan_shape(Hq, Hkv, D, BLOCK, dtype), BLOCK,
                                               target_tokens);
        return KVC_OK;
    });
}

int kvc_decode_plan_capacity(int N, long long total_tokens, int Hq, int Hkv, int D, int BLOCK, int dtype,
                             int* max_units) {
    return guarded([&]() -> int {
        if (!max_units) return set_error(KVC_ERR_ARG, "null out pointer");
        *max_units = 0;
        if (N < 0 || total_tokens < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || BLOCK <= 0)
            return set_error(KVC_ERR_ARG, "bad plan capacity arguments");
        const kvc::PlanShape ps = kvc::plan_shape(Hq, Hkv, D, BLOCK, dtype);
        // a sequence of L tokens is cut into at most L / min_chunk + 1 chunks per head slot
        const long long units = (long long)ps.hks * ((long long)N + total_tokens / std::max(ps.min_chunk, 1) + 1);
        if (units > INT_MAX) return set_error(KVC_ERR_ARG, "plan capacity too large");
        *max_units = (int)units;
        return KVC_OK;
    });
}

size_t kvc_decode_workspace_size(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int split, int dtype) {
    if (N <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || !d_ok(D) || cap < 0 || split < 0 || !dtype_ok(dtype)) return 0;
    if (split == 0 && tuning().self_plan != 0) {
        const int b = BLOCK > 0 ? BLOCK : kSelfContigBlock;
        if (self_plan_ok(N, Hq, Hkv, D, b, dtype, cap)) return self_plan_workspace(N, Hq, Hkv, D, b, dtype, cap);
        // paged batches larger than one self-planned launch: consecutive groups
        const int g = BLOCK > 0 ? self_plan_group(N, Hq, Hkv, D, b, dtype, cap) : 0;
        if (g > 0) return self_plan_workspace(g, Hq, Hkv, D, b, dtype, cap);
    }
    return plan_batched(N, Hq, Hkv, D, BLOCK, cap, dtype, split, BLOCK > 0).ws_bytes;
}

int kvc_decode_auto_split(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int dtype) {
    if (N <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || !d_ok(D) || cap < 0 || !dtype_ok(dtype)) return 0;
    return auto_split(N, Hq, Hkv, D, BLOCK, cap, dtype);
}

size_t kvc_flash_decode_workspace_size(int H, int D, int num_splits) {
    if (H <= 0 || !d_ok(D) || num_splits <= 1) return 0;
    Plan pl;
    pl.max_chunks = num_splits;
    size_workspace(pl, 1, H, H, D);
    return pl.ws_bytes;
}

int kvc_set_tuning(const char* key, int value) {
    if (!key) return set_error(KVC_ERR_ARG, "null key");
    const std::string k(key);
    if (k == "fused_merge" && value >= -1 && value <= 2) tuning().fused_merge = value;
    else if (k == "target_units" && value > 0) tuning().target_units = value;
    else if (k == "min_chunk_bytes" && value > 0) tuning().min_chunk_bytes = value;
    else if (k == "waves_per_block" && (value == 0 || value == 4 || value == 8)) tuning().waves_per_block = value;
    else if (k == "batch" && (value == 2 || value == 4 || value == 8)) tuning().batch = value;
    else if (k == "last_chunk_first" && (value == 0 || value == 1)) tuning().last_chunk_first = value;
    else if (k == "mfma" && value >= -1 && value <= 1) tuning().mfma = value;
    else if (k == "wg_per_cu" && value >= -1 && value <= 32) tuning().wg_per_cu = value;
    else if (k == "split_first" && (value == 0 || value == 1)) tuning().split_first = value;
    else if (k == "mfma_min_chunk" && value >= 16 && value <= 1 << 20) tuning().mfma_min_chunk = value;
    else if (k == "self_plan" && (value == 0 || value == 1)) tuning().self_plan = value;
    else if (k == "self_grid" && value >= 0) tuning().self_grid = value;
    else if (k == "self_prefetch_kib" && value >= 0) tuning().self_prefetch_kib = value;
    else if (k == "self_prefetch_min_len" && value >= 0) tuning().self_prefetch_min_len = value;
    else if (k == "self_prefetch_xcd" && (value == 0 || value == 1)) tuning().self_prefetch_xcd = value;
    else if (k == "self_lead_tokens" && value >= 0) tuning().self_lead_tokens = value;
    else if (k == "chain_spin" && value >= 0) tuning().chain_spin = value;
    else return set_error(KVC_ERR_ARG, "unknown tuning key or bad value: " + k);
    return KVC_OK;
}

int kvc_get_tuning(const char* key, int* value) {
    if (!key || !value) return set_error(KVC_ERR_ARG, "null argument");
    const std::string k(key);
    if (k == "fused_merge") *value = tuning().fused_merge;
    else if (k == "target_units") *value = tuning().target_units;
    else if (k == "min_chunk_bytes") *value = tuning().min_chunk_bytes;
    else if (k == "waves_per_block") *value = tuning().waves_per_block;
    else if (k == "batch") *value = tuning().batch;
    else if (k == "last_chunk_first") *value = tuning().last_chunk_first;
    else if (k == "mfma") *value = tuning().mfma;
    else if (k == "wg_per_cu") *value = tuning().wg_per_cu;
    else if (k == "split_first") *value = tuning().split_first;
    else if (k == "mfma_min_chunk") *value = tuning().mfma_min_chunk;
    else if (k == "self_plan") *value = tuning().self_plan;
    else if (k == "self_grid") *value = tuning().self_grid;
    else if (k == "self_prefetch_kib") *value = tuning().self_prefetch_kib;
    else if (k == "self_prefetch_min_len") *value = tuning().self_prefetch_min_len;
    else if (k == "self_prefetch_xcd") *value = tuning().self_prefetch_xcd;
    else if (k == "self_lead_tokens") *value = tuning().self_lead_tokens;
    else if (k == "chain_spin") *value = tuning().chain_spin;
    else return set_error(KVC_ERR_ARG, "unknown tuning key: " + k);
    return KVC_OK;
}

int kvc_flash_decode(const void* q, const void* k_cache, const void* v_cache, void* out, int cur_len, int H, int D,
                     int S_, float scale, int num_splits, int dtype, void* ws, size_t ws_bytes, kvc_stream_t st) {
    return guarded([&]() -> int {
        int rc = check_common(1, H, H, D, dtype, q, k_cache, v_cache, out);
        if (rc) return rc;
        if (S_ < 0 || cur_len > S_) return set_error(KVC_ERR_ARG, "cur_len must be <= S");
        if (!std::isfinite(scale)) return set_error(KVC_ERR_ARG, "scale must be finite");
        int ns = std::max(1, num_splits);          // flash_decode.cu:106-107
        ns = std::max(1, std::min(ns, cur_len));
        Plan pl;
        pl.max_chunks = ns;
        size_workspace(pl, 1, H, H, D);
        DecodeLaunch L{};
        DecodeParams& p = L.p;
        p.q = q; p.k = k_cache; p.v = v_cache; p.out = out;
        p.fixed_len = std::max(cur_len, 0);
        p.cap = p.fixed_len;
        p.seq_stride = 0; p.head_stride = (long long)S_ * D;
        p.N = 1; p.Hq = H; p.Hkv = H; p.block = 1; p.group = 1; p.nsub = 1;
        p.chunk_tokens = 0; p.num_splits = ns; p.max_chunks = ns;
        p.scale_log2 = scale * 1.4426950408889634f;
        rc = resolve_workspace(pl, ws, ws_bytes, p, S(st));
        if (rc) return rc;
        p.last_chunk_first = tuning().last_chunk_first;
        L.dtype = dtype; L.D = D; L.G = 1; L.mode = kContiguous; L.wpb = choose_wpb((long long)ns * H);
        L.batch = tuning().batch;
        L.need_merge = ns > 1;
        return launch_decode(L, S(st));
    });
}

}  // extern "C"
