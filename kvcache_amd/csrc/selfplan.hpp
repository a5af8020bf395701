// selfplan.hpp -- decode units planned by the kernel from lengths in device memory.
//
// Included by decode_kernels.hpp inside namespace kvc::{anonymous}; uses its helpers.
//
// The reference's launchers take the lengths as a device array
// (launch_batched_paged, batched.cu:140-147; qk_batched_paged_decode_attn,
// qwen_kernels.cu:293-326), so the host cannot plan the launch without a copy and
// a synchronisation.  Instead every workgroup of a persistent grid derives the
// host planner's work (kvc_decode_plan: the same chunk target, the same chunks,
// the same partial-record and counter numbering) from the lengths, puts the units in
// one order -- eight buckets, chunks of split sequences first, then by length,
// longest first; within a bucket by sequence -- and serves ranks in rounds of
// gridDim.x (self_plan_rank).  Every workgroup computes the same order from the same
// data, so each unit runs exactly once, and outputs equal the host-planned launch's
// bit for bit (same chunks, same merge order); only the order in which units run
// differs from the host plan's.  On the VALU kernel a sequence of at most p.sp_lead
// tokens is attended instead by waves 1.. of workgroup s * hks + h while wave 0 plans
// (self_plan_loop), and the plan leaves it out: the other sequences' units are the
// host plan's, the short ones differ from it only in rounding (three waves share them).
//
// Budget: every (sequence, KV head) may use up to p.sp_records partial records (64,
// or more when the caller states a long bound), and on the matrix-core path a
// sequence has at most 64 chunks; the chunk target is raised when the lengths need
// it (mean length / (sp_records - 1), longest length / 63).  A batch that cannot fit
// even at the largest chunk, or with a length past its contiguous cache (p.cap),
// gets NaN outputs: never a silent partial attention.
//
// Cost structure.  A lone wave issues a dependent VALU instruction every ~6 cycles,
// so the setup is one wave of short dependent chains: the lengths load at wave start
// (their pointer is the kernel's preloaded first argument); wave scans give the
// totals (tokens, longest length, table blocks) and the chunk target, in 32-bit
// integer arithmetic (the 64-bit forms only past 2^32 tokens); each lane splits its
// sequences and counts their units per bucket; eight wave scans give every lane the
// first rank of its runs in each bucket; then the lane holding each of this
// workgroup's ranks in a window of kSelfWindow rounds writes its header into LDS; one
// barrier, and the persistent loop only reads a header per unit.  Batches needing
// more rounds repeat the setup per window.

constexpr int kSelfMaxNValu = 1024;   // sequences per launch (their plan rows live in LDS)
constexpr int kSelfMaxNMfma = 512;    // (keeps the matrix-core kernel's LDS within two workgroups per CU)
constexpr int kSelfSpt = 4;           // length loads in flight per lane of the planning wave
constexpr int kSelfBuckets = 8;       // order buckets: 4 for chunks of split sequences, 4 for whole sequences
constexpr int kSelfMaxChunks = 0xFFFF;  // chunks of one sequence (16-bit plan field)
constexpr int kSelfWindow = 16;       // rounds whose unit headers a workgroup resolves per setup

template <int NMAX, int NW, bool LEAD = false>
struct SelfPlanLds {
    static constexpr bool kLead = LEAD;  // the kernel attends short sequences while it plans (sp_lead)
    int len[NMAX];             // attended length of each sequence (>= 0)
    int to[NMAX];              // first table entry of each sequence
    int cut[NMAX];             // chunks | chunk length in blocks << 16
    int bk[NMAX];              // bucket of run A | bucket of run B << 4
    int plan[4];               // chunk target, units, overflow
    int hdr[kSelfWindow][8];   // unit headers of this workgroup's ranks in the window (hdr[k][0] < 0: none)
    int sink[kWave];           // destination of the prefetch loads (never read)
};

struct SelfPlan {
    int T, units, overflow;
};

// Inclusive prefix sum over the 64 lanes with DPP: shifts of 1, 2, 4, 8 within each
// row of 16 lanes, then row 0's total into row 1 and row 2's into row 3 (row_bcast:15),
// then the first two rows' total into rows 2 and 3 (row_bcast:31).  Out-of-row sources
// and disabled rows contribute 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
    return x;
}

// Running maximum over the lanes (the same pattern); values >= 0.
__device__ __forceinline__ int wave_incl_max(int x) {
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));
    return x;
}

// ceil(a / b), 64-bit, for the rare launches past 32-bit token counts (a < 2^53,
// 0 < b < 2^53): a double quotient corrected to the exact integer.
__device__ __forceinline__ long long ceil_div_u64(long long a, long long b) {
    long long q = (long long)((double)a / (double)b);
    while (q * b < a) ++q;
    while (q > 0 && (q - 1) * b >= a) --q;
    return q;
}

// ceil(a / b) in 32 bits (b > 0), without overflow near 2^32.
__device__ __forceinline__ unsigned ceil_div_u32(unsigned a, unsigned b) {
    const unsigned q = a / b;
    return q + (q * b < a ? 1u : 0u);
}

// Chunks of a sequence of L tokens at chunk target T (make_plan in abi.hip), in
// 32-bit unsigned arithmetic (L < 2^31, T < 2^30).  BLOCK is a power of two.
__device__ __forceinline__ void self_split(const DecodeParams& p, int L, int T, int bsh, int& nc, int& chunk) {
    nc = 1;
    chunk = max(L, 1);
    const unsigned uL = (unsigned)L, uT = (unsigned)T, mc = (unsigned)p.sp_max_chunk;
    if (uL > mc || uL > uT + uT / 2) {
        unsigned n = max(2u, (uL + uT / 2) / uT);
        n = max(n, (uL + mc - 1) / mc);
        if (p.sp_nc_max) n = min(n, (unsigned)p.sp_nc_max);
        unsigned ch = (uL + n - 1) / n;
        ch = ((ch + (1u << bsh) - 1) >> bsh) << bsh;
        chunk = (int)ch;
        nc = (int)((uL + ch - 1) / ch);
    }
}

// Order bucket of a run of units of `len` tokens each: chunks of split sequences
// (4..7) above whole sequences (0..3), longer above shorter, in quarters of 3T/8
// (kscale = 8 / 3T).  Buckets only order the units; chunks, records and counters do
// not depend on them.
__device__ __forceinline__ int self_bucket(bool split, int len, float kscale) {
    return (split ? 4 : 0) + min(3, (int)((float)len * kscale));
}

// The k-th rank workgroup b serves: the grid walks the ranks in rounds of gridDim.x,
// in alternating direction (ranks run longest first, so the workgroup with the
// longest unit of one round gets the shortest of the next).  Each rank is served
// once; no counter, no atomics (a shared counter serialised ~1000 arrivals into tens
// of microseconds).
__device__ __forceinline__ int self_plan_rank(int k) {
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
    return k * G + ((k & 1) ? G - 1 - b : b);
}

// Reads the lengths (`lens`, device memory; NULL: causal prompt queries) and table
// offsets, picks the chunk target, cuts every sequence into chunks, orders the units
// and writes the headers of this workgroup's ranks in rounds [kw, kw + kSelfWindow)
// into S.hdr.  Wave 0 does all of it -- lane l owns the consecutive sequences
// [l * spl, l * spl + spl), so every reduction and ordering is one wave scan -- while
// the other waves wait at the closing barrier; every wave then returns the same plan.
// Order: eight buckets (self_bucket), descending; within a bucket by sequence, and
// within a sequence run A (chunks 0..nc-2, the hks heads of each chunk in turn)
// before run B (its last chunk of every head).  Every run holds a multiple of hks
// units, so a unit's rank is congruent to its head modulo hks: with hks a multiple of
// 8, the unit of head h at rank r < gridDim.x runs on workgroup r, which the hardware
// places on XCD r mod 8 = h mod 8 (self_prefetch relies on this).
// Wave 0's first kSelfSpt lengths (lane l: sequences l * spl ...), loaded before
// anything else of the kernel: they depend only on the preloaded arguments.
__device__ __forceinline__ void self_first_lengths(const int* lens, int N, int (&lv0)[kSelfSpt]) {
    const int lane = threadIdx.x & (kWave - 1);
    const int i0 = min(lane * ((N + kWave - 1) / kWave), N);
    const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(lens, lens ? N * 4 : 0);
#pragma unroll
    for (int j = 0; j < kSelfSpt; ++j) lv0[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(lrs, (i0 + j) * 4, 0, 0);
}

template <int NT, typename Lds>
__device__ SelfPlan self_plan_setup(const int* lens, int n_seq, const DecodeParams& p, Lds& S, int kw,
                                    const int (&lv0)[kSelfSpt]) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    if (tid < kWave) {
        const int N = n_seq;
        const int spl = (N + kWave - 1) / kWave;  // consecutive sequences per lane
        const int i0 = min(lane * spl, N), i1 = min(i0 + spl, N);
        const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(lens, lens ? N * 4 : 0);
        const int B = p.block, hks = p.Hkv * p.nsub;
        const int bsh = __builtin_ctz((unsigned)B);
        const int first = lens ? 0 : (p.dev_base ? *p.dev_base : p.fixed_len);  // causal prompt queries
        const int P = Lds::kLead ? p.sp_lead : 0;  // sequences of at most P tokens are not planned
        if (lane < kSelfWindow) S.hdr[lane][0] = -1;
        // this lane's table offsets: issued as soon as the parameter block is in, first
        // used when the headers are written (bounded buffer loads: indices past N read
        // 0 and touch no memory)
        const bool offsets = p.tab_off && !p.causal;
        const __amdgpu_buffer_rsrc_t trs = tile_rsrc(p.tab_off, offsets ? N * 4 : 0);
        int tv0[kSelfSpt];
#pragma unroll
        for (int j = 0; j < kSelfSpt; ++j) tv0[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(trs, (i0 + j) * 4, 0, 0);
        // this lane's lengths, kSelfSpt loads in flight at a time
        unsigned tlo = 0, thi = 0;  // sum of max(L, 1): low 20 bits and the rest, apart
        int lmax = 0, nb = 0;
#pragma unroll 1
        for (int ib = i0; ib < i1; ib += kSelfSpt) {
            int lv[kSelfSpt];
#pragma unroll
            for (int j = 0; j < kSelfSpt; ++j)
                lv[j] = ib == i0 ? lv0[j] : (int)__builtin_amdgcn_raw_buffer_load_b32(lrs, (ib + j) * 4, 0, 0);
#pragma unroll
            for (int j = 0; j < kSelfSpt; ++j) {
                const int i = ib + j;
                if (i < i1) {
                    const int L = max(lens ? lv[j] : (p.causal ? first + i + 1 : p.fixed_len), 0);
                    S.len[i] = L;
                    const unsigned w = (unsigned)max(L, 1);
                    tlo += w & 0xFFFFF;
                    thi += w >> 20;
                    lmax = max(lmax, L);
                    nb += (int)(((unsigned)L + B - 1) >> bsh);
                }
            }
        }
        // the chunk target: the host planner's (make_plan with target 0) ...
        const int slo = wave_incl_scan((int)tlo), shi = wave_incl_scan((int)thi);
        const int lall = __builtin_amdgcn_readlane(wave_incl_max(lmax), kWave - 1);
        nb = wave_incl_scan(nb) - nb;  // blocks of the sequences before this lane's (packed tables)
        const unsigned long long tokens =
            ((unsigned long long)(unsigned)__builtin_amdgcn_readlane(shi, kWave - 1) << 20) +
            (unsigned)__builtin_amdgcn_readlane(slo, kWave - 1);
        const int M = p.sp_max_chunk;  // a multiple of BLOCK; T never exceeds it
        const unsigned long long prod = tokens * (unsigned)hks;
        const unsigned long long pmax = (unsigned long long)(unsigned)p.sp_slots * (unsigned)M;
        long long c;  // ceil(tokens * hks / slots), capped at M (the same T follows)
        if (prod >= pmax) c = M;
        else if (pmax <= 0xFFFFFFFFull) c = ceil_div_u32((unsigned)prod, (unsigned)p.sp_slots);
        else c = ceil_div_u64((long long)prod, p.sp_slots);
        long long T = min(c, (long long)p.sp_target_cap);
        T = max(T, (long long)p.sp_min_chunk);
        T = (T + B - 1) >> bsh << bsh;
        T = min(T, (long long)M);
        // ... raised to the record budget (and the 64-chunk merge of the matrix-core
        // path): fit = ceil(tokens / ((sp_records - 1) * N)); past M only that matters
        const unsigned long long den = (unsigned long long)(unsigned)(p.sp_records - 1) * (unsigned)N;
        long long fit;
        if (tokens > den * (unsigned)M) fit = (long long)M + B;
        else if (tokens <= 0xFFFFFFFFull && den <= 0xFFFFFFFFull) fit = ceil_div_u32((unsigned)tokens, (unsigned)den);
        else fit = ceil_div_u64((long long)tokens, (long long)den);
        if (p.sp_nc_max) fit = max(fit, ((long long)lall + 62) / 63);
        fit = (fit + B - 1) >> bsh << bsh;
        const bool t_over = fit > M;
        if (fit > T) T = min(fit, (long long)M);
        const int Ti = uniform((int)T);
        const float kscale = 8.0f / (3.0f * (float)Ti);
        // this lane's sequences: chunks, and the buckets of their two runs
        int cnt[kSelfBuckets];
#pragma unroll
        for (int b = 0; b < kSelfBuckets; ++b) cnt[b] = 0;
        int nrec = 0, nctr = 0, over = 0;
#pragma unroll 2
        for (int i = i0; i < i1; ++i) {
            const int L = S.len[i];
            if (p.causal) {
                S.to[i] = 0;  // prompt queries: one shared table
            } else if (!p.tab_off) {
                S.to[i] = nb;  // packed tables in sequence order
                nb += (int)(((unsigned)L + B - 1) >> bsh);
            }
            if (P > 0 && L <= P) {  // attended while the plan is made: no units, no records
                over |= L > p.cap;
                S.cut[i] = 0;
                S.bk[i] = 0;
                continue;
            }
            int nc, chunk;
            self_split(p, L, Ti, bsh, nc, chunk);
            over |= nc > kSelfMaxChunks || L > p.cap;
            nc = min(nc, kSelfMaxChunks);
            const int ka = self_bucket(nc > 1, chunk, kscale);
            const int kb = self_bucket(nc > 1, nc > 1 ? L - (nc - 1) * chunk : L, kscale);
            S.cut[i] = nc | ((chunk >> bsh) << 16);
            S.bk[i] = ka | (kb << 4);
            const int ca = nc > 1 ? hks * (nc - 1) : 0;
#pragma unroll
            for (int b = 0; b < kSelfBuckets; ++b) cnt[b] += (b == ka ? ca : 0) + (b == kb ? hks : 0);
            nrec += nc > 1 ? nc : 0;
            nctr += nc > 1 ? 1 : 0;
        }
        if (offsets) {  // the table offsets, loaded at the start
#pragma unroll 1
            for (int ib = i0; ib < i1; ib += kSelfSpt) {
                int tv[kSelfSpt];
#pragma unroll
                for (int j = 0; j < kSelfSpt; ++j)
                    tv[j] = ib == i0 ? tv0[j] : (int)__builtin_amdgcn_raw_buffer_load_b32(trs, (ib + j) * 4, 0, 0);
#pragma unroll
                for (int j = 0; j < kSelfSpt; ++j)
                    if (ib + j < i1) S.to[ib + j] = tv[j];
            }
        }
        // the order: buckets descending, sequences ascending within a bucket (run A
        // before run B); first rank of this lane's units per bucket
        int excl[kSelfBuckets];
        int units = 0;
#pragma unroll
        for (int b = kSelfBuckets - 1; b >= 0; --b) {
            const int inc = wave_incl_scan(cnt[b]);
            excl[b] = units + inc - cnt[b];
            units += __builtin_amdgcn_readlane(inc, kWave - 1);
        }
        const int rec0 = wave_incl_scan(nrec) - nrec, ctrb = wave_incl_scan(nctr) - nctr;
        const bool overflow = t_over || __ballot(over) != 0;
        units = overflow ? N * hks : units;
        const int G = (int)gridDim.x;
        const int kcount = overflow ? 0 : min(kSelfWindow, (units + G - 1) / G - kw);
        if (lane == 0) {
            S.plan[0] = Ti;
            S.plan[1] = units;
            S.plan[2] = overflow ? 1 : 0;
        }
        // the headers of this workgroup's ranks in the window: the lane holding a rank
        // walks its sequences' runs in that bucket
#pragma unroll 1
        for (int k = 0; k < kcount; ++k) {
            const int r = self_plan_rank(kw + k);
            int bsel = -1, x = 0;
#pragma unroll
            for (int b = 0; b < kSelfBuckets; ++b) {
                const bool in = (unsigned)(r - excl[b]) < (unsigned)cnt[b];
                bsel = in ? b : bsel;
                x = in ? r - excl[b] : x;
            }
            if (bsel < 0) continue;
            int rec = rec0, ctr = ctrb;
#pragma unroll 1
            for (int i = i0; i < i1; ++i) {
                const int cut = S.cut[i], bk = S.bk[i];
                const int nc = cut & 0xFFFF, cblk = (unsigned)cut >> 16;
                const int ka = bk & 15, kb = bk >> 4;
                const int ca = ka == bsel && nc > 1 ? hks * (nc - 1) : 0;
                const int cb = kb == bsel && nc > 0 ? hks : 0;
                if (x < ca + cb) {
                    int h, cc;
                    if (x < ca) {  // run A: chunks 0..nc-2, every head of a chunk in turn
                        cc = x / hks;
                        h = x - cc * hks;
                    } else {       // run B: the last chunk of every head
                        h = x - ca;
                        cc = nc - 1;
                    }
                    const int L = S.len[i];
                    const int j0 = nc > 1 ? cc * cblk * B : 0;
                    int* e = S.hdr[k];
                    e[1] = h | (cc << 16);
                    e[2] = j0;
                    e[3] = nc > 1 ? min(j0 + cblk * B, L) : L;
                    e[4] = nc;
                    e[5] = nc > 1 ? hks * rec + h * nc : -1;
                    e[6] = nc > 1 ? hks * ctr + h : -1;
                    e[7] = S.to[i] + (nc > 1 ? cc * cblk : 0);
                    e[0] = i;
                    break;
                }
                x -= ca + cb;
                rec += nc > 1 ? nc : 0;
                ctr += nc > 1 ? 1 : 0;
            }
        }
    }
    __syncthreads();
    SelfPlan sp;
    sp.T = uniform(S.plan[0]);
    sp.units = uniform(S.plan[1]);
    sp.overflow = uniform(S.plan[2]);
    return sp;
}

// The unit of window slot k as a planned-entry header (read by every thread of the
// workgroup from LDS); false when this workgroup has no unit in that round.
template <typename Lds>
__device__ __forceinline__ bool self_plan_header(const Lds& S, int k, int (&hdr)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) hdr[e] = uniform(S.hdr[k][e]);
    return hdr[0] >= 0;
}

// A batch past the plan's budget: NaN in the output rows of every (sequence, KV
// head subgroup), rank r = s * hks + h, ranks served as in the planned loop.
template <typename E, int D, int NT>
__device__ void self_plan_nan(const DecodeParams& p, int heads) {
    report_device_error(p, kDevErrBudget);
    const int hks = p.Hkv * p.nsub;
    for (int k = 0, r = self_plan_rank(0); r < p.N * hks; r = self_plan_rank(++k)) {
        const int s = r / hks, h = r % hks;
        const int hq0 = (h / p.nsub) * p.group + (h % p.nsub) * heads;
        E* ob = static_cast<E*>(p.out) + ((size_t)s * p.Hq + hq0) * D;
        for (int e = threadIdx.x; e < heads * D; e += NT) ob[e] = (E)__builtin_nanf("");
    }
}

// While wave 0 plans, no K/V bytes move: wave 1 of every workgroup reads the first
// p.sp_pf_blocks blocks of every sequence (at most its first quarter) so that they
// are on their way from HBM into the memory-side cache while the plan is made, and
// the units that read them later find them there.  Item t = s + N * j is block j of
// sequence s; workgroup b takes items b, b + G, ..., one per lane.  Every block id is
// that of a block below the sequence's length, read from its table as the units read
// it; each pool block is touched once per 64 bytes by loads whose data land in an LDS
// sink (no registers held; wave 1's first wait for its own unit's loads also covers
// these, issued microseconds earlier).
//
// Targeted form (p.sp_pf_xcd, set when every unit covers one whole KV head and Hkv is
// a multiple of 8): the unit of KV head h at rank r < gridDim.x runs on XCD h mod 8
// (self_plan_setup's order), so the read-ahead of head h's slice of a block is made
// by a workgroup of that XCD (workgroup b sits on XCD b mod 8) and lands in the L2
// that the unit reads through: the unit finds the bytes there instead of requesting
// them again from the memory-side cache.  Item t = s + N * (j + pf * hh) is block j
// of sequence s, KV head x + 8 * hh of this workgroup's XCD x; workgroup 8 * q + x
// takes items q, q + Q, ... (Q = gridDim.x / 8 workgroups per XCD), one per lane.
template <typename E, int D, typename Lds>
__device__ __forceinline__ void self_prefetch(const int* lens, int N, const DecodeParams& p, Lds& S) {
    const int lane = threadIdx.x & (kWave - 1);
    if (p.sp_pf_xcd) {
        const unsigned Q = gridDim.x >> 3, xcd = blockIdx.x & 7u, q = blockIdx.x >> 3;
        const unsigned per_head = (unsigned)N * (unsigned)p.sp_pf_blocks;  // N <= kSelfMaxNValu, blocks <= 4096
        const unsigned items = per_head * (unsigned)(p.Hkv >> 3);
        const unsigned t = q + (unsigned)lane * Q;
        const bool has = q < Q && t < items;
        const unsigned hh = has ? t / per_head : 0, r = has ? t - hh * per_head : 0;
        const int s = (int)(r % (unsigned)N), j = (int)(r / (unsigned)N);
        const int h = (int)(xcd + 8 * hh);
        const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(lens, N * 4), ors = tile_rsrc(p.tab_off, N * 4);
        const int L = (int)__builtin_amdgcn_raw_buffer_load_b32(lrs, s * 4, 0, 0);
        const int to = (int)__builtin_amdgcn_raw_buffer_load_b32(ors, s * 4, 0, 0);
        const bool ok = has && L >= p.sp_pf_min_len && 4LL * j * p.block < (long long)L;
        const __amdgpu_buffer_rsrc_t tbr = tile_rsrc(p.table_all, p.table_len * 4);
        const int bid = ok ? (int)__builtin_amdgcn_raw_buffer_load_b32(tbr, (int)(((unsigned)to + (unsigned)j) * 4u), 0, 0) : -1;
        const int bytes = p.block * D * (int)sizeof(E);  // one block of one KV head, one pool
        unsigned long long live = __ballot(ok);
        auto* sink = (__attribute__((address_space(3))) void*)S.sink;
#pragma unroll 1
        while (live) {
            const int i = __builtin_ctzll(live);
            live &= live - 1;
            const size_t base = ((size_t)(unsigned)__builtin_amdgcn_readlane(bid, i) * (unsigned)p.Hkv +
                                 (unsigned)__builtin_amdgcn_readlane(h, i)) * (size_t)bytes;
            const __amdgpu_buffer_rsrc_t kr = tile_rsrc(static_cast<const char*>(p.k) + base, bytes);
            const __amdgpu_buffer_rsrc_t vr = tile_rsrc(static_cast<const char*>(p.v) + base, bytes);
#pragma unroll 1
            for (int x = lane * 64; x < bytes; x += kWave * 64) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, sink, 4, x, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, sink, 4, x, 0, 0, 0);
            }
        }
        return;
    }
    const unsigned items = (unsigned)N * (unsigned)p.sp_pf_blocks;  // N <= kSelfMaxNValu, blocks <= 4096
    const unsigned t = blockIdx.x + (unsigned)lane * gridDim.x;
    const bool has = t < items;
    const int s = has ? (int)(t % (unsigned)N) : 0, j = has ? (int)(t / (unsigned)N) : 0;
    const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(lens, N * 4), ors = tile_rsrc(p.tab_off, N * 4);
    const int L = (int)__builtin_amdgcn_raw_buffer_load_b32(lrs, s * 4, 0, 0);
    const int to = (int)__builtin_amdgcn_raw_buffer_load_b32(ors, s * 4, 0, 0);
    // at most the first quarter of a sequence, and none of a short one: short units
    // start streaming almost as soon as the plan is made, and reading them ahead as
    // well only doubles their requests
    const bool ok = has && L >= p.sp_pf_min_len && 4LL * j * p.block < (long long)L;
    // block id through a descriptor over the table (an offset past it reads 0), as the units read it
    const __amdgpu_buffer_rsrc_t tbr = tile_rsrc(p.table_all, p.table_len * 4);
    const int bid = ok ? (int)__builtin_amdgcn_raw_buffer_load_b32(tbr, (int)(((unsigned)to + (unsigned)j) * 4u), 0, 0) : -1;
    const int bytes = p.Hkv * p.block * D * (int)sizeof(E);  // one block of one pool, every KV head
    const unsigned long long live = __ballot(ok);
    auto* sink = (__attribute__((address_space(3))) void*)S.sink;
#pragma unroll 1
    for (int i = 0; i < kWave; ++i) {
        if (!((live >> i) & 1ull)) continue;
        const size_t base = (size_t)(unsigned)__builtin_amdgcn_readlane(bid, i) * (size_t)bytes;
        const __amdgpu_buffer_rsrc_t kr = tile_rsrc(static_cast<const char*>(p.k) + base, bytes);
        const __amdgpu_buffer_rsrc_t vr = tile_rsrc(static_cast<const char*>(p.v) + base, bytes);
#pragma unroll 1
        for (int x = lane * 64; x < bytes; x += kWave * 64) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, sink, 4, x, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, sink, 4, x, 0, 0, 0);
        }
    }
}

// The persistent loop of a self-planned launch: windows of kSelfWindow rounds, each
// planned by self_plan_setup, then its units (run(hdr)) in round order.  lens and
// n_seq (= p.N) are the kernel's register-preloaded first two arguments.  Each window
// reads its own copy of the parameter block (fresh_params): with the kernel argument
// itself, the compiler hoists the planner's parameter arithmetic in front of the
// loop -- ahead of the lengths loads, with its results spilled -- and keeps it live
// across every unit.
//
// Short sequences (Lds::kLead and p.sp_lead > 0): while wave 0 plans the first window,
// the other waves run lead() -- a sequence of at most p.sp_lead tokens whole, for this
// workgroup's (sequence, head subgroup), its partials left in LDS; false when there is
// none, and wave 1 then reads ahead -- and after the window's first unit (whose
// epilogue runs on wave 0 alone) wave 1 writes its output (lead_finish).
template <typename E, int D, int NT, typename Lds, typename Run, typename Lead, typename LeadFinish>
__device__ __forceinline__ void self_plan_loop(const int* lens, int n_seq, Lds& S, int heads, Run&& run, Lead&& lead,
                                               LeadFinish&& lead_finish) {
    const int G = (int)gridDim.x;
    // one window: plan it, run its units; false once every round is done
    auto window = [&](int kw, int (&lv)[kSelfSpt]) -> bool {
        const DecodeParams p = fresh_params();
        const bool leads = Lds::kLead && kw == 0 && p.sp_lead > 0;
        const int w = threadIdx.x >> 6;
        bool led = false;
        if (leads && w != 0) led = lead();
        if (kw == 0 && p.sp_pf_blocks > 0 && w == 1 && !led) self_prefetch<E, D>(lens, n_seq, p, S);
        const SelfPlan sp = self_plan_setup<NT>(lens, n_seq, p, S, kw, lv);
        if (sp.overflow) {
            self_plan_nan<E, D, NT>(p, heads);
            return false;
        }
        const int rounds = (sp.units + G - 1) / G;
        const int kend = min(rounds - kw, kSelfWindow);
        for (int k = 0; k < kend; ++k) {
            int hdr[8];
            if (self_plan_header(S, k, hdr)) run(hdr);
            if (leads && k == 0) lead_finish();
            // the unit's epilogue (one wave in the VALU kernel) still reads the other
            // waves' partials in LDS: no wave starts the next unit before it is done
            __syncthreads();
        }
        if (leads && kend <= 0) lead_finish();
        return kw + kSelfWindow < rounds;
    };
    // the first window's lengths load before anything else (the later windows' load
    // in their own iteration, so no lengths stay live across the units)
    int lv0[kSelfSpt] = {};
    if (threadIdx.x < kWave) self_first_lengths(lens, n_seq, lv0);
    __builtin_amdgcn_sched_barrier(0);
    if (!window(0, lv0)) return;
    for (int kw = kSelfWindow;; kw += kSelfWindow) {
        int lv[kSelfSpt] = {};
        if (threadIdx.x < kWave) self_first_lengths(lens, n_seq, lv);
        if (!window(kw, lv)) return;
    }
}

