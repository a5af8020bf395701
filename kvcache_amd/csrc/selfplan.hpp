// selfplan.hpp -- decode units planned by the kernel from lengths in device memory.
//
// Included by decode_kernels.hpp inside namespace kvc::{anonymous}; uses its helpers.
//
// The reference's launchers take the lengths as a device array
// (launch_batched_paged, batched.cu:140-147; qk_batched_paged_decode_attn,
// qwen_kernels.cu:293-326), so the host cannot plan the launch without a copy and
// a synchronisation.  Instead every workgroup of a persistent grid derives the
// host planner's work (kvc_decode_plan: the same chunk target, the same chunks,
// the same partial-record and counter numbering) from the lengths, orders the units
// as the planner does (up to rounding at bucket edges) -- chunks of split sequences
// first, then by length, longest first (64 length buckets relative to the chunk
// target) -- and serves ranks in
// rounds of gridDim.x (self_plan_rank).  Every workgroup computes the same order
// from the same data, so each unit runs exactly once.  Per workgroup: one round of
// loads (lengths, table offsets) into LDS, two reductions and a key histogram; per
// rank, one wave-wide scan over the sequences.  Outputs equal the host-planned
// launch's on the same lengths bit for bit (same chunks, same merge order); only the
// order in which units run differs within a length bucket.
//
// Budget: every (sequence, KV head) may use up to p.sp_records partial records (64,
// or more when the caller states a long bound), and on the matrix-core path a
// sequence has at most 64 chunks; the chunk target is raised when the lengths need
// it (mean length / (sp_records - 1), longest length / 63).  A batch that cannot fit
// even at the largest chunk, or with a length past its contiguous cache (p.cap),
// gets NaN outputs: never a silent partial attention.
//
// Cost structure: the lengths pointer arrives as the kernel's first (preloaded)
// argument, so their loads issue at wave start, beside the parameter block's; the
// setup then needs two barriers.  Finding a rank's unit is wave-local: every wave
// holds the key table in registers and scans the plan rows with lane shuffles, so
// the persistent loop has no barrier and no LDS broadcast between units.

constexpr int kSelfMaxNValu = 1024;    // sequences per launch (their plan rows live in LDS)
constexpr int kSelfMaxNMfma = 512;     // (keeps two matrix-core workgroups per CU)
constexpr int kSelfBuckets = 64;       // length buckets per split flag
constexpr int kSelfKeys = 2 * kSelfBuckets;
constexpr int kSelfMaxChunks = 0xFFFF;  // chunks of one sequence (16-bit plan field)
constexpr int kSelfSpt = 4;            // sequences per setup thread (kSelfMaxNValu / 256)

template <int NMAX, int NW>
struct SelfPlanLds {
    int len[NMAX];             // attended length of each sequence (>= 0)
    int to[NMAX];              // first table entry of each sequence
    int cut[NMAX];             // chunks | chunk length in blocks << 16
    int keys[NMAX];            // key of chunks 0..nc-2 | key of the last chunk << 8
    int hist[NW][kSelfKeys + 1];  // per-wave units per order key; [kSelfKeys]: sequences past the limits
    unsigned long long tot[NW];  // per-wave sums of max(L, 1)
    int lmax[NW];
    int nb[NW];                // per-wave blocks (packed tables)
};

// The plan as every wave holds it after self_plan_setup: the chunk target, the
// number of ranks and, per lane, the first rank and the unit count of keys
// kSelfKeys-1-2*lane (a) and kSelfKeys-2-2*lane (b); ranks run over the keys in
// descending order.
struct SelfPlan {
    int T, units, overflow;
    int base_a, cnt_a, base_b, cnt_b;
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

// ceil(a / b) for 0 <= a < 2^53, 0 < b < 2^31 (uniform operands: a double quotient
// corrected to the exact integer, instead of a 64-bit integer division)
__device__ __forceinline__ long long ceil_div_u(long long a, long long b) {
    long long q = (long long)((double)a / (double)b);
    while (q * b < a) ++q;
    while (q > 0 && (q - 1) * b >= a) --q;
    return q;
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

// Order key of a unit of `len` tokens: split units above whole ones, longer above
// shorter; kscale = 42 / T.  The planner's bucket len * 42 / T, in float: the key
// only orders the units (their chunks, records and counters do not depend on it),
// so a unit at a bucket edge may sort one bucket away from the host plan's order.
__device__ __forceinline__ int self_key(bool split, int len, float kscale) {
    const int b = min(kSelfBuckets - 1, (int)((float)len * kscale));
    return (split ? kSelfBuckets : 0) + b;
}

// Units of a sequence in key `key`: run A = chunks 0..nc-2 of every head (nc > 1),
// run B = the last chunk of every head.
__device__ __forceinline__ void self_runs(int nc, int keys, int key, int hks, int& ca, int& cb) {
    ca = nc > 1 && (keys & 0xFF) == key ? hks * (nc - 1) : 0;
    cb = (keys >> 8) == key ? hks : 0;
}

// Reads the lengths (`lens`, device memory; NULL: causal prompt queries) and table
// offsets, picks the chunk target, cuts every sequence into chunks and counts the
// units per order key.  Every thread of the workgroup calls it; every wave returns
// the same plan.
template <int NT, typename Lds>
__device__ SelfPlan self_plan_setup(const int* lens, const DecodeParams& p, Lds& S) {
    constexpr int NW = NT / kWave;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
    const int N = p.N, B = p.block, hks = p.Hkv * p.nsub;
    const int bsh = __builtin_ctz((unsigned)B);
    const int spt = (N + NT - 1) / NT;  // consecutive sequences per thread
    const int i0 = min(tid * spt, N), i1 = min(i0 + spt, N);
    const int first = p.dev_base ? *p.dev_base : p.fixed_len;  // causal prompt queries
    int* hist = S.hist[wave];
    for (int k = lane; k <= kSelfKeys; k += kWave) hist[k] = 0;
    // the thread's lengths and table offsets, all loads issued before any is used
    // (bounded buffer loads: indices past N read 0 and touch no memory)
    static_assert(NT >= 256, "at most kSelfSpt sequences per thread");
    const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(lens, lens ? N * 4 : 0);
    const __amdgpu_buffer_rsrc_t trs = tile_rsrc(p.tab_off, p.tab_off ? N * 4 : 0);
    int lv[kSelfSpt], tv[kSelfSpt];
#pragma unroll
    for (int j = 0; j < kSelfSpt; ++j) {
        lv[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(lrs, (i0 + j) * 4, 0, 0);
        tv[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(trs, (i0 + j) * 4, 0, 0);
    }
    unsigned long long tot = 0;  // at most 4 sequences per thread: < 2^33
    int lmax = 0, nb = 0;
#pragma unroll
    for (int j = 0; j < kSelfSpt; ++j) {
        const int i = i0 + j;
        if (i < i1) {
            const int L = max(lens ? lv[j] : (p.causal ? first + i + 1 : p.fixed_len), 0);
            S.len[i] = L;
            S.to[i] = tv[j];
            tot += (unsigned)max(L, 1);
            lmax = max(lmax, L);
            nb += (int)(((unsigned)L + B - 1) >> bsh);
        }
    }
    // wave totals: the 64-bit sum as two 32-bit scans of its low 20 and high bits
    const int tlo = wave_incl_scan((int)(tot & 0xFFFFF)), thi = wave_incl_scan((int)(tot >> 20));
    const int lmx = wave_incl_max(lmax);
    const int nb_incl = wave_incl_scan(nb);
    if (lane == kWave - 1) {
        S.tot[wave] = ((unsigned long long)(unsigned)thi << 20) + (unsigned)tlo;
        S.lmax[wave] = lmx;
        S.nb[wave] = nb_incl;
    }
    __syncthreads();
    unsigned long long tall = 0;
    int lall = 0, nb_pre = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        tall += S.tot[w];
        lall = max(lall, S.lmax[w]);
        nb_pre += w < wave ? S.nb[w] : 0;
    }
    // chunk target: the host planner's (make_plan, target 0) ...
    const long long tokens = (long long)tall;
    long long target = ceil_div_u(tokens * hks, p.sp_slots);
    target = min(target, (long long)p.sp_target_cap);
    target = min(target, (long long)(INT_MAX / 2));
    long long T = max(target, (long long)p.sp_min_chunk);
    T = (T + B - 1) >> bsh << bsh;
    T = min(T, (long long)p.sp_max_chunk);
    // ... raised to the record budget (and the 64-chunk merge of the matrix-core path)
    long long fit = ceil_div_u(tokens, (long long)(p.sp_records - 1) * N);
    if (p.sp_nc_max) fit = max(fit, ((long long)lall + 62) / 63);
    fit = (fit + B - 1) >> bsh << bsh;
    const bool overflow = fit > p.sp_max_chunk;
    if (fit > T) T = min(fit, (long long)p.sp_max_chunk);
    const int Ti = uniform((int)T);
    const float kscale = 42.0f / (float)Ti;
    int run = nb_pre + nb_incl - nb;  // packed tables: first entry of sequence i0
    int over = 0;
    for (int i = i0; i < i1; ++i) {
        const int L = S.len[i];
        if (p.causal) {
            S.to[i] = 0;  // prompt queries: one shared table
        } else if (!p.tab_off) {
            S.to[i] = run;
            run += (int)(((unsigned)L + B - 1) >> bsh);
        }
        int nc, chunk;
        self_split(p, L, Ti, bsh, nc, chunk);
        over += nc > kSelfMaxChunks || L > p.cap ? 1 : 0;
        const int ka = self_key(nc > 1, chunk, kscale);
        const int kb = self_key(nc > 1, nc > 1 ? L - (nc - 1) * chunk : L, kscale);
        S.cut[i] = min(nc, kSelfMaxChunks) | ((chunk >> bsh) << 16);
        S.keys[i] = ka | (kb << 8);
        if (nc > 1) atomicAdd(&hist[ka], hks * (nc - 1));
        atomicAdd(&hist[kb], hks);
    }
    if (over) atomicAdd(&hist[kSelfKeys], over);
    __syncthreads();
    // every wave adds the per-wave histograms and scans the keys in descending order
    const int ka = kSelfKeys - 1 - 2 * lane, kb = ka - 1;
    int ca = 0, cb = 0, ov = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        ca += S.hist[w][ka];
        cb += S.hist[w][kb];
        ov += S.hist[w][kSelfKeys];
    }
    const int incl = wave_incl_scan(ca + cb);
    SelfPlan sp;
    sp.T = Ti;
    sp.overflow = overflow || uniform(ov) > 0;
    sp.units = sp.overflow ? N * hks : __builtin_amdgcn_readlane(incl, kWave - 1);
    sp.base_a = incl - ca - cb;
    sp.cnt_a = ca;
    sp.base_b = incl - cb;
    sp.cnt_b = cb;
    return sp;
}

// The unit of rank r (r < sp.units) as a planned-entry header.  Every thread of the
// workgroup calls it with the same r; each wave finds the unit on its own (lane
// shuffles over the plan rows, no barrier).  Returns false (after writing NaN to the
// unit's output rows) when the batch overflowed the plan's budget.
template <typename E, int D, int NT, typename Lds>
__device__ bool self_plan_unit(const DecodeParams& p, const Lds& S, const SelfPlan& sp, int r, int heads,
                               int (&hdr)[8]) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int N = p.N, hks = p.Hkv * p.nsub;
    if (sp.overflow) {
        const int s = r / hks, h = r % hks;
        const int hq0 = (h / p.nsub) * p.group + (h % p.nsub) * heads;
        E* ob = static_cast<E*>(p.out) + ((size_t)s * p.Hq + hq0) * D;
        for (int e = tid; e < heads * D; e += NT) ob[e] = (E)__builtin_nanf("");
        return false;
    }
    // the key holding rank r
    const unsigned long long ma = __ballot(r >= sp.base_a && r < sp.base_a + sp.cnt_a);
    const unsigned long long mb = __ballot(r >= sp.base_b && r < sp.base_b + sp.cnt_b);
    if (!ma && !mb) return false;
    int key, q;
    if (ma) {
        const int l = __ffsll((long long)ma) - 1;
        key = kSelfKeys - 1 - 2 * l;
        q = r - __builtin_amdgcn_readlane(sp.base_a, l);
    } else {
        const int l = __ffsll((long long)mb) - 1;
        key = kSelfKeys - 2 - 2 * l;
        q = r - __builtin_amdgcn_readlane(sp.base_b, l);
    }
    // this lane's sequences, in order: units in `key`, records, counters
    const int spl = (N + kWave - 1) / kWave;
    const int i0 = min(lane * spl, N), i1 = min(i0 + spl, N);
    int own = 0, nrec = 0, nctr = 0;
    for (int i = i0; i < i1; ++i) {
        const int nc = S.cut[i] & 0xFFFF;
        int ca, cb;
        self_runs(nc, S.keys[i], key, hks, ca, cb);
        own += ca + cb;
        nrec += nc > 1 ? nc : 0;
        nctr += nc > 1 ? 1 : 0;
    }
    int base = wave_incl_scan(own) - own;
    int rec = wave_incl_scan(nrec) - nrec;
    int ctr = wave_incl_scan(nctr) - nctr;
    const bool mine = q >= base && q < base + own;  // exactly one lane
    int h0 = 0, h1 = 0, h2 = 0, h3 = 0, h4 = 0, h5 = 0, h6 = 0, h7 = 0;
    if (mine) {
        for (int i = i0; i < i1; ++i) {
            const int nc = S.cut[i] & 0xFFFF;
            int ca, cb;
            self_runs(nc, S.keys[i], key, hks, ca, cb);
            if (q < base + ca + cb) {
                const int x = q - base;
                int h, c;
                if (x < ca) {
                    h = x / (nc - 1);
                    c = x - h * (nc - 1);
                } else {
                    h = x - ca;
                    c = nc - 1;
                }
                const int L = S.len[i];
                const int cblk = S.cut[i] >> 16;
                const int j0 = c * cblk * p.block;
                h0 = i;
                h1 = h | (c << 16);
                h2 = nc > 1 ? j0 : 0;
                h3 = nc > 1 ? min(j0 + cblk * p.block, L) : L;
                h4 = nc;
                h5 = nc > 1 ? hks * rec + h * nc : -1;
                h6 = nc > 1 ? hks * ctr + h : -1;
                h7 = S.to[i] + (nc > 1 ? c * cblk : 0);
                break;
            }
            base += ca + cb;
            rec += nc > 1 ? nc : 0;
            ctr += nc > 1 ? 1 : 0;
        }
    }
    const unsigned long long mm = __ballot(mine);
    if (!mm) return false;
    const int src = __ffsll((long long)mm) - 1;
    hdr[0] = __builtin_amdgcn_readlane(h0, src);
    hdr[1] = __builtin_amdgcn_readlane(h1, src);
    hdr[2] = __builtin_amdgcn_readlane(h2, src);
    hdr[3] = __builtin_amdgcn_readlane(h3, src);
    hdr[4] = __builtin_amdgcn_readlane(h4, src);
    hdr[5] = __builtin_amdgcn_readlane(h5, src);
    hdr[6] = __builtin_amdgcn_readlane(h6, src);
    hdr[7] = __builtin_amdgcn_readlane(h7, src);
    return true;
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
