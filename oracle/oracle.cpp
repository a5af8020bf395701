// oracle.cpp -- CPU restatement of the kimxinw/kvcache decode hot path.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product (kvcache_amd/, include/) may
// link, load or call this file; it is imported by tests/, by the smoke() check in
// __graft_entry__.py and by the cpu_baseline leg of bench.py, always as the
// checker and never as the thing measured or shipped.
//
// Everything here is a restatement (own code) of the reference's algorithm, with
// the reference file:line it follows cited on each function:
//   * attention in double accumulation: two-pass (batched.cu:97-130,49-88),
//     online split-K + LSE merge (flash_decode.cu:18-101), GQA head map
//     (qwen_kernels.cu:299);
//   * block free-list, KV block accounting, continuous Engine policy, static
//     baseline (block_alloc.h:10-43, kv_cache_manager.h:56-91, engine.h:47-140,
//     scheduler.h:33-89) with the per-step packing of model_runner.h:61-69;
//   * the two workload generators whose outputs the reference's README pins
//     (bench_throughput.cu:50-57 lengths, bench_continuous.cu:38-50 trace).  The
//     other harness generators (hval, the fill and shuffle of bench_paged.cu /
//     main_paged.cu, the demo trace) are plain input generators in
//     kvcache_amd/workloads.py: no parity check depends on their values (hval and
//     the shuffle are still compared with the reference's own code, compiled by
//     oracle/Makefile into _ref/ref_gen_driver).
//
// Pinning (what checks each function independently of this text) is listed in
// tests/test_oracle_*.py; the header comment of every exported function names
// the reference lines it restates.
//
// Build: oracle/Makefile (g++ -O2 -shared -fPIC), output oracle/_build/liboracle.so.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <thread>
#include <vector>

#define ORC_API extern "C" __attribute__((visibility("default")))

// ---------------------------------------------------------------------------
// element loads: dtype 0 = float32, 1 = IEEE binary16 (decoded exactly)
// ---------------------------------------------------------------------------
static inline double half_bits_to_double(uint16_t h) {
    int sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    double v;
    if (exp == 0)       v = std::ldexp((double)man, -24);             // subnormal / zero
    else if (exp == 31) v = man ? NAN : INFINITY;
    else                v = std::ldexp((double)(man | 0x400), exp - 25);
    return sign ? -v : v;
}
struct HalfTable {
    double v[65536];
    HalfTable() { for (int i = 0; i < 65536; ++i) v[i] = half_bits_to_double((uint16_t)i); }
};
static const HalfTable g_half;
static inline double ld(const void* p, size_t i, int dtype) {
    return dtype == 1 ? g_half.v[((const uint16_t*)p)[i]] : (double)((const float*)p)[i];
}

// ---------------------------------------------------------------------------
// Attention, two-pass softmax in double.
// Restates batched.cu:97-130 (batched_paged: scores over [0,L), max, exp-sum,
// normalise, PV) with the paged offset of batched.cu:91-95
// ((phys*H + h)*BLOCK + pos%BLOCK)*D, and the GQA map kv_head = h / (Hq/Hkv)
// of qwen_kernels.cu:299.  L = 0 gives 0 (qwen_kernels.cu:326 convention).
// ---------------------------------------------------------------------------
struct AttnJob {
    const void* q; const void* k; const void* v; double* out;
    const int* table_all; const int* tab_off; const int* cur_len;
    int N, Hq, Hkv, D, BLOCK; long long MAXS; double scale; int dtype; int paged;
};

static void attn_one(const AttnJob& J, int s, int h, std::vector<double>& score) {
    const int L = J.cur_len[s];
    const int g = J.Hq / J.Hkv;
    const int hk = h / g;                                   // qwen_kernels.cu:299
    double* o = J.out + ((size_t)s * J.Hq + h) * J.D;
    for (int d = 0; d < J.D; ++d) o[d] = 0.0;
    if (L <= 0) return;
    score.resize(L);
    auto row = [&](int pos) -> size_t {                     // element offset of token pos
        if (J.paged) {
            int phys = J.table_all[J.tab_off[s] + pos / J.BLOCK];
            return (((size_t)phys * J.Hkv + hk) * J.BLOCK + pos % J.BLOCK) * J.D;
        }
        return (((size_t)s * J.Hkv + hk) * J.MAXS + pos) * J.D;
    };
    const size_t qo = ((size_t)s * J.Hq + h) * J.D;
    double m = -INFINITY;
    for (int pos = 0; pos < L; ++pos) {
        size_t r = row(pos);
        double acc = 0.0;
        for (int d = 0; d < J.D; ++d) acc += ld(J.q, qo + d, J.dtype) * ld(J.k, r + d, J.dtype);
        score[pos] = acc * J.scale;
        m = std::max(m, score[pos]);
    }
    double sum = 0.0;
    for (int pos = 0; pos < L; ++pos) { score[pos] = std::exp(score[pos] - m); sum += score[pos]; }
    for (int pos = 0; pos < L; ++pos) {
        size_t r = row(pos);
        double p = score[pos] / sum;
        for (int d = 0; d < J.D; ++d) o[d] += p * ld(J.v, r + d, J.dtype);
    }
}

static void attn_run(const AttnJob& J, int nthreads) {
    const int total = J.N * J.Hq;
    if (nthreads <= 1) {
        std::vector<double> sc;
        for (int i = 0; i < total; ++i) attn_one(J, i / J.Hq, i % J.Hq, sc);
        return;
    }
    std::vector<std::thread> th;
    for (int t = 0; t < nthreads; ++t)
        th.emplace_back([&, t] {
            std::vector<double> sc;
            for (int i = t; i < total; i += nthreads) attn_one(J, i / J.Hq, i % J.Hq, sc);
        });
    for (auto& x : th) x.join();
}

// Batched paged GQA decode: q[N,Hq,D], pools [NB,Hkv,BLOCK,D], out[N,Hq,D] (double).
// Restates batched.cu:97-130 + qwen_kernels.cu:293-327.
ORC_API void orc_batched_paged(const void* q, const void* k_pool, const void* v_pool,
                               const int* table_all, const int* tab_off, const int* cur_len,
                               double* out, int N, int Hq, int Hkv, int D, int BLOCK,
                               double scale, int dtype, int nthreads) {
    AttnJob J{q, k_pool, v_pool, out, table_all, tab_off, cur_len, N, Hq, Hkv, D, BLOCK, 0, scale, dtype, 1};
    attn_run(J, nthreads);
}

// Batched contiguous GQA decode: caches [N,Hkv,MAXS,D].  Restates batched.cu:49-88.
ORC_API void orc_batched_contig(const void* q, const void* k, const void* v, const int* cur_len,
                                double* out, int N, int Hq, int Hkv, int D, long long MAXS,
                                double scale, int dtype, int nthreads) {
    AttnJob J{q, k, v, out, nullptr, nullptr, cur_len, N, Hq, Hkv, D, 0, MAXS, scale, dtype, 0};
    attn_run(J, nthreads);
}

// ---------------------------------------------------------------------------
// Split-K flash decode on a contiguous single sequence [H,S,D].
// Restates flash_decode.cu:18-78 (chunk = ceil(L/ns), split j covers
// [j*chunk, min(j*chunk+chunk, L)), online running max/sum, empty split leaves
// m = -FLT_MAX, l = 0, acc = 0) and flash_decode.cu:82-101 (LSE merge
// M = max m_s; out = sum e^{m_s-M} acc_s / sum e^{m_s-M} l_s), with the clamp
// 1 <= ns <= L of flash_decode.cu:106-107.  Arithmetic in double.
// part_acc [H,ns,D], part_m/part_l [H,ns].
// ---------------------------------------------------------------------------
ORC_API void orc_flash_split(const void* q, const void* k, const void* v,
                             double* part_acc, double* part_m, double* part_l,
                             int H, int D, long long S, int cur_len, double scale,
                             int num_splits, int dtype) {
    const int chunk = (cur_len + num_splits - 1) / num_splits;
    for (int h = 0; h < H; ++h)
        for (int sp = 0; sp < num_splits; ++sp) {
            const int j0 = sp * chunk, j1 = std::min(j0 + chunk, cur_len);
            double m = -DBL_MAX, l = 0.0;
            std::vector<double> acc(D, 0.0);
            for (int j = j0; j < j1; ++j) {
                const size_t r = ((size_t)h * S + j) * D;
                double sc = 0.0;
                for (int d = 0; d < D; ++d) sc += ld(q, (size_t)h * D + d, dtype) * ld(k, r + d, dtype);
                sc *= scale;
                const double mn = std::max(m, sc);
                const double corr = std::exp(m - mn), p = std::exp(sc - mn);
                l = l * corr + p;
                for (int d = 0; d < D; ++d) acc[d] = acc[d] * corr + p * ld(v, r + d, dtype);
                m = mn;
            }
            const size_t b = (size_t)h * num_splits + sp;
            for (int d = 0; d < D; ++d) part_acc[b * D + d] = acc[d];
            part_m[b] = m; part_l[b] = l;
        }
}

ORC_API void orc_flash_merge(const double* part_acc, const double* part_m, const double* part_l,
                             double* out, int H, int D, int num_splits) {
    for (int h = 0; h < H; ++h) {
        double M = -DBL_MAX;
        for (int s = 0; s < num_splits; ++s) M = std::max(M, part_m[(size_t)h * num_splits + s]);
        double l = 0.0;
        std::vector<double> acc(D, 0.0);
        for (int s = 0; s < num_splits; ++s) {
            const size_t b = (size_t)h * num_splits + s;
            const double w = std::exp(part_m[b] - M);
            l += w * part_l[b];
            for (int d = 0; d < D; ++d) acc[d] += w * part_acc[b * D + d];
        }
        for (int d = 0; d < D; ++d) out[(size_t)h * D + d] = l > 0.0 ? acc[d] / l : 0.0;
    }
}

// launch_flash_decode (flash_decode.cu:103-126): clamp, split, merge.
ORC_API void orc_flash_decode(const void* q, const void* k, const void* v, double* out,
                              int cur_len, int H, int D, long long S, double scale,
                              int num_splits, int dtype) {
    if (num_splits < 1) num_splits = 1;
    if (num_splits > cur_len) num_splits = cur_len;
    if (num_splits < 1) { for (int i = 0; i < H * D; ++i) out[i] = 0.0; return; }
    std::vector<double> pa((size_t)H * num_splits * D), pm((size_t)H * num_splits), pl((size_t)H * num_splits);
    orc_flash_split(q, k, v, pa.data(), pm.data(), pl.data(), H, D, S, cur_len, scale, num_splits, dtype);
    orc_flash_merge(pa.data(), pm.data(), pl.data(), out, H, D, num_splits);
}

// ---------------------------------------------------------------------------
// Workload generators (uint32 LCG s = s*1103515245 + 12345; r = (s>>9)/2^23).
// ---------------------------------------------------------------------------
static inline float lcg01(unsigned& seed) {
    seed = seed * 1103515245u + 12345u;
    return (seed >> 9) / 8388608.0f;
}

// bench_throughput.cu:50-57: L = 16 + (int)((LMAX-16)*r*r), seed 12345 by default.
ORC_API void orc_ref_lengths(int N, int LMAX, unsigned seed, int* out) {
    for (int s = 0; s < N; ++s) {
        float r = lcg01(seed);
        out[s] = 16 + (int)((LMAX - 16) * r * r);
    }
}

// bench_continuous.cu:38-50: per request draw rp, rg, then (only if rate>0) u.
ORC_API void orc_ref_trace(int nreq, int prompt_max, int gen_max, double rate, unsigned seed,
                           int* prompt, int* gen, double* arrival_us) {
    double t_arr = 0.0;
    for (int i = 0; i < nreq; ++i) {
        float rp = lcg01(seed), rg = lcg01(seed);
        prompt[i] = 16 + (int)((prompt_max - 16) * rp * rp);
        gen[i] = 8 + (int)((gen_max - 8) * rg * rg);
        if (rate > 0) {
            double u = lcg01(seed);
            if (u < 1e-9) u = 1e-9;
            t_arr += -std::log(u) / rate * 1e6;
        }
        arrival_us[i] = rate > 0 ? t_arr : 0.0;
    }
}

// ---------------------------------------------------------------------------
// Block free-list (block_alloc.h:10-43): LIFO stack initialised n-1..0 so fresh
// allocations return 0,1,2,...; free pushes a table back in table order;
// alloc on an empty list returns -1; reset restores the initial stack.
// ---------------------------------------------------------------------------
struct OAlloc {
    int total;
    std::vector<int> st;
    explicit OAlloc(int n) : total(n) { reset(); }
    void reset() { st.clear(); for (int i = total - 1; i >= 0; --i) st.push_back(i); }
    int alloc() { if (st.empty()) return -1; int b = st.back(); st.pop_back(); return b; }
    void free_blocks(const std::vector<int>& t) { for (int b : t) st.push_back(b); }
    int free_count() const { return (int)st.size(); }
    int used_count() const { return total - (int)st.size(); }
};
static inline int blocks_needed(int len, int block) { return (len + block - 1) / block; }

struct OSeq {
    int id = -1, prompt_len = 0, cur_len = 0, max_new = 0;
    double arrival_us = 0;
    std::vector<int> table;
    int status = 0;  // 0 waiting, 1 running, 2 finished
    bool done() const { return cur_len - prompt_len >= max_new; }
};

// KV block accounting (kv_cache_manager.h:56-91).
struct OKvm {
    int num_blocks, block_size, n_kv_heads, head_dim;
    OAlloc a;
    OKvm(int nb, int bs, int hkv, int d) : num_blocks(nb), block_size(bs), n_kv_heads(hkv), head_dim(d), a(nb) {}
    int slack(const OSeq& s) const { return (int)s.table.size() * block_size - s.cur_len; }
    bool allocate_prompt(OSeq& s) {                 // all-or-nothing
        int need = blocks_needed(s.prompt_len, block_size);
        if (a.free_count() < need) return false;
        for (int i = 0; i < need; ++i) s.table.push_back(a.alloc());
        s.cur_len = s.prompt_len;
        return true;
    }
    bool append_token(OSeq& s) {                    // grow on a boundary; no advance on OOM
        if (blocks_needed(s.cur_len + 1, block_size) > (int)s.table.size()) {
            int b = a.alloc();
            if (b < 0) return false;
            s.table.push_back(b);
        }
        s.cur_len++;
        return true;
    }
    void free(OSeq& s) { a.free_blocks(s.table); s.table.clear(); }
    size_t slot_offset(int phys, int h, int in) const {
        return (((size_t)phys * n_kv_heads + h) * block_size + in) * head_dim;
    }
};

// ---- small handle API over the accounting restatement (for known-answer tests) ----
struct OKvmHandle { OKvm kvm; std::map<int, OSeq> seqs; };
ORC_API void* orc_kvm_new(int nb, int bs, int hkv, int d) { return new OKvmHandle{OKvm(nb, bs, hkv, d), {}}; }
ORC_API void orc_kvm_delete(void* h) { delete (OKvmHandle*)h; }
ORC_API int orc_kvm_free_blocks(void* h) { return ((OKvmHandle*)h)->kvm.a.free_count(); }
ORC_API int orc_kvm_allocate_prompt(void* h, int id, int prompt_len) {
    auto* H = (OKvmHandle*)h; OSeq& s = H->seqs[id]; s.id = id; s.prompt_len = prompt_len;
    return H->kvm.allocate_prompt(s) ? 1 : 0;
}
ORC_API int orc_kvm_append_token(void* h, int id) { auto* H = (OKvmHandle*)h; return H->kvm.append_token(H->seqs[id]) ? 1 : 0; }
ORC_API void orc_kvm_free(void* h, int id) { auto* H = (OKvmHandle*)h; H->kvm.free(H->seqs[id]); }
ORC_API int orc_kvm_slack(void* h, int id) { auto* H = (OKvmHandle*)h; return H->kvm.slack(H->seqs[id]); }
ORC_API int orc_kvm_cur_len(void* h, int id) { return ((OKvmHandle*)h)->seqs[id].cur_len; }
ORC_API int orc_kvm_table(void* h, int id, int* out, int cap) {
    auto& t = ((OKvmHandle*)h)->seqs[id].table;
    for (int i = 0; i < (int)t.size() && i < cap; ++i) out[i] = t[i];
    return (int)t.size();
}
ORC_API long long orc_kvm_slot_offset(void* h, int phys, int kvh, int in) {
    return (long long)((OKvmHandle*)h)->kvm.slot_offset(phys, kvh, in);
}

// Scripted allocator run: ops[i] >= 0 -> alloc() (result to out), ops[i] = -1 ->
// free the first `arg` blocks still held (in allocation order), -2 -> reset.
ORC_API void orc_alloc_script(int total, const int* ops, const int* args, int nops, int* out) {
    OAlloc a(total);
    std::vector<int> held;
    for (int i = 0; i < nops; ++i) {
        if (ops[i] == 0) { int b = a.alloc(); out[i] = b; if (b >= 0) held.push_back(b); }
        else if (ops[i] == -1) {
            int n = std::min(args[i], (int)held.size());
            std::vector<int> fr(held.begin(), held.begin() + n);
            held.erase(held.begin(), held.begin() + n);
            a.free_blocks(fr); out[i] = a.free_count();
        } else { a.reset(); held.clear(); out[i] = a.free_count(); }
    }
}

// ---------------------------------------------------------------------------
// Scheduling policies with a deterministic virtual clock.
//   step cost (us) = c0 + c1 * N + c2 * sum(len) for the packed batch.
// The per-step packed metadata follows model_runner.h:61-69 (concatenated
// block tables, offsets, lengths clamped to >= 1).  With kv_write = 1 the step
// follows qwen_serve.cu:130-141 instead: each running sequence first grows its
// table for position cur_len, writes there (wpos), and attends over cur_len+1.
// Every step folds (N, tab_off[0..N], len[0..N), wpos[0..N) if kv_write,
// table_all) into an FNV-1a 64-bit digest over little-endian int32 words.
// ---------------------------------------------------------------------------
struct OStats {
    int iters; long long tokens; double gpu_us; double wall_us; long long slot_steps;
    long long useful_steps; int peak_blocks; int finished; double avg_latency_us;
    double p50_latency_us; double p99_latency_us; unsigned long long digest;
};

struct Digest {
    uint64_t h = 1469598103934665603ull;
    void word(int32_t x) {
        uint32_t u = (uint32_t)x;
        for (int i = 0; i < 4; ++i) { h ^= (u >> (8 * i)) & 0xffu; h *= 1099511628211ull; }
    }
};

struct Packer {
    std::vector<int> tab, off, len, wpos;
    double c0, c1, c2;
    Digest* dg;
    // pack the batch exactly as the runner would upload it; returns virtual step cost
    double pack(const std::vector<OSeq*>& b, bool kv_write, const std::vector<int>* wp) {
        tab.clear(); off.clear(); len.clear();
        long long sum_len = 0;
        for (OSeq* s : b) {
            off.push_back((int)tab.size());
            for (int x : s->table) tab.push_back(x);
            int L = s->cur_len > 0 ? s->cur_len : 1;
            len.push_back(L); sum_len += L;
        }
        off.push_back((int)tab.size());
        dg->word((int)b.size());
        for (int x : off) dg->word(x);
        for (int x : len) dg->word(x);
        if (kv_write) for (int x : *wp) dg->word(x);
        for (int x : tab) dg->word(x);
        return c0 + c1 * (double)b.size() + c2 * (double)sum_len;
    }
};

static void fill_latency(OStats& R, std::vector<double>& lat) {    // engine.h:48-54 (+ p50)
    if (lat.empty()) { R.avg_latency_us = R.p50_latency_us = R.p99_latency_us = 0; return; }
    std::sort(lat.begin(), lat.end());
    double s = 0; for (double x : lat) s += x;
    R.avg_latency_us = s / lat.size();
    R.p50_latency_us = lat[std::min((size_t)(lat.size() * 0.5), lat.size() - 1)];
    R.p99_latency_us = lat[std::min((size_t)(lat.size() * 0.99), lat.size() - 1)];
}

// Continuous batching (engine.h:77-148).  Returns 0, or 1 if it stopped because
// no request could ever be admitted (the reference would spin forever there).
ORC_API int orc_sim_engine(const int* prompt, const int* gen, const double* arrival, int n,
                           int block_size, int num_blocks, int max_batch, int kv_write,
                           double c0, double c1, double c2, OStats* out) {
    OKvm kvm(num_blocks, block_size, 1, 1);
    std::deque<OSeq> store; std::deque<OSeq*> waiting; std::vector<OSeq*> running;
    std::vector<double> lat; int reserved = 0; double clock = 0;
    OStats R{}; Digest dg; Packer pk{{}, {}, {}, {}, c0, c1, c2, &dg};
    auto worst = [&](const OSeq& s) { return blocks_needed(s.prompt_len + s.max_new, block_size); };
    for (int i = 0; i < n; ++i) {
        store.push_back(OSeq{}); OSeq& s = store.back();
        s.id = i; s.prompt_len = prompt[i]; s.max_new = gen[i]; s.arrival_us = arrival[i];
        waiting.push_back(&s);
    }
    int rc = 0;
    for (;;) {
        for (size_t i = 0; i < running.size();) {                       // 1) retire
            OSeq* s = running[i];
            if (s->done()) {
                kvm.free(*s); reserved -= worst(*s);
                lat.push_back(clock - s->arrival_us); s->status = 2; R.finished++;
                running[i] = running.back(); running.pop_back();
            } else ++i;
        }
        while ((int)running.size() < max_batch && !waiting.empty() &&   // 2) admit FIFO
               waiting.front()->arrival_us <= clock) {
            OSeq* s = waiting.front();
            int fp = worst(*s);
            if (reserved + fp > num_blocks) break;
            if (!kvm.allocate_prompt(*s)) break;
            reserved += fp; s->status = 1; running.push_back(s); waiting.pop_front();
        }
        if (running.empty()) {                                          // 3) idle / done
            if (waiting.empty()) break;
            if (waiting.front()->arrival_us <= clock) { rc = 1; break; } // can never fit
            clock = std::max(clock, waiting.front()->arrival_us);
            continue;
        }
        double us;
        if (kv_write) {                                                 // qwen_serve.cu:130-141
            std::vector<int> wp;
            for (OSeq* s : running) { int pos = s->cur_len; kvm.append_token(*s); wp.push_back(pos); }
            us = pk.pack(running, true, &wp);
            R.tokens += (long long)running.size();
        } else {                                                        // engine.h:132-137
            us = pk.pack(running, false, nullptr);
            for (OSeq* s : running) { kvm.append_token(*s); }
            R.tokens += (long long)running.size();
        }
        R.gpu_us += us; clock += us; R.iters++;
        R.slot_steps += (long long)running.size(); R.useful_steps += (long long)running.size();
        R.peak_blocks = std::max(R.peak_blocks, kvm.a.used_count());
    }
    R.wall_us = clock;
    fill_latency(R, lat);
    R.digest = dg.h;
    *out = R;
    return rc;
}

// Static (request-level) batching (scheduler.h:33-89): std::sort by arrival
// (unstable: equal keys are permuted the way libstdc++'s introsort does), groups
// of <= maxB already-arrived requests under the pool reservation, each group runs
// until its longest member finishes with finished slots still in the batch.
struct OReq { int id; double arrival_us; int prompt_len; int gen_len; };

ORC_API int orc_sim_static(const int* prompt, const int* gen, const double* arrival, int n,
                           int block_size, int num_blocks, int max_batch, int kv_write,
                           double c0, double c1, double c2, OStats* out, int* order_out) {
    std::vector<OReq> reqs(n);
    for (int i = 0; i < n; ++i) reqs[i] = OReq{i, arrival[i], prompt[i], gen[i]};
    std::sort(reqs.begin(), reqs.end(), [](const OReq& a, const OReq& b) { return a.arrival_us < b.arrival_us; });
    if (order_out) for (int i = 0; i < n; ++i) order_out[i] = reqs[i].id;
    OKvm kvm(num_blocks, block_size, 1, 1);
    std::vector<OSeq> seqs(n);
    for (int i = 0; i < n; ++i) {
        seqs[i].id = reqs[i].id; seqs[i].prompt_len = reqs[i].prompt_len;
        seqs[i].max_new = reqs[i].gen_len; seqs[i].arrival_us = reqs[i].arrival_us;
    }
    auto wc = [&](const OSeq& s) { return blocks_needed(s.prompt_len + s.max_new, block_size); };
    OStats R{}; Digest dg; Packer pk{{}, {}, {}, {}, c0, c1, c2, &dg};
    std::vector<double> lat; size_t idx = 0; double clock = 0; int rc = 0;
    while (idx < seqs.size()) {
        if (seqs[idx].arrival_us > clock) clock = seqs[idx].arrival_us;
        std::vector<OSeq*> group; int reserved = 0;
        while ((int)group.size() < max_batch && idx < seqs.size() && seqs[idx].arrival_us <= clock) {
            int fp = wc(seqs[idx]);
            if (reserved + fp > kvm.num_blocks) break;
            kvm.allocate_prompt(seqs[idx]); reserved += fp;
            group.push_back(&seqs[idx]); ++idx;
        }
        if (group.empty()) { rc = 1; break; }
        int active = (int)group.size();
        while (active > 0) {
            double us;
            int still = 0;
            std::vector<OSeq*> newly_done;
            if (kv_write) {
                std::vector<int> wp;
                for (OSeq* s : group) {
                    if (!s->done()) { int pos = s->cur_len; kvm.append_token(*s); wp.push_back(pos); ++still; if (s->done()) newly_done.push_back(s); }
                    else wp.push_back(-1);
                }
                us = pk.pack(group, true, &wp);
            } else {
                us = pk.pack(group, false, nullptr);
                for (OSeq* s : group)
                    if (!s->done()) { kvm.append_token(*s); ++still; if (s->done()) newly_done.push_back(s); }
            }
            R.gpu_us += us; clock += us; R.iters++;
            R.slot_steps += (long long)group.size();
            R.tokens += still; R.useful_steps += still;
            for (OSeq* s : newly_done) { lat.push_back(clock - s->arrival_us); R.finished++; }
            R.peak_blocks = std::max(R.peak_blocks, kvm.a.used_count());
            active = 0; for (OSeq* s : group) if (!s->done()) ++active;
        }
        for (OSeq* s : group) kvm.free(*s);
    }
    R.wall_us = clock;
    fill_latency(R, lat);
    R.digest = dg.h;
    *out = R;
    return rc;
}
