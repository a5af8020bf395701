// model_runner.h -- executes one decode step of a running batch on the GPU.
//
// Drop-in for the reference's ModelRunner (src/include/model_runner.h:28-84):
// same constructor (n_heads, head_dim, block_size, max_batch, max_pool_blocks)
// and decode_step(batch, kvm) -> step time in us, with the same packing
// (model_runner.h:61-69): block tables concatenated in batch order, offsets,
// lengths clamped to >= 1.  What changes on MI355X:
//   * the step's metadata {N, tab_off[N+1], len[N], wpos[N], slot[N], table_all}
//     is packed into ONE pinned host buffer (a ring of them, so the host can
//     run ahead of the GPU) and moved with ONE async copy (kvc_step_upload)
//     instead of three blocking cudaMemcpy;
//   * GQA (n_kv_heads < n_heads), fp16 KV and n_layers layer slices;
//   * with kv_write the step follows the model path (qwen_serve.cu:130-160):
//     per layer, the new token's K/V go to slot[r] (= phys*BLOCK + pos%BLOCK,
//     precomputed here) and attention covers cur_len (which already includes it);
//   * every packed step is folded into an FNV-1a digest so the schedule can be
//     compared bit for bit with an independent restatement;
//   * the clock is either measured (events around the step's kernels, as the
//     reference) or a deterministic cost model c0 + c1*N + c2*sum(len);
//   * decode is host-planned by default: the lengths are known here, so the step
//     cuts every sequence into near-equal chunks (kvc_decode_plan), appends the
//     work list to the same upload and launches the planned kernel, which needs
//     no per-sequence device lookups and balances ragged batches;
//   * with `graph` the planned step's n_layers launches are captured once as a HIP
//     graph of graph-safe launches (counts read from device memory, fixed-capacity
//     grids) and each step uploads its metadata to fixed places and replays it.
// Query/key/value inputs are synthetic N(0,1) buffers filled once on the device.
#pragma once
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../kvc_abi.h"
#include "kv_cache_manager.h"
#include "sequence.h"

struct RunnerOptions {
    int n_kv_heads = 0;      // 0: = n_heads (MHA)
    int n_layers = 1;
    int dtype = KVC_F32;
    bool kv_write = false;
    int clock_mode = 0;      // 0 measured, 1 virtual
    double c0 = 0, c1 = 0, c2 = 0;
    bool device = true;
    int split_tokens = 0;    // device-lengths path: 0 automatic
    int decode_path = KVC_DECODE_PLANNED;  // or KVC_DECODE_DEVICE_LENGTHS
    int plan_target = 0;     // planned path: tokens per unit (0 automatic)
    bool fuse_append = true; // planned path with kv_write: write the new rows inside the decode launch
    bool prefill = false;    // run each admitted prompt's K/V writes + causal attention (prefill)
    bool graph = false;      // planned steps replay one captured HIP graph
    uint64_t seed = 0x6b76636163686531ull;
};

struct ModelRunner {
    static constexpr int kRing = 4;
    int n_heads, head_dim, block_size, max_batch, max_pool_blocks;
    float scale;
    RunnerOptions opt;
    int n_kv_heads;

    void *dq = nullptr, *dk = nullptr, *dv = nullptr, *dout = nullptr;
    int* d_meta = nullptr;
    int* h_meta[kRing] = {};
    void* h_ev[kRing] = {};
    bool h_ev_used[kRing] = {};
    int ring = 0;
    void *ev0 = nullptr, *ev1 = nullptr;
    kvc_stream_t stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;

    size_t meta_cap = 0;     // ints in d_meta and in each pinned ring buffer
    std::vector<int> h_tab, h_off, h_len, h_wpos, h_slot, h_work;
    // prefill: synthetic prompt q/k/v and output for up to pf_cap tokens, the prompt's table
    void *pq = nullptr, *pk = nullptr, *pv = nullptr, *pout = nullptr;
    int* d_ptab = nullptr;
    int* h_ptab = nullptr;
    void* h_ptab_ev = nullptr;
    int pf_cap = 0, ptab_cap = 0;
    // batched prefill: causal plan and its upload [slot | tables | work]
    std::vector<int> pf_len, pf_off, pf_tab, pf_work;
    int* d_pf = nullptr;
    int* h_pf = nullptr;
    void* h_pf_ev = nullptr;
    size_t pf_meta_cap = 0;
    double last_prefill_us = 0;
    uint64_t digest = 1469598103934665603ull;
    long long last_sum_len = 0;
    int last_cap = 0;
    // graph replay: metadata at fixed places [N, units, records, 0 | wpos cap_n |
    // work cap_units*ipu | table cap_tab] in d_g, a pinned ring h_g of the same layout
    void* gexec = nullptr;
    std::vector<const void*> g_pools;       // pools the graph was captured with (K and V of every layer)
    bool graph_failed = false;
    int* d_g = nullptr;
    int* h_g[kRing] = {};
    int g_cap_units = 0, g_ipu = 0;
    size_t g_off_work = 0, g_off_tab = 0;
    long long graph_steps = 0;

    ModelRunner(int n_heads_, int head_dim_, int block_size_, int max_batch_, int max_pool_blocks_,
                const RunnerOptions& o = RunnerOptions())
        : n_heads(n_heads_), head_dim(head_dim_), block_size(block_size_), max_batch(max_batch_),
          max_pool_blocks(max_pool_blocks_), scale(1.0f / __builtin_sqrtf((float)head_dim_)), opt(o),
          n_kv_heads(o.n_kv_heads > 0 ? o.n_kv_heads : n_heads_) {
        if (n_heads <= 0 || head_dim <= 0 || block_size <= 0 || max_batch <= 0 || max_pool_blocks <= 0)
            throw kvc::Error(KVC_ERR_ARG, "ModelRunner: sizes must be positive");
        if (n_heads % n_kv_heads) throw kvc::Error(KVC_ERR_ARG, "ModelRunner: n_heads % n_kv_heads != 0");
        if (opt.n_layers <= 0) opt.n_layers = 1;
        h_tab.reserve(max_pool_blocks);
        h_off.reserve(max_batch + 1);
        h_len.reserve(max_batch);
        if (!opt.device) return;
        const size_t es = kvc::dtype_size(opt.dtype);
        const size_t nq = (size_t)opt.n_layers * max_batch * n_heads * head_dim;
        const size_t nkv = (size_t)opt.n_layers * max_batch * n_kv_heads * head_dim;
        kvc::check(kvc_stream_create(&stream), "ModelRunner stream");
        kvc::check(kvc_malloc(&dq, nq * es), "ModelRunner q");
        kvc::check(kvc_malloc(&dk, nkv * es), "ModelRunner k");
        kvc::check(kvc_malloc(&dv, nkv * es), "ModelRunner v");
        kvc::check(kvc_malloc(&dout, (size_t)max_batch * n_heads * head_dim * es), "ModelRunner out");
        for (int i = 0; i < kRing; ++i) kvc::check(kvc_event_create(&h_ev[i]), "ModelRunner event");
        // metadata plus a work list of ~4 units per (sequence, KV head); grown on demand
        ensure_meta(meta_ints() + (size_t)8 * 4 * max_batch * n_kv_heads * (n_heads / n_kv_heads));
        kvc::check(kvc_event_create(&ev0), "ModelRunner event");
        kvc::check(kvc_event_create(&ev1), "ModelRunner event");
        kvc::check(kvc_fill_normal(dq, nq, opt.dtype, opt.seed, 1.0f, stream), "ModelRunner fill q");
        kvc::check(kvc_fill_normal(dk, nkv, opt.dtype, opt.seed + 1, 1.0f, stream), "ModelRunner fill k");
        kvc::check(kvc_fill_normal(dv, nkv, opt.dtype, opt.seed + 2, 1.0f, stream), "ModelRunner fill v");
        kvc::check(kvc_stream_synchronize(stream), "ModelRunner init");
    }
    ~ModelRunner() {
        if (stream) kvc_stream_synchronize(stream);
        kvc_free(dq); kvc_free(dk); kvc_free(dv); kvc_free(dout); kvc_free(d_meta); kvc_free(ws);
        kvc_free(pq); kvc_free(pk); kvc_free(pv); kvc_free(pout); kvc_free(d_ptab); kvc_host_free(h_ptab);
        kvc_event_destroy(h_ptab_ev);
        kvc_free(d_pf); kvc_host_free(h_pf); kvc_event_destroy(h_pf_ev);
        for (int i = 0; i < kRing; ++i) { kvc_host_free(h_meta[i]); kvc_event_destroy(h_ev[i]); }
        kvc_event_destroy(ev0); kvc_event_destroy(ev1);
        kvc_graph_destroy(gexec);
        kvc_free(d_g);
        for (int i = 0; i < kRing; ++i) kvc_host_free(h_g[i]);
        kvc_stream_destroy(stream);
    }
    ModelRunner(const ModelRunner&) = delete;
    ModelRunner& operator=(const ModelRunner&) = delete;

    size_t meta_ints() const { return 1 + (size_t)(max_batch + 1) + 3 * (size_t)max_batch + max_pool_blocks; }
    // (Re)allocates d_meta and the pinned ring for at least `ints` ints.
    void ensure_meta(size_t ints) {
        if (ints <= meta_cap) return;
        const size_t cap = std::max(ints, meta_cap * 2);
        if (stream) kvc::check(kvc_stream_synchronize(stream), "meta growth");
        kvc_free(d_meta);
        d_meta = nullptr;
        for (int i = 0; i < kRing; ++i) {
            kvc_host_free(h_meta[i]);
            h_meta[i] = nullptr;
            h_ev_used[i] = false;
        }
        meta_cap = 0;
        kvc::check(kvc_malloc((void**)&d_meta, cap * sizeof(int)), "ModelRunner meta");
        for (int i = 0; i < kRing; ++i)
            kvc::check(kvc_host_alloc((void**)&h_meta[i], cap * sizeof(int)), "ModelRunner pinned meta");
        meta_cap = cap;
    }
    void ensure_workspace(size_t need) {
        if (need <= ws_bytes) return;
        kvc::check(kvc_stream_synchronize(stream), "workspace growth");
        kvc_graph_destroy(gexec);  // it holds the old workspace
        gexec = nullptr;
        kvc_free(ws);
        ws = nullptr;
        ws_bytes = 0;
        const size_t sz = std::max(need * 2, (size_t)1 << 20);
        kvc::check(kvc_malloc(&ws, sz), "decode workspace");
        ws_bytes = sz;
    }
    void reset_digest() { digest = 1469598103934665603ull; }
    void fold(int32_t x) {
        const uint32_t u = (uint32_t)x;
        for (int i = 0; i < 4; ++i) { digest ^= (u >> (8 * i)) & 0xffu; digest *= 1099511628211ull; }
    }
    // Synthetic per-layer inputs ([n_layers][max_batch][H][D]).
    void* q_layer(int l) const { return (char*)dq + (size_t)l * max_batch * n_heads * head_dim * kvc::dtype_size(opt.dtype); }
    void* k_layer(int l) const { return (char*)dk + (size_t)l * max_batch * n_kv_heads * head_dim * kvc::dtype_size(opt.dtype); }
    void* v_layer(int l) const { return (char*)dv + (size_t)l * max_batch * n_kv_heads * head_dim * kvc::dtype_size(opt.dtype); }

    // One decode step over `batch`.  wpos (kv_write only): per sequence the position
    // its new K/V are written to this step, or -1 for a slot that only idles.
    double decode_step(const std::vector<Sequence*>& batch, KVCacheManager& kvm, const int* wpos = nullptr) {
        const int n = (int)batch.size();
        if (n == 0) return 0.0;
        if (n > max_batch) throw kvc::Error(KVC_ERR_ARG, "decode_step: batch larger than max_batch");
        h_tab.clear(); h_off.clear(); h_len.clear(); h_wpos.clear(); h_slot.clear();
        int cap = 1;
        long long sum_len = 0;
        for (int r = 0; r < n; ++r) {
            const Sequence* s = batch[r];
            h_off.push_back((int)h_tab.size());
            h_tab.insert(h_tab.end(), s->block_table.begin(), s->block_table.end());
            const int L = s->cur_len > 0 ? s->cur_len : 1;
            h_len.push_back(L);
            cap = std::max(cap, L);
            sum_len += L;
            if (opt.kv_write) {
                const int p = wpos ? wpos[r] : -1;
                h_wpos.push_back(p);
                h_slot.push_back(p >= 0 ? s->block_table[p / block_size] * block_size + p % block_size : -1);
            }
        }
        h_off.push_back((int)h_tab.size());
        if ((int)h_tab.size() > max_pool_blocks) throw kvc::Error(KVC_ERR_ARG, "decode_step: tables exceed max_pool_blocks");
        fold(n);
        for (int x : h_off) fold(x);
        for (int x : h_len) fold(x);
        if (opt.kv_write) for (int x : h_wpos) fold(x);
        for (int x : h_tab) fold(x);
        last_sum_len = sum_len;
        last_cap = cap;
        const double virt = opt.c0 + opt.c1 * (double)n + opt.c2 * (double)sum_len;
        if (!opt.device) return virt;
        if (!kvm.has_device()) throw kvc::Error(KVC_ERR_STATE, "decode_step: KV manager has no device pools");

        const int T = (int)h_tab.size();
        const bool planned = opt.decode_path == KVC_DECODE_PLANNED && T > 0;
        int n_units = 0, n_records = 0;
        if (planned) {
            kvc::check(kvc_decode_plan(h_len.data(), h_off.data(), h_tab.data(), T, n, n_heads, n_kv_heads, head_dim,
                                       block_size, opt.dtype, opt.plan_target, nullptr, 0, &n_units, &n_records),
                       "decode plan");
            const int ipu = kvc_decode_plan_entry_ints(n_heads, n_kv_heads, head_dim, block_size, opt.dtype);
            h_work.resize((size_t)n_units * ipu);
            kvc::check(kvc_decode_plan(h_len.data(), h_off.data(), h_tab.data(), T, n, n_heads, n_kv_heads, head_dim,
                                       block_size, opt.dtype, opt.plan_target, h_work.data(), n_units, &n_units,
                                       &n_records),
                       "decode plan");
        } else {
            h_work.clear();
        }
        // pack: [N | off N+1 | len N | wpos N | slot N | tab T | work units*entry_ints]
        ensure_meta(1 + (size_t)(n + 1) + 3 * (size_t)n + T + h_work.size());
        if (h_ev_used[ring]) kvc::check(kvc_event_synchronize(h_ev[ring]), "meta ring wait");
        int* h = h_meta[ring];
        size_t o = 0;
        h[o++] = n;
        std::memcpy(h + o, h_off.data(), h_off.size() * sizeof(int)); o += h_off.size();
        std::memcpy(h + o, h_len.data(), n * sizeof(int)); o += n;
        if (opt.kv_write) {
            std::memcpy(h + o, h_wpos.data(), n * sizeof(int));
            std::memcpy(h + o + n, h_slot.data(), n * sizeof(int));
        }
        o += 2 * (size_t)n;
        std::memcpy(h + o, h_tab.data(), h_tab.size() * sizeof(int)); o += h_tab.size();
        std::memcpy(h + o, h_work.data(), h_work.size() * sizeof(int)); o += h_work.size();
        kvc::check(kvc_step_upload(d_meta, h, o * sizeof(int), stream), "step upload");
        kvc::check(kvc_event_record(h_ev[ring], stream), "meta ring record");
        h_ev_used[ring] = true;
        ring = (ring + 1) % kRing;
        const int* d_off = d_meta + 1;
        const int* d_len = d_off + n + 1;
        const int* d_slot = d_len + 2 * n;
        const int* d_tab = d_len + 3 * n;
        const int* d_work = d_tab + T;

        if (planned && opt.graph && (!opt.kv_write || opt.fuse_append) && ensure_graph(kvm) &&
            n_units <= g_cap_units && n_records <= g_cap_units)
            return replay(n, T, n_units, n_records, virt);
        ensure_workspace(planned ? kvc_decode_planned_workspace_size(n_heads, n_kv_heads, head_dim, block_size,
                                                                   opt.dtype, n_records)
                                 : kvc_decode_workspace_size(n, n_heads, n_kv_heads, head_dim, block_size, cap,
                                                             opt.split_tokens, opt.dtype));
        kvc::check(kvc_event_record(ev0, stream), "event");
        const bool fused = planned && opt.kv_write && opt.fuse_append;
        const int* d_wpos = d_len + n;
        for (int l = 0; l < opt.n_layers; ++l) {
            if (fused) {
                kvc::check(kvc_batched_paged_append_decode_planned(
                               q_layer(l), k_layer(l), v_layer(l), d_wpos, kvm.k_layer(l), kvm.v_layer(l), d_tab, T,
                               dout, n, n_heads, n_kv_heads, head_dim, block_size, scale, opt.dtype, d_work, n_units,
                               n_records, ws, ws_bytes, stream),
                           "planned append + decode");
                continue;
            }
            if (opt.kv_write)
                kvc::check(kvc_write_kv_slots(k_layer(l), v_layer(l), kvm.k_layer(l), kvm.v_layer(l), d_slot, n,
                                              n_kv_heads, head_dim, block_size, opt.dtype, stream),
                           "write_kv");
            if (planned)
                kvc::check(kvc_batched_paged_decode_planned(q_layer(l), kvm.k_layer(l), kvm.v_layer(l), d_tab, T, dout,
                                                            n, n_heads, n_kv_heads, head_dim, block_size, scale,
                                                            opt.dtype, d_work, n_units, n_records, ws, ws_bytes,
                                                            stream),
                           "planned paged decode");
            else
                kvc::check(kvc_batched_paged_decode_split(q_layer(l), kvm.k_layer(l), kvm.v_layer(l), d_tab, d_off,
                                                          d_len, dout, n, n_heads, n_kv_heads, head_dim, block_size,
                                                          cap, scale, opt.dtype, opt.split_tokens, ws, ws_bytes,
                                                          stream),
                           "paged decode");
        }
        kvc::check(kvc_event_record(ev1, stream), "event");
        if (opt.clock_mode != 0) return virt;
        float ms = 0.f;
        kvc::check(kvc_event_elapsed_ms(&ms, ev0, ev1), "event elapsed");
        return (double)ms * 1e3;
    }

    // Captures the planned step (n_layers graph-safe launches) for these pools.
    std::vector<const void*> pools_of(const KVCacheManager& kvm) const {
        std::vector<const void*> p;
        for (int l = 0; l < opt.n_layers; ++l) { p.push_back(kvm.k_layer(l)); p.push_back(kvm.v_layer(l)); }
        return p;
    }
    bool ensure_graph(const KVCacheManager& kvm) {
        if (gexec && g_pools == pools_of(kvm)) return true;
        if (graph_failed) return false;
        kvc_graph_destroy(gexec);
        gexec = nullptr;
        if (!d_g) {
            g_ipu = kvc_decode_plan_entry_ints(n_heads, n_kv_heads, head_dim, block_size, opt.dtype);
            kvc::check(kvc_decode_plan_capacity(max_batch, (long long)max_pool_blocks * block_size, n_heads,
                                                n_kv_heads, head_dim, block_size, opt.dtype, &g_cap_units),
                       "plan capacity");
            g_off_work = 4 + (size_t)max_batch;
            g_off_tab = g_off_work + (size_t)g_cap_units * g_ipu;
            const size_t ints = g_off_tab + max_pool_blocks;
            kvc::check(kvc_malloc((void**)&d_g, ints * sizeof(int)), "graph metadata");
            for (int i = 0; i < kRing; ++i)
                kvc::check(kvc_host_alloc((void**)&h_g[i], ints * sizeof(int)), "pinned graph metadata");
            kvc::check(kvc_memset(d_g, 0, ints * sizeof(int), stream), "graph metadata");
        }
        ensure_workspace(kvc_decode_planned_workspace_size(n_heads, n_kv_heads, head_dim, block_size, opt.dtype,
                                                           g_cap_units));
        kvc::check(kvc_stream_synchronize(stream), "graph setup");
        const int* d_counts = d_g;
        const int* d_wpos = d_g + 4;
        const int* d_work = d_g + g_off_work;
        const int* d_tab = d_g + g_off_tab;
        kvc::check(kvc_graph_begin(stream), "graph capture");
        int rc = KVC_OK;
        for (int l = 0; l < opt.n_layers && rc == KVC_OK; ++l)
            rc = kvc_batched_paged_decode_planned_dev(
                q_layer(l), opt.kv_write ? k_layer(l) : nullptr, opt.kv_write ? v_layer(l) : nullptr,
                opt.kv_write ? d_wpos : nullptr, kvm.k_layer(l), kvm.v_layer(l), d_tab, max_pool_blocks, dout,
                max_batch, n_heads, n_kv_heads, head_dim, block_size, scale, opt.dtype, d_work, g_cap_units,
                g_cap_units, d_counts, ws, ws_bytes, stream);
        void* exec = nullptr;
        const int rc_end = kvc_graph_end(stream, &exec);
        if (rc != KVC_OK || rc_end != KVC_OK) {
            kvc_graph_destroy(exec);
            graph_failed = true;
            return false;
        }
        gexec = exec;
        g_pools = pools_of(kvm);
        return true;
    }

    // One planned step by graph replay (the metadata of h_tab/h_wpos/h_work).
    double replay(int n, int T, int n_units, int n_records, double virt) {
        if (h_ev_used[ring]) kvc::check(kvc_event_synchronize(h_ev[ring]), "meta ring wait");
        int* h = h_g[ring];
        h[0] = n; h[1] = n_units; h[2] = n_records; h[3] = 0;
        if (opt.kv_write) std::memcpy(h + 4, h_wpos.data(), n * sizeof(int));
        std::memcpy(h + g_off_work, h_work.data(), h_work.size() * sizeof(int));
        std::memcpy(h + g_off_tab, h_tab.data(), (size_t)T * sizeof(int));
        kvc::check(kvc_step_upload(d_g, h, (g_off_work + h_work.size()) * sizeof(int), stream), "step upload");
        kvc::check(kvc_step_upload(d_g + g_off_tab, h + g_off_tab, (size_t)T * sizeof(int), stream), "table upload");
        kvc::check(kvc_event_record(h_ev[ring], stream), "meta ring record");
        h_ev_used[ring] = true;
        ring = (ring + 1) % kRing;
        kvc::check(kvc_event_record(ev0, stream), "event");
        kvc::check(kvc_graph_launch(gexec, stream), "graph launch");
        kvc::check(kvc_event_record(ev1, stream), "event");
        ++graph_steps;
        if (opt.clock_mode != 0) return virt;
        float ms = 0.f;
        kvc::check(kvc_event_elapsed_ms(&ms, ev0, ev1), "event elapsed");
        return (double)ms * 1e3;
    }

    // Prompt processing of one admitted sequence, the attention part of the model
    // path's prefill (qwen_serve.cu:90-124): per layer, write the prompt's K/V rows
    // through its table (qk_write_kv) and run the causal prompt attention
    // (qk_paged_causal_attn).  Inputs are synthetic.  Returns the GPU time (us)
    // on the measured clock, 0 on the virtual clock.
    double prefill(const Sequence& s, KVCacheManager& kvm) {
        last_prefill_us = 0;
        if (!opt.device || !opt.prefill || s.prompt_len <= 0) return 0.0;
        if (!kvm.has_device()) throw kvc::Error(KVC_ERR_STATE, "prefill: KV manager has no device pools");
        const int P = s.prompt_len;
        const int nb = (int)s.block_table.size();
        const size_t es = kvc::dtype_size(opt.dtype);
        if (P > pf_cap) {
            kvc::check(kvc_stream_synchronize(stream), "prefill growth");
            kvc_free(pq); kvc_free(pk); kvc_free(pv); kvc_free(pout);
            pq = pk = pv = pout = nullptr;
            pf_cap = 0;
            const int cap = std::max(P, 256);
            kvc::check(kvc_malloc(&pq, (size_t)cap * n_heads * head_dim * es), "prefill q");
            kvc::check(kvc_malloc(&pout, (size_t)cap * n_heads * head_dim * es), "prefill out");
            kvc::check(kvc_malloc(&pk, (size_t)cap * n_kv_heads * head_dim * es), "prefill k");
            kvc::check(kvc_malloc(&pv, (size_t)cap * n_kv_heads * head_dim * es), "prefill v");
            kvc::check(kvc_fill_normal(pq, (size_t)cap * n_heads * head_dim, opt.dtype, opt.seed + 3, 1.0f, stream), "fill");
            kvc::check(kvc_fill_normal(pk, (size_t)cap * n_kv_heads * head_dim, opt.dtype, opt.seed + 4, 1.0f, stream), "fill");
            kvc::check(kvc_fill_normal(pv, (size_t)cap * n_kv_heads * head_dim, opt.dtype, opt.seed + 5, 1.0f, stream), "fill");
            pf_cap = cap;
        }
        if (nb > ptab_cap) {
            kvc::check(kvc_stream_synchronize(stream), "prefill table growth");
            kvc_free(d_ptab); kvc_host_free(h_ptab);
            d_ptab = nullptr; h_ptab = nullptr;
            const int cap = std::max(nb, 64);
            kvc::check(kvc_malloc((void**)&d_ptab, cap * sizeof(int)), "prefill table");
            kvc::check(kvc_host_alloc((void**)&h_ptab, cap * sizeof(int)), "prefill pinned table");
            if (!h_ptab_ev) kvc::check(kvc_event_create(&h_ptab_ev), "prefill event");
            ptab_cap = cap;
        } else {
            kvc::check(kvc_event_synchronize(h_ptab_ev), "prefill table wait");  // previous upload done
        }
        std::memcpy(h_ptab, s.block_table.data(), nb * sizeof(int));
        kvc::check(kvc_step_upload(d_ptab, h_ptab, nb * sizeof(int), stream), "prefill table upload");
        kvc::check(kvc_event_record(h_ptab_ev, stream), "prefill event");
        ensure_workspace(kvc_paged_causal_attn_workspace_size(0, P, n_heads, n_kv_heads, head_dim, block_size,
                                                              opt.dtype));
        kvc::check(kvc_event_record(ev0, stream), "event");
        for (int l = 0; l < opt.n_layers; ++l) {
            kvc::check(kvc_write_kv(pk, pv, kvm.k_layer(l), kvm.v_layer(l), d_ptab, 0, P, n_kv_heads, head_dim,
                                    block_size, opt.dtype, stream),
                       "prefill write_kv");
            kvc::check(kvc_paged_causal_attn(pq, pout, kvm.k_layer(l), kvm.v_layer(l), d_ptab, 0, P, n_heads,
                                             n_kv_heads, head_dim, block_size, scale, opt.dtype, ws, ws_bytes, stream),
                       "prefill attention");
        }
        kvc::check(kvc_event_record(ev1, stream), "event");
        if (opt.clock_mode != 0) return 0.0;
        float ms = 0.f;
        kvc::check(kvc_event_elapsed_ms(&ms, ev0, ev1), "event elapsed");
        last_prefill_us = (double)ms * 1e3;
        return last_prefill_us;
    }

    // Prompt processing of the sequences admitted in one step, together: per layer one
    // slot-mapped write of every prompt row's K/V and ONE planned decode launch in
    // which row r of a prompt is a query of length r + 1 over that prompt's table (the
    // causal definition of qwen_kernels.cu:146-181).  A single prompt takes prefill().
    // Returns the GPU time (us) on the measured clock, 0 on the virtual clock.
    double prefill_batch(const std::vector<Sequence*>& ss, KVCacheManager& kvm) {
        last_prefill_us = 0;
        if (!opt.device || !opt.prefill || ss.empty()) return 0.0;
        if (ss.size() == 1) return prefill(*ss[0], kvm);
        if (!kvm.has_device()) throw kvc::Error(KVC_ERR_STATE, "prefill: KV manager has no device pools");
        const size_t es = kvc::dtype_size(opt.dtype);
        int R = 0, T = 0;
        for (const Sequence* s : ss) { R += std::max(s->prompt_len, 0); T += (int)s->block_table.size(); }
        if (R == 0) return 0.0;
        if (R > pf_cap) {
            kvc::check(kvc_stream_synchronize(stream), "prefill growth");
            kvc_free(pq); kvc_free(pk); kvc_free(pv); kvc_free(pout);
            pq = pk = pv = pout = nullptr;
            pf_cap = 0;
            const int cap = std::max(R, 256);
            kvc::check(kvc_malloc(&pq, (size_t)cap * n_heads * head_dim * es), "prefill q");
            kvc::check(kvc_malloc(&pout, (size_t)cap * n_heads * head_dim * es), "prefill out");
            kvc::check(kvc_malloc(&pk, (size_t)cap * n_kv_heads * head_dim * es), "prefill k");
            kvc::check(kvc_malloc(&pv, (size_t)cap * n_kv_heads * head_dim * es), "prefill v");
            kvc::check(kvc_fill_normal(pq, (size_t)cap * n_heads * head_dim, opt.dtype, opt.seed + 3, 1.0f, stream), "fill");
            kvc::check(kvc_fill_normal(pk, (size_t)cap * n_kv_heads * head_dim, opt.dtype, opt.seed + 4, 1.0f, stream), "fill");
            kvc::check(kvc_fill_normal(pv, (size_t)cap * n_kv_heads * head_dim, opt.dtype, opt.seed + 5, 1.0f, stream), "fill");
            pf_cap = cap;
        }
        // plan: rows of every prompt with causal lengths over their own tables
        pf_len.resize(R); pf_off.resize(R); pf_tab.resize(T);
        std::vector<int> slot(R);
        int r0 = 0, t0 = 0;
        for (const Sequence* s : ss) {
            std::memcpy(pf_tab.data() + t0, s->block_table.data(), s->block_table.size() * sizeof(int));
            for (int r = 0; r < s->prompt_len; ++r) {
                pf_len[r0 + r] = r + 1;
                pf_off[r0 + r] = t0;
                slot[r0 + r] = s->block_table[r / block_size] * block_size + r % block_size;
            }
            r0 += s->prompt_len;
            t0 += (int)s->block_table.size();
        }
        int nu = 0, nr = 0;
        kvc::check(kvc_decode_plan(pf_len.data(), pf_off.data(), pf_tab.data(), T, R, n_heads, n_kv_heads, head_dim,
                                   block_size, opt.dtype, opt.plan_target, nullptr, 0, &nu, &nr),
                   "prefill plan");
        const int ipu = kvc_decode_plan_entry_ints(n_heads, n_kv_heads, head_dim, block_size, opt.dtype);
        pf_work.resize((size_t)nu * ipu);
        kvc::check(kvc_decode_plan(pf_len.data(), pf_off.data(), pf_tab.data(), T, R, n_heads, n_kv_heads, head_dim,
                                   block_size, opt.dtype, opt.plan_target, pf_work.data(), nu, &nu, &nr),
                   "prefill plan");
        // one upload: [slot R | tables T | work]
        const size_t ints = (size_t)R + T + pf_work.size();
        if (ints > pf_meta_cap) {
            kvc::check(kvc_stream_synchronize(stream), "prefill metadata growth");
            kvc_free(d_pf); kvc_host_free(h_pf);
            d_pf = nullptr; h_pf = nullptr;
            pf_meta_cap = std::max(ints, pf_meta_cap * 2);
            kvc::check(kvc_malloc((void**)&d_pf, pf_meta_cap * sizeof(int)), "prefill metadata");
            kvc::check(kvc_host_alloc((void**)&h_pf, pf_meta_cap * sizeof(int)), "pinned prefill metadata");
            if (!h_pf_ev) kvc::check(kvc_event_create(&h_pf_ev), "prefill event");
        } else if (h_pf_ev) {
            kvc::check(kvc_event_synchronize(h_pf_ev), "prefill metadata wait");  // previous upload done
        }
        std::memcpy(h_pf, slot.data(), (size_t)R * sizeof(int));
        std::memcpy(h_pf + R, pf_tab.data(), (size_t)T * sizeof(int));
        std::memcpy(h_pf + R + T, pf_work.data(), pf_work.size() * sizeof(int));
        kvc::check(kvc_step_upload(d_pf, h_pf, ints * sizeof(int), stream), "prefill upload");
        kvc::check(kvc_event_record(h_pf_ev, stream), "prefill event");
        const int* d_slot = d_pf;
        const int* d_tab = d_pf + R;
        const int* d_work = d_tab + T;
        ensure_workspace(kvc_decode_planned_workspace_size(n_heads, n_kv_heads, head_dim, block_size, opt.dtype, nr));
        kvc::check(kvc_event_record(ev0, stream), "event");
        for (int l = 0; l < opt.n_layers; ++l) {
            kvc::check(kvc_write_kv_slots(pk, pv, kvm.k_layer(l), kvm.v_layer(l), d_slot, R, n_kv_heads, head_dim,
                                          block_size, opt.dtype, stream),
                       "prefill write_kv");
            kvc::check(kvc_batched_paged_decode_planned(pq, kvm.k_layer(l), kvm.v_layer(l), d_tab, T, pout, R,
                                                        n_heads, n_kv_heads, head_dim, block_size, scale, opt.dtype,
                                                        d_work, nu, nr, ws, ws_bytes, stream),
                       "prefill attention");
        }
        kvc::check(kvc_event_record(ev1, stream), "event");
        if (opt.clock_mode != 0) return 0.0;
        float ms = 0.f;
        kvc::check(kvc_event_elapsed_ms(&ms, ev0, ev1), "event elapsed");
        last_prefill_us = (double)ms * 1e3;
        return last_prefill_us;
    }

    void synchronize() {
        if (stream) kvc::check(kvc_stream_synchronize(stream), "ModelRunner sync");
    }
};
