// engine.h -- continuous (iteration-level) batching over KVCacheManager + ModelRunner.
//
// Drop-in for the reference's Engine (src/include/engine.h:24-149): same
// EngineConfig aggregate prefix {n_heads, head_dim, block_size, num_blocks,
// max_batch}, same EngineStats fields, same methods (add_request, step, run,
// reset) and the same policy, decision for decision:
//   1. retire every finished sequence (swap-with-back removal), free its blocks,
//      release its worst-case reservation, record latency = clock - arrival;
//   2. admit FIFO while the batch has room, the head has arrived and its worst
//      case ceil((prompt + max_new)/BLOCK) fits the unreserved pool;
//   3. with nothing running, advance the clock to the next arrival;
//   4. run one decode step and advance the clock by its time;
//   5. append one token to every running sequence.
// Extensions (defaulted trailing config fields): GQA, fp16, layer slices, the
// model-path step ordering (kv_write), a deterministic clock, a host-only mode,
// p50 latency and a digest of every step's packed metadata.  Where the
// reference would spin forever (a request whose worst case exceeds the whole
// pool) step() throws kvc::Error(KVC_ERR_STATE) instead.
#pragma once
#include <algorithm>
#include <chrono>
#include <deque>
#include <vector>

#include "kv_cache_manager.h"
#include "model_runner.h"
#include "sequence.h"

struct EngineConfig {
    int n_heads;       // query heads
    int head_dim;
    int block_size;    // tokens per physical block
    int num_blocks;    // physical blocks per layer slice
    int max_batch;     // max concurrently running sequences
    int n_kv_heads = 0;       // 0: = n_heads
    int n_layers = 1;
    int dtype = KVC_F32;
    bool kv_write = false;
    int clock_mode = 0;       // 0: measured GPU time, 1: c0 + c1*N + c2*sum(len)
    double c0 = 0, c1 = 0, c2 = 0;
    bool device = true;
    int split_tokens = 0;
    int decode_path = KVC_DECODE_PLANNED;
    bool prefill = false;     // admitted prompts run K/V writes + causal attention (measured clock)
    uint64_t seed = 0x6b76636163686531ull;
    bool graph = false;       // planned decode steps replay one captured HIP graph
};

struct EngineStats {
    const char* name = "";
    int iters = 0;
    long long tokens = 0;
    double gpu_us = 0;
    double wall_us = 0;
    long long slot_steps = 0;
    long long useful_steps = 0;
    int peak_blocks = 0;
    int finished = 0;
    double avg_latency_us = 0;
    double p99_latency_us = 0;
    double p50_latency_us = 0;
    uint64_t step_digest = 0;
    double host_wall_us = 0;
    double prefill_us = 0;    // GPU time of prompt processing (included in gpu_us and the clock)
};

// avg / p50 / p99 (nearest rank: sorted[min(floor(q*n), n-1)], engine.h:48-54).
inline void fill_latency_stats(EngineStats& R, std::vector<double>& lat) {
    if (lat.empty()) {
        R.avg_latency_us = R.p50_latency_us = R.p99_latency_us = 0;
        return;
    }
    std::sort(lat.begin(), lat.end());
    double s = 0;
    for (double x : lat) s += x;
    R.avg_latency_us = s / lat.size();
    R.p50_latency_us = lat[std::min((size_t)(lat.size() * 0.5), lat.size() - 1)];
    R.p99_latency_us = lat[std::min((size_t)(lat.size() * 0.99), lat.size() - 1)];
}

inline RunnerOptions runner_options(const EngineConfig& c) {
    RunnerOptions o;
    o.n_kv_heads = c.n_kv_heads;
    o.n_layers = c.n_layers;
    o.dtype = c.dtype;
    o.kv_write = c.kv_write;
    o.clock_mode = c.clock_mode;
    o.c0 = c.c0; o.c1 = c.c1; o.c2 = c.c2;
    o.device = c.device;
    o.split_tokens = c.split_tokens;
    o.decode_path = c.decode_path;
    o.prefill = c.prefill;
    o.seed = c.seed;
    o.graph = c.graph;
    return o;
}

struct Engine {
    EngineConfig cfg;
    KVCacheManager kvm;
    ModelRunner runner;
    std::deque<Sequence> store;
    std::deque<Sequence*> waiting;   // non-decreasing arrival (add_request order)
    std::vector<Sequence*> running;
    std::vector<double> latencies;
    std::vector<int> wpos;
    std::vector<Sequence*> admitted;  // this step's admissions (prefilled together)
    int reserved_blocks = 0;
    double clock = 0;
    int next_id = 0;
    EngineStats stats;

    explicit Engine(const EngineConfig& c)
        : cfg(c),
          kvm(c.num_blocks, c.block_size, c.n_kv_heads > 0 ? c.n_kv_heads : c.n_heads, c.head_dim, c.dtype,
              c.n_layers, c.device),
          runner(c.n_heads, c.head_dim, c.block_size, c.max_batch, c.num_blocks, runner_options(c)) {
        stats.name = "continuous";
    }

    void reset() {
        kvm.reset();
        store.clear(); waiting.clear(); running.clear(); latencies.clear();
        reserved_blocks = 0; clock = 0; next_id = 0;
        stats = EngineStats{};
        stats.name = "continuous";
        runner.reset_digest();
    }

    int worstcase_blocks(const Sequence& s) const { return blocks_needed(s.prompt_len + s.max_new_tokens, cfg.block_size); }

    void add_request(int prompt_len, int max_new_tokens, double arrival_us = 0.0) {
        store.push_back(Sequence{});
        Sequence& s = store.back();
        s.id = next_id++;
        s.prompt_len = prompt_len;
        s.max_new_tokens = max_new_tokens;
        s.arrival_us = arrival_us;
        s.status = SeqStatus::Waiting;
        waiting.push_back(&s);
    }

    bool step() {
        for (size_t i = 0; i < running.size();) {  // 1) retire
            Sequence* s = running[i];
            if (s->done()) {
                kvm.free(*s);
                reserved_blocks -= worstcase_blocks(*s);
                latencies.push_back(clock - s->arrival_us);
                s->status = SeqStatus::Finished;
                stats.finished++;
                running[i] = running.back();
                running.pop_back();
            } else {
                ++i;
            }
        }
        admitted.clear();
        while ((int)running.size() < cfg.max_batch && !waiting.empty() &&  // 2) admit
               waiting.front()->arrival_us <= clock) {
            Sequence* s = waiting.front();
            const int fp = worstcase_blocks(*s);
            if (reserved_blocks + fp > cfg.num_blocks) break;
            if (!kvm.allocate_prompt(*s)) break;
            reserved_blocks += fp;
            s->status = SeqStatus::Running;
            running.push_back(s);
            waiting.pop_front();
            admitted.push_back(s);
        }
        if (cfg.prefill && !admitted.empty()) {  // the step's admitted prompts are processed together
            const double pu = runner.prefill_batch(admitted, kvm);
            stats.prefill_us += pu;
            stats.gpu_us += pu;
            clock += pu;
        }
        if (running.empty()) {  // 3) idle or done
            if (waiting.empty()) return false;
            if (waiting.front()->arrival_us <= clock)
                throw kvc::Error(KVC_ERR_STATE, "Engine: request " + std::to_string(waiting.front()->id) +
                                                    " can never be admitted (worst case exceeds the pool)");
            clock = std::max(clock, waiting.front()->arrival_us);
            return true;
        }
        double us;  // 4) one decode step, 5) one token per running sequence
        if (cfg.kv_write) {
            wpos.clear();
            for (Sequence* s : running) {
                wpos.push_back(s->cur_len);
                kvm.append_token(*s);
                stats.tokens++;
            }
            us = runner.decode_step(running, kvm, wpos.data());
        } else {
            us = runner.decode_step(running, kvm);
            for (Sequence* s : running) {
                kvm.append_token(*s);
                stats.tokens++;
            }
        }
        stats.gpu_us += us;
        clock += us;
        stats.iters++;
        stats.slot_steps += (int)running.size();
        stats.useful_steps += (int)running.size();
        stats.peak_blocks = std::max(stats.peak_blocks, kvm.used_blocks());
        return true;
    }

    EngineStats run() {
        const auto t0 = std::chrono::steady_clock::now();
        while (step()) {
        }
        runner.synchronize();
        stats.host_wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        stats.wall_us = clock;
        fill_latency_stats(stats, latencies);
        stats.step_digest = runner.digest;
        return stats;
    }
};
