// scheduler.h -- workload trace type and the static (request-level) batching baseline.
//
// Drop-in for the reference's Request / run_static (src/include/scheduler.h:24-89):
// requests are std::sort-ed by arrival (the same unstable sort, so equal arrival
// times are permuted exactly as the reference's libstdc++ build does), then run
// in groups of at most maxB already-arrived requests under the pool
// reservation.  A group runs until its longest member finishes; finished
// members keep their slot (the kernel still attends for them) and their blocks
// are returned only when the whole group ends.  Shares the Engine's
// KVCacheManager and ModelRunner; with the runner's kv_write option the step
// ordering is the model path's (grow, write at cur_len, attend).
#pragma once
#include <algorithm>
#include <chrono>
#include <vector>

#include "engine.h"

struct Request {
    int id = 0;
    double arrival_us = 0;
    int prompt_len = 0;
    int gen_len = 0;
};

inline EngineStats run_static(std::vector<Request> reqs, KVCacheManager& kvm, ModelRunner& runner, int maxB) {
    const auto t_start = std::chrono::steady_clock::now();
    EngineStats R;
    R.name = "static";
    std::sort(reqs.begin(), reqs.end(), [](const Request& a, const Request& b) { return a.arrival_us < b.arrival_us; });
    kvm.reset();
    runner.reset_digest();

    std::vector<Sequence> seqs(reqs.size());
    for (size_t i = 0; i < reqs.size(); ++i) {
        seqs[i].id = reqs[i].id;
        seqs[i].prompt_len = reqs[i].prompt_len;
        seqs[i].max_new_tokens = reqs[i].gen_len;
        seqs[i].arrival_us = reqs[i].arrival_us;
    }
    auto wc = [&](const Sequence& s) { return blocks_needed(s.prompt_len + s.max_new_tokens, kvm.block_size); };

    std::vector<double> lat;
    std::vector<int> wpos;
    std::vector<Sequence*> newly_done;
    size_t idx = 0;
    double clock = 0;
    while (idx < seqs.size()) {
        if (seqs[idx].arrival_us > clock) clock = seqs[idx].arrival_us;
        std::vector<Sequence*> group;
        int reserved = 0;
        while ((int)group.size() < maxB && idx < seqs.size() && seqs[idx].arrival_us <= clock) {
            const int fp = wc(seqs[idx]);
            if (reserved + fp > kvm.num_blocks) break;
            kvm.allocate_prompt(seqs[idx]);
            reserved += fp;
            group.push_back(&seqs[idx]);
            ++idx;
        }
        if (group.empty()) break;  // not even one request fits the pool
        if (runner.opt.prefill) {  // the group's prompts are processed together on admission
            const double pu = runner.prefill_batch(group, kvm);
            R.prefill_us += pu;
            R.gpu_us += pu;
            clock += pu;
        }
        int active = (int)group.size();
        while (active > 0) {
            int still = 0;
            newly_done.clear();
            double us;
            if (runner.opt.kv_write) {
                wpos.clear();
                for (Sequence* s : group) {
                    if (!s->done()) {
                        wpos.push_back(s->cur_len);
                        kvm.append_token(*s);
                        ++still;
                        if (s->done()) newly_done.push_back(s);
                    } else {
                        wpos.push_back(-1);
                    }
                }
                us = runner.decode_step(group, kvm, wpos.data());
            } else {
                us = runner.decode_step(group, kvm);
                for (Sequence* s : group)
                    if (!s->done()) {
                        kvm.append_token(*s);
                        ++still;
                        if (s->done()) newly_done.push_back(s);
                    }
            }
            R.gpu_us += us;
            clock += us;
            R.iters++;
            R.slot_steps += (int)group.size();
            R.tokens += still;
            R.useful_steps += still;
            for (Sequence* s : newly_done) {
                lat.push_back(clock - s->arrival_us);
                R.finished++;
            }
            R.peak_blocks = std::max(R.peak_blocks, kvm.used_blocks());
            active = 0;
            for (Sequence* s : group)
                if (!s->done()) ++active;
        }
        for (Sequence* s : group) kvm.free(*s);
    }
    runner.synchronize();
    R.host_wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t_start).count();
    R.wall_us = clock;
    fill_latency_stats(R, lat);
    R.step_digest = runner.digest;
    return R;
}
