// engine_abi.cpp -- extern "C" handles over the C++ BlockAllocator, Engine and
// run_static (include/kvc/*.h), so non-C++ hosts (ctypes, FFI) drive the very
// same header code a C++ caller compiles.  Exceptions never cross the boundary.
#include <exception>
#include <string>
#include <vector>

#include "status.hpp"
#include "kvc/block_alloc.h"
#include "kvc/engine.h"
#include "kvc/scheduler.h"
#include "kvc_abi.h"

struct kvc_block_allocator {
    BlockAllocator a;
};
struct kvc_engine {
    Engine e;
    explicit kvc_engine(const EngineConfig& c) : e(c) {}
};

namespace {
template <class F>
int guard(F&& f) {
    try {
        return f();
    } catch (const kvc::Error& e) {
        return kvc::set_error(e.status, e.what());
    } catch (const std::exception& e) {
        return kvc::set_error(KVC_ERR_ARG, std::string("internal error: ") + e.what());
    } catch (...) {
        return kvc::set_error(KVC_ERR_ARG, "internal error");
    }
}

void to_c(const EngineStats& s, kvc_engine_stats* o) {
    o->iters = s.iters;
    o->tokens = s.tokens;
    o->gpu_us = s.gpu_us;
    o->wall_us = s.wall_us;
    o->slot_steps = s.slot_steps;
    o->useful_steps = s.useful_steps;
    o->peak_blocks = s.peak_blocks;
    o->finished = s.finished;
    o->avg_latency_us = s.avg_latency_us;
    o->p50_latency_us = s.p50_latency_us;
    o->p99_latency_us = s.p99_latency_us;
    o->step_digest = s.step_digest;
    o->host_wall_us = s.host_wall_us;
    o->prefill_us = s.prefill_us;
}
}  // namespace

extern "C" {

int kvc_block_allocator_create(int total_blocks, kvc_block_allocator** out) {
    if (!out) return kvc::set_error(KVC_ERR_ARG, "null out pointer");
    *out = nullptr;
    if (total_blocks < 0) return kvc::set_error(KVC_ERR_ARG, "total_blocks must be >= 0");
    return guard([&]() -> int {
        *out = new kvc_block_allocator{BlockAllocator(total_blocks)};
        return KVC_OK;
    });
}
void kvc_block_allocator_destroy(kvc_block_allocator* a) { delete a; }
int kvc_block_allocator_alloc(kvc_block_allocator* a) { return a ? a->a.alloc() : -1; }
void kvc_block_allocator_free(kvc_block_allocator* a, const int* blocks, int n) {
    if (a && blocks && n > 0) a->a.free_blocks(blocks, n);
}
void kvc_block_allocator_reset(kvc_block_allocator* a) {
    if (a) a->a.reset();
}
int kvc_block_allocator_free_count(const kvc_block_allocator* a) { return a ? a->a.free_count() : 0; }
int kvc_block_allocator_used_count(const kvc_block_allocator* a) { return a ? a->a.used_count() : 0; }
void kvc_block_allocator_shuffle(kvc_block_allocator* a, uint64_t seed) {
    if (a) a->a.shuffle(seed);
}
int kvc_blocks_needed(int seq_len, int block) { return block > 0 ? blocks_needed(seq_len, block) : -1; }

int kvc_engine_create(const kvc_engine_config* c, kvc_engine** out) {
    if (!c || !out) return kvc::set_error(KVC_ERR_ARG, "null config / out pointer");
    *out = nullptr;
    return guard([&]() -> int {
        EngineConfig ec{c->n_heads, c->head_dim, c->block_size, c->num_blocks, c->max_batch};
        ec.n_kv_heads = c->n_kv_heads;
        ec.n_layers = c->n_layers > 0 ? c->n_layers : 1;
        ec.dtype = c->dtype;
        ec.kv_write = c->kv_write != 0;
        ec.clock_mode = c->clock_mode;
        ec.c0 = c->virt_c0;
        ec.c1 = c->virt_c1;
        ec.c2 = c->virt_c2;
        ec.device = c->device != 0;
        ec.split_tokens = c->split_tokens;
        if (c->decode_path != KVC_DECODE_PLANNED && c->decode_path != KVC_DECODE_DEVICE_LENGTHS)
            return kvc::set_error(KVC_ERR_ARG, "decode_path must be KVC_DECODE_PLANNED or KVC_DECODE_DEVICE_LENGTHS");
        ec.decode_path = c->decode_path;
        ec.prefill = c->prefill != 0;
        ec.graph = c->graph != 0;
        if (c->seed) ec.seed = c->seed;
        if (c->max_batch <= 0) return kvc::set_error(KVC_ERR_ARG, "max_batch must be > 0");
        *out = new kvc_engine(ec);
        return KVC_OK;
    });
}
void kvc_engine_destroy(kvc_engine* e) {
    try {
        delete e;
    } catch (...) {
    }
}
int kvc_engine_reset(kvc_engine* e) {
    if (!e) return kvc::set_error(KVC_ERR_ARG, "null engine");
    return guard([&]() -> int {
        e->e.reset();
        return KVC_OK;
    });
}
int kvc_engine_add_request(kvc_engine* e, int prompt_len, int max_new_tokens, double arrival_us) {
    if (!e) return kvc::set_error(KVC_ERR_ARG, "null engine");
    if (prompt_len < 0 || max_new_tokens < 0) return kvc::set_error(KVC_ERR_ARG, "lengths must be >= 0");
    if (!e->e.waiting.empty() && arrival_us < e->e.waiting.back()->arrival_us)
        return kvc::set_error(KVC_ERR_ARG, "requests must be added in non-decreasing arrival order");
    return guard([&]() -> int {
        e->e.add_request(prompt_len, max_new_tokens, arrival_us);
        return KVC_OK;
    });
}
int kvc_engine_step(kvc_engine* e, int* more) {
    if (!e || !more) return kvc::set_error(KVC_ERR_ARG, "null engine / out pointer");
    return guard([&]() -> int {
        *more = e->e.step() ? 1 : 0;
        return KVC_OK;
    });
}
int kvc_engine_run(kvc_engine* e, kvc_engine_stats* out) {
    if (!e || !out) return kvc::set_error(KVC_ERR_ARG, "null engine / out pointer");
    return guard([&]() -> int {
        to_c(e->e.run(), out);
        return KVC_OK;
    });
}
int kvc_engine_last_step(const kvc_engine* e, int* n, int* lens, int* tab_off, int* table, int table_cap,
                         int* wpos, int* slots, void** dev) {
    if (!e || !n) return kvc::set_error(KVC_ERR_ARG, "null engine / out pointer");
    return guard([&]() -> int {
        const ModelRunner& r = e->e.runner;
        const int m = (int)r.h_len.size();
        *n = m;
        if (m == 0) return KVC_OK;
        const int T = (int)r.h_tab.size();
        if (!lens || !tab_off || !table || !dev) return kvc::set_error(KVC_ERR_ARG, "null output array");
        if (table_cap < T) return kvc::set_error(KVC_ERR_ARG, "table_cap < " + std::to_string(T));
        std::copy(r.h_len.begin(), r.h_len.end(), lens);
        std::copy(r.h_off.begin(), r.h_off.end(), tab_off);
        std::copy(r.h_tab.begin(), r.h_tab.end(), table);
        if (wpos && slots) {
            for (int i = 0; i < m; ++i) {
                wpos[i] = i < (int)r.h_wpos.size() ? r.h_wpos[i] : -1;
                slots[i] = i < (int)r.h_slot.size() ? r.h_slot[i] : -1;
            }
        }
        const KVCacheManager& kvm = e->e.kvm;
        dev[0] = r.dq; dev[1] = r.dk; dev[2] = r.dv; dev[3] = r.dout;
        dev[4] = kvm.k_layer(0); dev[5] = kvm.v_layer(0);
        return KVC_OK;
    });
}
int kvc_engine_stats_get(const kvc_engine* e, kvc_engine_stats* out) {
    if (!e || !out) return kvc::set_error(KVC_ERR_ARG, "null engine / out pointer");
    to_c(e->e.stats, out);
    return KVC_OK;
}
int kvc_run_static(kvc_engine* e, const kvc_request* reqs, int n, int max_batch, kvc_engine_stats* out) {
    if (!e || !out || (n > 0 && !reqs)) return kvc::set_error(KVC_ERR_ARG, "null argument");
    if (max_batch <= 0 || max_batch > e->e.cfg.max_batch)
        return kvc::set_error(KVC_ERR_ARG, "max_batch must be in [1, engine max_batch]");
    return guard([&]() -> int {
        std::vector<Request> rq((size_t)n);
        for (int i = 0; i < n; ++i) rq[i] = Request{reqs[i].id, reqs[i].arrival_us, reqs[i].prompt_len, reqs[i].gen_len};
        to_c(run_static(rq, e->e.kvm, e->e.runner, max_batch), out);
        return KVC_OK;
    });
}

}  // extern "C"
