// model_abi.cpp -- extern "C" handle over the Qwen2-shaped decoder (include/kvc/qwen_model.h)
// for non-C++ hosts: create with random weights, read a weight tensor's device address
// (the CPU restatement copies the weights from there), serve requests greedily with
// continuous batching, and prefill one prompt returning its last-position logits.
#include <cstring>
#include <exception>
#include <string>

#include "status.hpp"
#include "kvc/qwen_model.h"
#include "kvc_abi.h"

struct kvc_qwen {
    QwenModel m;
    explicit kvc_qwen(const QwenConfig& c) : m(c) {}
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
}  // namespace

extern "C" {

int kvc_qwen_create(const kvc_qwen_config* cfg, kvc_qwen** out) {
    if (!cfg || !out) return kvc::set_error(KVC_ERR_ARG, "null config / out pointer");
    *out = nullptr;
    return guard([&]() -> int {
        QwenConfig c;
        c.layers = cfg->layers; c.hidden = cfg->hidden; c.n_heads = cfg->n_heads; c.n_kv_heads = cfg->n_kv_heads;
        c.head_dim = cfg->head_dim; c.inter = cfg->inter; c.vocab = cfg->vocab;
        c.eps = cfg->eps; c.theta = cfg->theta; c.init_std = cfg->init_std;
        c.block_size = cfg->block_size; c.num_blocks = cfg->num_blocks; c.max_batch = cfg->max_batch;
        c.max_rows = cfg->max_rows;
        if (cfg->seed) c.seed = cfg->seed;
        if (cfg->step_path != 0 && cfg->step_path != 1) return kvc::set_error(KVC_ERR_ARG, "qwen config: step_path 0 or 1");
        c.step_path = cfg->step_path;
        if (cfg->graph != 0 && cfg->graph != 1) return kvc::set_error(KVC_ERR_ARG, "qwen config: graph 0 or 1");
        c.graph = cfg->graph;
        if (cfg->prefill_rows < 0) return kvc::set_error(KVC_ERR_ARG, "qwen config: prefill_rows >= 0");
        if (cfg->prefill_rows > 0) c.prefill_rows = cfg->prefill_rows;
        if (cfg->chain != 0 && cfg->chain != 1) return kvc::set_error(KVC_ERR_ARG, "qwen config: chain 0 or 1");
        c.chain = cfg->chain;
        if (c.layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.inter <= 0 ||
            c.vocab <= 0 || c.block_size <= 0 || c.num_blocks <= 0 || c.max_batch <= 0 || c.max_rows <= 0)
            return kvc::set_error(KVC_ERR_ARG, "qwen config: sizes must be positive");
        *out = new kvc_qwen(c);
        return KVC_OK;
    });
}

void kvc_qwen_destroy(kvc_qwen* h) { delete h; }

int kvc_qwen_tensor(kvc_qwen* h, const char* name, int layer, void** ptr, size_t* bytes) {
    if (!h || !name || !ptr || !bytes) return kvc::set_error(KVC_ERR_ARG, "null argument");
    return guard([&]() -> int {
        const QwenModel& m = h->m;
        const QwenConfig& c = m.c;
        const size_t H = c.hidden, QD = (size_t)c.n_heads * c.head_dim, KD = (size_t)c.n_kv_heads * c.head_dim,
                     I = c.inter;
        const std::string n(name);
        if (n == "embed") { *ptr = m.embed; *bytes = (size_t)c.vocab * H * 2; return KVC_OK; }
        if (n == "norm") { *ptr = m.normf; *bytes = H * 2; return KVC_OK; }
        if (layer < 0 || layer >= c.layers) return kvc::set_error(KVC_ERR_ARG, "layer out of range");
        const QwenModel::Layer& l = m.L[layer];
        struct T { const char* n; void* p; size_t b; };
        const T ts[] = {{"ln1", l.ln1, H * 2}, {"wq", l.wq, QD * H * 2}, {"bq", l.bq, QD * 2},
                        {"wk", l.wk, KD * H * 2}, {"bk", l.bk, KD * 2}, {"wv", l.wv, KD * H * 2},
                        {"bv", l.bv, KD * 2}, {"wo", l.wo, H * QD * 2}, {"ln2", l.ln2, H * 2},
                        {"wg", l.wg, I * H * 2}, {"wu", l.wu, I * H * 2}, {"wd", l.wd, H * I * 2}};
        for (const T& t : ts)
            if (n == t.n) { *ptr = t.p; *bytes = t.b; return KVC_OK; }
        return kvc::set_error(KVC_ERR_ARG, "unknown tensor " + n);
    });
}

int kvc_qwen_serve(kvc_qwen* h, int n_req, const int* prompt_off, const int* prompt_tokens, const int* gen_len,
                   int* out_tokens, kvc_qwen_stats* stats) {
    if (!h || n_req < 0 || (n_req > 0 && (!prompt_off || !prompt_tokens || !gen_len || !out_tokens)))
        return kvc::set_error(KVC_ERR_ARG, "null argument");
    return guard([&]() -> int {
        std::vector<QwenModel::Request> reqs(n_req);
        for (int i = 0; i < n_req; ++i) {
            if (prompt_off[i + 1] < prompt_off[i] || gen_len[i] < 1)
                return kvc::set_error(KVC_ERR_ARG, "bad prompt offsets or generation length");
            reqs[i].prompt.assign(prompt_tokens + prompt_off[i], prompt_tokens + prompt_off[i + 1]);
            reqs[i].gen_len = gen_len[i];
        }
        std::vector<std::vector<int>> out;
        const QwenModel::ServeStats st = h->m.serve(reqs, out);
        size_t o = 0;
        for (int i = 0; i < n_req; ++i) {
            std::memcpy(out_tokens + o, out[i].data(), out[i].size() * sizeof(int));
            o += out[i].size();
        }
        if (stats) {
            stats->steps = st.steps; stats->finished = st.finished; stats->tokens = st.tokens;
            stats->prompt_tokens = st.prompt_tokens; stats->wall_us = st.wall_us; stats->prefill_us = st.prefill_us;
            stats->decode_us = st.decode_us;
            stats->graph_steps = st.graph_steps;
            stats->graph_captures = st.graph_captures;
            stats->chain_launches = st.chain_launches;
        }
        return KVC_OK;
    });
}

int kvc_qwen_load_weights(kvc_qwen* h, const char* dir) {
    if (!h || !dir) return kvc::set_error(KVC_ERR_ARG, "null argument");
    return guard([&]() -> int {
        h->m.load_weights(dir);
        return KVC_OK;
    });
}

int kvc_qwen_save_weights(kvc_qwen* h, const char* dir) {
    if (!h || !dir) return kvc::set_error(KVC_ERR_ARG, "null argument");
    return guard([&]() -> int {
        h->m.save_weights(dir);
        return KVC_OK;
    });
}

int kvc_qwen_prefill_logits(kvc_qwen* h, const int* tokens, int P, float* logits_host, int* token) {
    if (!h || !tokens || P <= 0) return kvc::set_error(KVC_ERR_ARG, "bad argument");
    return guard([&]() -> int {
        QwenModel& m = h->m;
        m.kvm.reset();
        Sequence s;
        s.prompt_len = P;
        if (!m.kvm.allocate_prompt(s)) return kvc::set_error(KVC_ERR_NOMEM, "pool too small for the prompt");
        const int t = m.prefill(s, tokens);
        if (token) *token = t;
        if (logits_host) {
            kvc::check(kvc_memcpy_d2h(logits_host, m.logits, (size_t)m.c.vocab * sizeof(float), m.stream), "logits");
            kvc::check(kvc_stream_synchronize(m.stream), "logits");
        }
        m.kvm.free(s);
        return KVC_OK;
    });
}

}  // extern "C"
