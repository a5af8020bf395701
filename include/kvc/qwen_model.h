// qwen_model.h -- a Qwen2-shaped decoder served with continuous batching over the
// paged KV cache (the model track of the reference, qwen_serve.cu:60-210), built on
// the C ABI: embedding, RMSNorm, biased q/k/v projections, rotary embedding, K/V
// writes into the paged pool, causal prompt attention (prefill) and the planned
// grouped-query decode with the new token's K/V written in the same launch, output
// projection, SwiGLU MLP, residuals, final norm, tied lm_head (fp32 logits) and
// greedy argmax.  Weights are random N(0, init_std) (norm weights 1), generated on
// the device from a seed; activations fp16, arithmetic fp32.
//
// Decode steps of at most 32 rows run five fused kernels per layer (step_path 0):
// RMSNorm + q/k/v projection + bias + rotary; the planned attention with the new
// K/V written in the same launch; output projection + residual; RMSNorm + gate/up
// projection + SwiGLU; down projection + residual; then final norm + lm_head +
// argmax.  step_path 1 (and larger batches, and prompts) run one kernel per op with
// rocBLAS linear layers; both round to fp16 at the same points.  With `graph` the
// fused step is captured once as a HIP graph whose kernels read the step's counts
// (rows, attention units, partial records) from device memory; each step then
// uploads its metadata into fixed places and replays the graph (the reference
// captures its single-sequence decode step, qwen_infer.cu:135-214).
//
// Greedy serving (QwenModel::serve): requests are admitted FIFO up to max_batch
// running sequences; the prompts admitted together are prefilled together (their
// rows stacked into one forward, up to prefill_rows rows; each request's first token
// comes from its prompt's last position), then every step decodes one token for
// every running sequence; a sequence retires after gen_len tokens.
#pragma once
#include <algorithm>
#include <chrono>
#include <cstring>
#include <deque>
#include <fstream>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "../kvc_abi.h"
#include "kv_cache_manager.h"
#include "sequence.h"

struct QwenConfig {
    int layers = 24, hidden = 896, n_heads = 14, n_kv_heads = 2, head_dim = 64, inter = 4864, vocab = 151936;
    float eps = 1e-6f, theta = 1e6f, init_std = 0.02f;
    int block_size = 16, num_blocks = 10922, max_batch = 32, max_rows = 1024;  // max_rows: prompt rows per prefill
    uint64_t seed = 0x71776e32ull;
    int step_path = 0;  // 0: fused kernels for steps of <= 32 rows; 1: one kernel per op
    int graph = 0;      // 1: fused steps replay one captured HIP graph (measured no faster than eager)
    int prefill_rows = 4096;  // prompt rows stacked into one prefill forward (a longer prompt runs alone)
    int chain = 0;  // eager fused steps: 1 runs the linear layers between two attention launches as one
                    // persistent launch (kvc_rows_chain) where the device and shapes allow; 0 one launch each
                    // (the default: ~1% faster per step measured, and it holds a grid barrier)
};

struct QwenModel {
    struct Layer {
        void *ln1, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *ln2, *wg, *wu, *wd;  // wq|wk|wv, bq|bk|bv, wg|wu adjacent
    };
    static constexpr int kRowsMax = 32;  // rows of the fused decode-step kernels
    QwenConfig c;
    KVCacheManager kvm;
    kvc_stream_t stream = nullptr;
    std::vector<void*> owned;
    void *embed = nullptr, *normf = nullptr;
    void* lm_head = nullptr;  // nullptr: tied to the embedding
    const void* lm_w() const { return lm_head ? lm_head : embed; }
    std::vector<Layer> L;
    // activations for up to max(max_rows, max_batch) rows
    void *x = nullptr, *nrm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *o = nullptr,
         *gate = nullptr, *up = nullptr;
    float* logits = nullptr;
    int* d_meta = nullptr;
    int* h_meta = nullptr;
    size_t meta_cap = 0;
    int* d_tok = nullptr;  // argmax results
    int* h_tok = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* rws = nullptr;  // fused kernels' workspace (zero between calls)
    size_t rws_bytes = 0;
    bool rows_ok = false;
    void* cws = nullptr;  // layer chain's workspace (its own: barrier counters persist between launches)
    size_t cws_bytes = 0;
    bool chain_ok = false;
    long long chain_launches = 0;
    // graph-replayed steps: metadata at fixed places,
    // [n, units, records, 0 | ids B | pos B | work cap_units*ipu | table cap_tab]
    void* gexec = nullptr;
    bool graph_failed = false;
    const void* g_ws = nullptr;  // the workspace and pools the captured graph holds
    const void* g_pools[2] = {nullptr, nullptr};
    int* d_g = nullptr;
    int* h_g = nullptr;
    int g_cap_units = 0, g_cap_tab = 0, g_ipu = 0;
    size_t g_off_work = 0, g_off_tab = 0;
    long long graph_steps = 0, graph_captures = 0;
    std::vector<int> h_work, h_tab, h_off, h_len;

    explicit QwenModel(const QwenConfig& cfg)
        : c(cfg), kvm(cfg.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, KVC_F16, cfg.layers) {
        if (c.hidden % 8 || c.inter % 8 || (c.n_heads * c.head_dim) % 8 || (c.n_kv_heads * c.head_dim) % 8 ||
            c.n_heads % c.n_kv_heads)
            throw kvc::Error(KVC_ERR_ARG, "QwenModel: unsupported shape");
        kvc::check(kvc_stream_create(&stream), "stream");
        const int H = c.hidden, QD = c.n_heads * c.head_dim, KD = c.n_kv_heads * c.head_dim, I = c.inter;
        uint64_t s = c.seed;
        auto fill = [&](void* p, size_t n) {
            kvc::check(kvc_fill_normal(p, n, KVC_F16, s++, c.init_std, stream), "init");
            return p;
        };
        auto param = [&](size_t n, bool ones = false) {
            void* p = alloc(n * 2);
            if (ones) fill_ones(p, n);
            else fill(p, n);
            return p;
        };
        auto at = [](void* p, size_t elems) { return static_cast<void*>(static_cast<char*>(p) + elems * 2); };
        embed = param((size_t)c.vocab * H);
        L.resize(c.layers);
        for (auto& l : L) {
            l.ln1 = param(H, true);
            void* wqkv = alloc((size_t)(QD + 2 * KD) * H * 2);
            void* bqkv = alloc((size_t)(QD + 2 * KD) * 2);
            l.wq = fill(wqkv, (size_t)QD * H); l.bq = fill(bqkv, QD);
            l.wk = fill(at(wqkv, (size_t)QD * H), (size_t)KD * H); l.bk = fill(at(bqkv, QD), KD);
            l.wv = fill(at(wqkv, (size_t)(QD + KD) * H), (size_t)KD * H); l.bv = fill(at(bqkv, QD + KD), KD);
            l.wo = param((size_t)H * QD);
            l.ln2 = param(H, true);
            void* wgu = alloc((size_t)2 * I * H * 2);
            l.wg = fill(wgu, (size_t)I * H); l.wu = fill(at(wgu, (size_t)I * H), (size_t)I * H);
            l.wd = param((size_t)H * I);
        }
        normf = param(H, true);
        const size_t R = std::max({c.max_rows, c.max_batch, c.prefill_rows});
        x = alloc(R * H * 2); nrm = alloc(R * H * 2); o = alloc(R * H * 2);
        q = alloc(R * QD * 2); att = alloc(R * QD * 2); k = alloc(R * KD * 2); v = alloc(R * KD * 2);
        gate = alloc(R * I * 2); up = alloc(R * I * 2);
        logits = static_cast<float*>(alloc((size_t)c.max_batch * c.vocab * 4));
        d_tok = static_cast<int*>(alloc(c.max_batch * 4));
        kvc::check(kvc_host_alloc((void**)&h_tok, c.max_batch * 4), "pinned tokens");
        rows_ok = c.step_path == 0 && H % 32 == 0 && H <= 1024 && QD % 32 == 0 && I % 32 == 0 &&
                  c.vocab % 32 == 0 && c.head_dim % 32 == 0;
        if (rows_ok) {
            rws_bytes = std::max({kvc_rows_workspace_size(H, QD), kvc_rows_workspace_size(H, I),
                                  kvc_rows_workspace_size(c.vocab, H)});
            rws = alloc(rws_bytes);
            kvc::check(kvc_memset(rws, 0, rws_bytes, stream), "rows workspace");
            cws_bytes = c.chain == 1 ? kvc_rows_chain_workspace_size(H, I) : 0;
            if (cws_bytes) {
                cws = alloc(cws_bytes);
                kvc::check(kvc_memset(cws, 0, cws_bytes, stream), "chain workspace");
                chain_ok = true;
            }
        }
        kvc::check(kvc_stream_synchronize(stream), "init");
    }
    ~QwenModel() {
        if (stream) kvc_stream_synchronize(stream);
        kvc_graph_destroy(gexec);
        kvc_free(d_g); kvc_host_free(h_g);
        for (void* p : owned) kvc_free(p);
        kvc_free(d_meta); kvc_free(ws);
        kvc_host_free(h_meta); kvc_host_free(h_tok);
        kvc_stream_destroy(stream);
    }
    QwenModel(const QwenModel&) = delete;
    QwenModel& operator=(const QwenModel&) = delete;

    void* alloc(size_t bytes) {
        void* p = nullptr;
        kvc::check(kvc_malloc(&p, (bytes + 255) / 256 * 256), "model allocation");
        owned.push_back(p);
        return p;
    }
    void fill_ones(void* p, size_t n) {
        std::vector<uint16_t> h(n, 0x3C00);  // fp16 1.0
        kvc::check(kvc_memcpy_h2d(p, h.data(), n * 2, stream), "ones");
        kvc::check(kvc_stream_synchronize(stream), "ones");
    }
    void ensure_meta(size_t ints) {
        if (ints <= meta_cap) return;
        kvc::check(kvc_stream_synchronize(stream), "meta growth");
        kvc_free(d_meta); kvc_host_free(h_meta);
        d_meta = nullptr; h_meta = nullptr;
        meta_cap = std::max(ints, meta_cap * 2);
        kvc::check(kvc_malloc((void**)&d_meta, meta_cap * 4), "meta");
        kvc::check(kvc_host_alloc((void**)&h_meta, meta_cap * 4), "pinned meta");
    }
    // Grows the split-K workspace.  A captured step graph holds the old address, so
    // it is destroyed here and captured again by the next decode step.
    void ensure_ws(size_t need) {
        if (need <= ws_bytes) return;
        kvc::check(kvc_stream_synchronize(stream), "workspace growth");
        if (gexec) {
            kvc_graph_destroy(gexec);
            gexec = nullptr;
            g_ws = nullptr;
        }
        kvc_free(ws);
        ws = nullptr;
        ws_bytes = std::max(need, (size_t)1 << 20) * 2;
        kvc::check(kvc_malloc(&ws, ws_bytes), "workspace");
    }
    void* kl(int l) const { return kvm.k_layer(l); }
    void* vl(int l) const { return kvm.v_layer(l); }

    // Rows [0, M) of x hold the layer input; attention is supplied by `attend(l)`.
    template <typename Attend>
    void layers(int M, const int* d_pos, int pos_base, Attend&& attend) {
        const int H = c.hidden, QD = c.n_heads * c.head_dim, KD = c.n_kv_heads * c.head_dim, I = c.inter;
        for (int l = 0; l < c.layers; ++l) {
            const Layer& w = L[l];
            kvc::check(kvc_rmsnorm(nrm, x, w.ln1, M, H, c.eps, stream), "rmsnorm");
            kvc::check(kvc_linear(q, nrm, w.wq, M, QD, H, KVC_F16, stream), "q_proj");
            kvc::check(kvc_add_bias(q, w.bq, M, QD, stream), "q bias");
            kvc::check(kvc_linear(k, nrm, w.wk, M, KD, H, KVC_F16, stream), "k_proj");
            kvc::check(kvc_add_bias(k, w.bk, M, KD, stream), "k bias");
            kvc::check(kvc_linear(v, nrm, w.wv, M, KD, H, KVC_F16, stream), "v_proj");
            kvc::check(kvc_add_bias(v, w.bv, M, KD, stream), "v bias");
            kvc::check(kvc_rope(q, d_pos, pos_base, M, c.n_heads, c.head_dim, c.theta, stream), "rope q");
            kvc::check(kvc_rope(k, d_pos, pos_base, M, c.n_kv_heads, c.head_dim, c.theta, stream), "rope k");
            attend(l);
            kvc::check(kvc_linear(o, att, w.wo, M, H, QD, KVC_F16, stream), "o_proj");
            kvc::check(kvc_add_residual(x, o, (size_t)M * H, stream), "residual");
            kvc::check(kvc_rmsnorm(nrm, x, w.ln2, M, H, c.eps, stream), "rmsnorm");
            kvc::check(kvc_linear(gate, nrm, w.wg, M, I, H, KVC_F16, stream), "gate_proj");
            kvc::check(kvc_linear(up, nrm, w.wu, M, I, H, KVC_F16, stream), "up_proj");
            kvc::check(kvc_silu_mul(gate, gate, up, (size_t)M * I, stream), "silu");
            kvc::check(kvc_linear(o, gate, w.wd, M, H, I, KVC_F16, stream), "down_proj");
            kvc::check(kvc_add_residual(x, o, (size_t)M * H, stream), "residual");
        }
    }

    // Decode-step layers over M <= 32 rows with the fused kernels.  With d_counts
    // (graph capture) M, T, nu and nr are capacities and the step's counts are read
    // from d_counts = {rows, units, records} in device memory.
    void rows_layers(int M, const int* d_pos, const int* d_table, int T, const int* d_work, int nu, int nr,
                     const int* d_counts = nullptr) {
        const int* d_rows = d_counts;
        const int H = c.hidden, QD = c.n_heads * c.head_dim, I = c.inter;
        const float scale = 1.0f / __builtin_sqrtf((float)c.head_dim);
        if (chain_ok && !d_counts && chain_layers(M, d_pos, d_table, T, d_work, nu, nr, scale)) return;
        for (int l = 0; l < c.layers; ++l) {
            const Layer& w = L[l];
            kvc::check(kvc_rows_qkv(q, k, v, x, w.ln1, c.eps, w.wq, w.bq, d_pos, M, H, c.n_heads, c.n_kv_heads,
                                    c.head_dim, c.theta, d_rows, stream),
                       "norm + qkv + rope");
            if (d_counts)
                kvc::check(kvc_batched_paged_decode_planned_dev(q, k, v, d_pos, kl(l), vl(l), d_table, T, att, M,
                                                                c.n_heads, c.n_kv_heads, c.head_dim, c.block_size,
                                                                scale, KVC_F16, d_work, nu, nr, d_counts, ws,
                                                                ws_bytes, stream),
                           "decode attention");
            else
                kvc::check(kvc_batched_paged_append_decode_planned(q, k, v, d_pos, kl(l), vl(l), d_table, T, att, M,
                                                                   c.n_heads, c.n_kv_heads, c.head_dim, c.block_size,
                                                                   scale, KVC_F16, d_work, nu, nr, ws, ws_bytes,
                                                                   stream),
                           "decode attention");
            kvc::check(kvc_rows_linear(x, att, w.wo, M, H, QD, nullptr, 0.f, 1, d_rows, rws, rws_bytes, stream),
                       "o_proj + residual");
            kvc::check(kvc_rows_swiglu(gate, x, w.ln2, c.eps, w.wg, M, I, H, d_rows, stream),
                       "norm + gate/up + swiglu");
            kvc::check(kvc_rows_linear(x, gate, w.wd, M, H, I, nullptr, 0.f, 1, d_rows, rws, rws_bytes, stream),
                       "down_proj + residual");
        }
    }

    // The same layers with the linear layers between two attention launches as one
    // launch (kvc_rows_chain): the head of layer 0, then per layer the attention and
    // one launch with that layer's tail and the next layer's head.  Returns false (and
    // turns the chain off) when the device or shapes do not allow it; it then launched
    // nothing.
    bool chain_layers(int M, const int* d_pos, const int* d_table, int T, const int* d_work, int nu, int nr,
                      float scale) {
        kvc_layer_chain ch{};
        ch.M = M; ch.H = c.hidden; ch.Hq = c.n_heads; ch.Hkv = c.n_kv_heads; ch.D = c.head_dim; ch.I = c.inter;
        ch.eps = c.eps; ch.theta = c.theta;
        ch.x = x; ch.att = att; ch.act = gate; ch.q = q; ch.k = k; ch.v = v; ch.pos = d_pos;
        auto set_head = [&](int l) {
            ch.ln1 = l < c.layers ? L[l].ln1 : nullptr;
            ch.w_qkv = l < c.layers ? L[l].wq : nullptr;
            ch.b_qkv = l < c.layers ? L[l].bq : nullptr;
        };
        set_head(0);
        const int rc = kvc_rows_chain(&ch, cws, cws_bytes, stream);
        if (rc == KVC_ERR_UNSUPPORTED) {
            chain_ok = false;
            return false;
        }
        kvc::check(rc, "layer chain");
        ++chain_launches;
        for (int l = 0; l < c.layers; ++l) {
            kvc::check(kvc_batched_paged_append_decode_planned(q, k, v, d_pos, kl(l), vl(l), d_table, T, att, M,
                                                               c.n_heads, c.n_kv_heads, c.head_dim, c.block_size,
                                                               scale, KVC_F16, d_work, nu, nr, ws, ws_bytes, stream),
                       "decode attention");
            const Layer& w = L[l];
            ch.w_o = w.wo; ch.ln2 = w.ln2; ch.w_gate_up = w.wg; ch.w_down = w.wd;
            set_head(l + 1);
            kvc::check(kvc_rows_chain(&ch, cws, cws_bytes, stream), "layer chain");
            ++chain_launches;
        }
        return true;
    }

    // Final norm of `rows` rows starting at x row `first` (consecutive), fp32 logits
    // (optional on the fused path), argmax.  d_rows_head: the row count in device
    // memory (graph capture; `rows` is then the capacity).
    void head(int first, int rows, bool want_logits = true, const int* d_rows_head = nullptr) {
        head_rows(static_cast<const char*>(x) + (size_t)first * c.hidden * 2, rows, want_logits, d_rows_head);
    }
    void head_rows(const void* xr, int rows, bool want_logits = true, const int* d_rows_head = nullptr) {
        const int H = c.hidden;
        if (rows_ok && rows <= kRowsMax) {
            kvc::check(kvc_rows_lm_head(want_logits ? logits : nullptr, d_tok, xr, normf, c.eps, lm_w(), rows, c.vocab,
                                        H, d_rows_head, rws, rws_bytes, stream),
                       "final norm + lm_head + argmax");
            return;
        }
        kvc::check(kvc_rmsnorm(nrm, xr, normf, rows, H, c.eps, stream), "final norm");
        kvc::check(kvc_linear(logits, nrm, lm_w(), rows, c.vocab, H, KVC_F32, stream), "lm_head");
        kvc::check(kvc_argmax(logits, rows, c.vocab, d_tok, stream), "argmax");
    }

    // Prompt processing of several admitted sequences in one forward: their rows are
    // stacked (row r of prompt i at position r), the K/V of every row go to its slot,
    // and the last row of each prompt gives its first token (first[i]).  Causal
    // attention over all prompts is one planned decode launch per layer: row r of
    // prompt i is a query of length r + 1 over prompt i's table (the causal form of
    // qwen_kernels.cu:146-181), planned once for the batch.  Rows are independent in
    // every op but attention, so each prompt's result is that of prefill() up to fp32
    // summation order.
    void prefill_batch(const std::vector<Sequence*>& ss, const std::vector<const int*>& toks, int* first) {
        const int n = (int)ss.size();
        if (n == 0) return;
        if (n > c.max_batch) throw kvc::Error(KVC_ERR_ARG, "prefill_batch: more prompts than max_batch");
        std::vector<int> off(n + 1, 0), toff(n + 1, 0);
        for (int i = 0; i < n; ++i) {
            const int P = ss[i]->prompt_len;
            if (P <= 0) throw kvc::Error(KVC_ERR_ARG, "prefill_batch: empty prompt");
            off[i + 1] = off[i] + P;
            toff[i + 1] = toff[i] + (int)ss[i]->block_table.size();
        }
        const int R = off[n];
        if (R > std::max({c.max_rows, c.max_batch, c.prefill_rows}))
            throw kvc::Error(KVC_ERR_ARG, "prefill_batch: more rows than the activation buffers hold");
        // the causal plan: row r of prompt i attends over r + 1 positions of table i
        const int T = toff[n];
        h_len.resize(R); h_off.resize(R); h_tab.resize(T);
        for (int i = 0; i < n; ++i) {
            std::memcpy(h_tab.data() + toff[i], ss[i]->block_table.data(), ss[i]->block_table.size() * 4);
            for (int r = 0; r < ss[i]->prompt_len; ++r) {
                h_len[off[i] + r] = r + 1;
                h_off[off[i] + r] = toff[i];
            }
        }
        int nu = 0, nr = 0;
        kvc::check(kvc_decode_plan(h_len.data(), h_off.data(), h_tab.data(), T, R, c.n_heads, c.n_kv_heads,
                                   c.head_dim, c.block_size, KVC_F16, 0, nullptr, 0, &nu, &nr),
                   "prefill plan");
        const int ipu = kvc_decode_plan_entry_ints(c.n_heads, c.n_kv_heads, c.head_dim, c.block_size, KVC_F16);
        h_work.resize((size_t)nu * ipu);
        kvc::check(kvc_decode_plan(h_len.data(), h_off.data(), h_tab.data(), T, R, c.n_heads, c.n_kv_heads,
                                   c.head_dim, c.block_size, KVC_F16, 0, h_work.data(), nu, &nu, &nr),
                   "prefill plan");
        // upload: [ids R | pos R | slot R | last n | tables T | work]
        const size_t ints = 3 * (size_t)R + n + T + h_work.size();
        ensure_meta(ints);
        kvc::check(kvc_stream_synchronize(stream), "meta reuse");
        int* h = h_meta;
        for (int i = 0; i < n; ++i) {
            const Sequence& s = *ss[i];
            const int P = s.prompt_len;
            std::memcpy(h + off[i], toks[i], P * 4);
            for (int r = 0; r < P; ++r) {
                h[R + off[i] + r] = r;
                h[2 * R + off[i] + r] = s.block_table[r / c.block_size] * c.block_size + r % c.block_size;
            }
            h[3 * R + i] = off[i + 1] - 1;
        }
        std::memcpy(h + 3 * R + n, h_tab.data(), (size_t)T * 4);
        std::memcpy(h + 3 * R + n + T, h_work.data(), h_work.size() * 4);
        kvc::check(kvc_step_upload(d_meta, h, ints * 4, stream), "prefill upload");
        const int* d_ids = d_meta;
        const int* d_pos = d_meta + R;
        const int* d_slot = d_meta + 2 * R;
        const int* d_last = d_meta + 3 * R;
        const int* d_tabs = d_meta + 3 * R + n;
        const int* d_work = d_tabs + T;
        ensure_ws(kvc_decode_planned_workspace_size(c.n_heads, c.n_kv_heads, c.head_dim, c.block_size, KVC_F16, nr));
        kvc::check(kvc_embed_gather(x, embed, d_ids, R, c.hidden, c.vocab, stream), "embed");
        const float scale = 1.0f / __builtin_sqrtf((float)c.head_dim);
        layers(R, d_pos, 0, [&](int l) {
            kvc::check(kvc_write_kv_slots(k, v, kl(l), vl(l), d_slot, R, c.n_kv_heads, c.head_dim, c.block_size,
                                          KVC_F16, stream),
                       "prefill write_kv");
            kvc::check(kvc_batched_paged_decode_planned(q, kl(l), vl(l), d_tabs, T, att, R, c.n_heads, c.n_kv_heads,
                                                        c.head_dim, c.block_size, scale, KVC_F16, d_work, nu, nr, ws,
                                                        ws_bytes, stream),
                       "prefill attention");
        });
        // the last row of every prompt, gathered, through the head
        kvc::check(kvc_embed_gather(o, x, d_last, n, c.hidden, R, stream), "last rows");
        head_rows(o, n, false);
        kvc::check(kvc_memcpy_d2h(h_tok, d_tok, n * 4, stream), "tokens");
        kvc::check(kvc_stream_synchronize(stream), "prefill");
        std::memcpy(first, h_tok, n * 4);
    }

    // Prompt processing of one admitted sequence (kvm.allocate_prompt done): writes the
    // prompt's K/V for every layer and returns the first generated token.
    int prefill(const Sequence& s, const int* tokens) {
        const int P = s.prompt_len;
        if (P <= 0 || P > c.max_rows) throw kvc::Error(KVC_ERR_ARG, "prefill: prompt length outside [1, max_rows]");
        const int nb = (int)s.block_table.size();
        ensure_meta((size_t)P + nb);
        kvc::check(kvc_stream_synchronize(stream), "meta reuse");
        std::memcpy(h_meta, tokens, P * 4);
        std::memcpy(h_meta + P, s.block_table.data(), nb * 4);
        kvc::check(kvc_step_upload(d_meta, h_meta, ((size_t)P + nb) * 4, stream), "prefill upload");
        const int* d_ids = d_meta;
        const int* d_table = d_meta + P;
        ensure_ws(kvc_paged_causal_attn_workspace_size(0, P, c.n_heads, c.n_kv_heads, c.head_dim, c.block_size,
                                                       KVC_F16));
        kvc::check(kvc_embed_gather(x, embed, d_ids, P, c.hidden, c.vocab, stream), "embed");
        const float scale = 1.0f / __builtin_sqrtf((float)c.head_dim);
        layers(P, nullptr, 0, [&](int l) {
            kvc::check(kvc_write_kv(k, v, kl(l), vl(l), d_table, 0, P, c.n_kv_heads, c.head_dim, c.block_size,
                                    KVC_F16, stream),
                       "prefill write_kv");
            kvc::check(kvc_paged_causal_attn(q, att, kl(l), vl(l), d_table, 0, P, c.n_heads, c.n_kv_heads,
                                             c.head_dim, c.block_size, scale, KVC_F16, ws, ws_bytes, stream),
                       "prefill attention");
        });
        head(P - 1, 1);
        kvc::check(kvc_memcpy_d2h(h_tok, d_tok, 4, stream), "token");
        kvc::check(kvc_stream_synchronize(stream), "prefill");
        return h_tok[0];
    }

    // One decode step: row r feeds token in[r] of batch[r] at position cur_len (the
    // manager has already grown the sequence by that token); returns next tokens.
    void decode(const std::vector<Sequence*>& batch, const int* in, int* out) {
        const int n = (int)batch.size();
        if (n == 0) return;
        if (n > c.max_batch) throw kvc::Error(KVC_ERR_ARG, "decode: batch larger than max_batch");
        h_tab.clear(); h_off.clear(); h_len.clear();
        for (const Sequence* s : batch) {
            h_off.push_back((int)h_tab.size());
            h_tab.insert(h_tab.end(), s->block_table.begin(), s->block_table.end());
            h_len.push_back(s->cur_len);
        }
        h_off.push_back((int)h_tab.size());
        const int T = (int)h_tab.size();
        int nu = 0, nr = 0;
        kvc::check(kvc_decode_plan(h_len.data(), h_off.data(), h_tab.data(), T, n, c.n_heads, c.n_kv_heads,
                                   c.head_dim, c.block_size, KVC_F16, 0, nullptr, 0, &nu, &nr),
                   "plan");
        const int ipu = kvc_decode_plan_entry_ints(c.n_heads, c.n_kv_heads, c.head_dim, c.block_size, KVC_F16);
        h_work.resize((size_t)nu * ipu);
        kvc::check(kvc_decode_plan(h_len.data(), h_off.data(), h_tab.data(), T, n, c.n_heads, c.n_kv_heads,
                                   c.head_dim, c.block_size, KVC_F16, 0, h_work.data(), nu, &nu, &nr),
                   "plan");
        if (rows_ok && c.graph && n <= kRowsMax && ensure_graph() && nu <= g_cap_units && nr <= g_cap_units &&
            T <= g_cap_tab) {
            decode_graph(n, in, T, nu, nr, ipu, out);
            return;
        }
        // upload: [ids n | pos n | table T | work]
        const size_t ints = 2 * (size_t)n + T + h_work.size();
        ensure_meta(ints);
        kvc::check(kvc_stream_synchronize(stream), "meta reuse");
        std::memcpy(h_meta, in, n * 4);
        for (int r = 0; r < n; ++r) h_meta[n + r] = h_len[r] - 1;  // the new token's position
        std::memcpy(h_meta + 2 * n, h_tab.data(), (size_t)T * 4);
        std::memcpy(h_meta + 2 * n + T, h_work.data(), h_work.size() * 4);
        kvc::check(kvc_step_upload(d_meta, h_meta, ints * 4, stream), "decode upload");
        const int* d_ids = d_meta;
        const int* d_pos = d_meta + n;
        const int* d_table = d_meta + 2 * n;
        const int* d_work = d_table + T;
        ensure_ws(kvc_decode_planned_workspace_size(c.n_heads, c.n_kv_heads, c.head_dim, c.block_size, KVC_F16, nr));
        kvc::check(kvc_embed_gather(x, embed, d_ids, n, c.hidden, c.vocab, stream), "embed");
        const float scale = 1.0f / __builtin_sqrtf((float)c.head_dim);
        if (rows_ok && n <= kRowsMax) {
            rows_layers(n, d_pos, d_table, T, d_work, nu, nr);
        } else {
            layers(n, d_pos, 0, [&](int l) {
                kvc::check(kvc_batched_paged_append_decode_planned(q, k, v, d_pos, kl(l), vl(l), d_table, T, att, n,
                                                                   c.n_heads, c.n_kv_heads, c.head_dim, c.block_size,
                                                                   scale, KVC_F16, d_work, nu, nr, ws, ws_bytes,
                                                                   stream),
                           "decode attention");
            });
        }
        head(0, n, false);
        kvc::check(kvc_memcpy_d2h(h_tok, d_tok, n * 4, stream), "tokens");
        kvc::check(kvc_stream_synchronize(stream), "decode");
        std::memcpy(out, h_tok, n * 4);
    }

    // The captured step: capacities fixed here, counts and metadata per step in d_g.
    bool ensure_graph() {
        if (gexec) return true;
        if (graph_failed) return false;
        const int B = c.max_batch;
        if (B > kRowsMax) { graph_failed = true; return false; }
        g_ipu = kvc_decode_plan_entry_ints(c.n_heads, c.n_kv_heads, c.head_dim, c.block_size, KVC_F16);
        // the planner's bound for B sequences over the whole pool; tables: the whole pool
        kvc::check(kvc_decode_plan_capacity(B, (long long)c.num_blocks * c.block_size, c.n_heads, c.n_kv_heads,
                                            c.head_dim, c.block_size, KVC_F16, &g_cap_units),
                   "plan capacity");
        g_cap_tab = c.num_blocks;
        g_off_work = 4 + 2 * (size_t)B;
        g_off_tab = g_off_work + (size_t)g_cap_units * g_ipu;
        const size_t ints = g_off_tab + g_cap_tab;
        if (!d_g) {  // kept across captures (a workspace growth makes the next step capture again)
            kvc::check(kvc_malloc((void**)&d_g, ints * 4), "graph metadata");
            kvc::check(kvc_host_alloc((void**)&h_g, ints * 4), "pinned graph metadata");
        }
        kvc::check(kvc_memset(d_g, 0, ints * 4, stream), "graph metadata");  // zero counts: an idle replay
        ensure_ws(kvc_decode_planned_workspace_size(c.n_heads, c.n_kv_heads, c.head_dim, c.block_size, KVC_F16,
                                                    g_cap_units));
        kvc::check(kvc_stream_synchronize(stream), "graph setup");
        const int* d_counts = d_g;
        const int* d_ids = d_g + 4;
        const int* d_pos = d_ids + B;
        const int* d_work = d_g + g_off_work;
        const int* d_table = d_g + g_off_tab;
        kvc::check(kvc_graph_begin(stream), "graph capture");
        try {
            kvc::check(kvc_embed_gather_dev(x, embed, d_ids, d_counts, B, c.hidden, c.vocab, stream), "embed");
            rows_layers(B, d_pos, d_table, g_cap_tab, d_work, g_cap_units, g_cap_units, d_counts);
            head(0, B, false, d_counts);
        } catch (...) {
            void* partial = nullptr;
            kvc_graph_end(stream, &partial);
            kvc_graph_destroy(partial);
            graph_failed = true;
            throw;
        }
        kvc::check(kvc_graph_end(stream, &gexec), "graph instantiate");
        ++graph_captures;
        g_ws = ws;
        g_pools[0] = kl(0);
        g_pools[1] = vl(0);
        return true;
    }

    void decode_graph(int n, const int* in, int T, int nu, int nr, int ipu, int* out) {
        if (ws != g_ws || kl(0) != g_pools[0] || vl(0) != g_pools[1])
            throw kvc::Error(KVC_ERR_STATE, "decode_graph: workspace or pools differ from those the graph captured");
        const int B = c.max_batch;
        int* h = h_g;
        h[0] = n; h[1] = nu; h[2] = nr; h[3] = 0;
        std::memcpy(h + 4, in, n * 4);
        for (int r = 0; r < n; ++r) h[4 + B + r] = h_len[r] - 1;  // the new token's position
        std::memcpy(h + g_off_work, h_work.data(), (size_t)nu * ipu * 4);
        std::memcpy(h + g_off_tab, h_tab.data(), (size_t)T * 4);
        kvc::check(kvc_step_upload(d_g, h, (g_off_work + (size_t)nu * ipu) * 4, stream), "step upload");
        kvc::check(kvc_step_upload(d_g + g_off_tab, h + g_off_tab, (size_t)T * 4, stream), "table upload");
        kvc::check(kvc_graph_launch(gexec, stream), "graph launch");
        kvc::check(kvc_memcpy_d2h(h_tok, d_tok, n * 4, stream), "tokens");
        kvc::check(kvc_stream_synchronize(stream), "decode");
        std::memcpy(out, h_tok, n * 4);
        ++graph_steps;
    }

    // ---- weights in the reference's dump format (qwen_loader.h:21-76, written by
    // tools/dump_weights.py:29-66): manifest.tsv lines "name<TAB>offset<TAB>nbytes<TAB>
    // shape_csv" over weights.bin, fp16 row-major [out, in], Hugging Face names.
    struct WeightRef {
        std::string name;
        void* dst;
        std::vector<int> shape;
    };
    std::vector<WeightRef> weight_refs() {
        const int H = c.hidden, QD = c.n_heads * c.head_dim, KD = c.n_kv_heads * c.head_dim, I = c.inter;
        std::vector<WeightRef> w{{"model.embed_tokens.weight", embed, {c.vocab, H}}};
        for (int l = 0; l < c.layers; ++l) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            const Layer& y = L[l];
            w.push_back({p + "input_layernorm.weight", y.ln1, {H}});
            w.push_back({p + "self_attn.q_proj.weight", y.wq, {QD, H}});
            w.push_back({p + "self_attn.q_proj.bias", y.bq, {QD}});
            w.push_back({p + "self_attn.k_proj.weight", y.wk, {KD, H}});
            w.push_back({p + "self_attn.k_proj.bias", y.bk, {KD}});
            w.push_back({p + "self_attn.v_proj.weight", y.wv, {KD, H}});
            w.push_back({p + "self_attn.v_proj.bias", y.bv, {KD}});
            w.push_back({p + "self_attn.o_proj.weight", y.wo, {H, QD}});
            w.push_back({p + "post_attention_layernorm.weight", y.ln2, {H}});
            w.push_back({p + "mlp.gate_proj.weight", y.wg, {I, H}});
            w.push_back({p + "mlp.up_proj.weight", y.wu, {I, H}});
            w.push_back({p + "mlp.down_proj.weight", y.wd, {H, I}});
        }
        w.push_back({"model.norm.weight", normf, {H}});
        return w;
    }
    static size_t elems(const std::vector<int>& s) {
        size_t n = 1;
        for (int d : s) n *= (size_t)d;
        return n;
    }

    // Loads every tensor of the model from `dir` (sizes and shapes must match the
    // configuration; other entries are ignored).  lm_head.weight, when present and
    // different from the embedding, becomes an untied output matrix.
    void load_weights(const std::string& dir) {
        struct Entry { size_t off, nbytes; std::vector<int> shape; };
        std::unordered_map<std::string, Entry> man;
        std::ifstream mf(dir + "/manifest.tsv");
        if (!mf) throw kvc::Error(KVC_ERR_ARG, "load_weights: cannot open " + dir + "/manifest.tsv");
        std::string line;
        size_t end = 0;
        while (std::getline(mf, line)) {
            if (line.empty()) continue;
            std::istringstream ss(line);
            std::string name, off, nb, shape;
            if (!std::getline(ss, name, '\t') || !std::getline(ss, off, '\t') || !std::getline(ss, nb, '\t'))
                throw kvc::Error(KVC_ERR_ARG, "load_weights: malformed manifest line: " + line);
            std::getline(ss, shape);
            Entry e{std::stoull(off), std::stoull(nb), {}};
            std::stringstream sc(shape);
            for (std::string d; std::getline(sc, d, ',');)
                if (!d.empty()) e.shape.push_back(std::stoi(d));
            end = std::max(end, e.off + e.nbytes);
            man[name] = e;
        }
        std::ifstream bf(dir + "/weights.bin", std::ios::binary | std::ios::ate);
        if (!bf) throw kvc::Error(KVC_ERR_ARG, "load_weights: cannot open " + dir + "/weights.bin");
        if ((size_t)bf.tellg() < end) throw kvc::Error(KVC_ERR_ARG, "load_weights: weights.bin shorter than the manifest");
        const size_t chunk = (size_t)64 << 20;
        char* stage = nullptr;
        kvc::check(kvc_host_alloc((void**)&stage, chunk), "pinned staging");
        auto read_into = [&](const Entry& e, void* dst) {
            for (size_t done = 0; done < e.nbytes; done += chunk) {
                const size_t n = std::min(chunk, e.nbytes - done);
                bf.seekg((std::streamoff)(e.off + done));
                bf.read(stage, (std::streamsize)n);
                if (!bf) throw kvc::Error(KVC_ERR_ARG, "load_weights: read failed");
                kvc::check(kvc_memcpy_h2d(static_cast<char*>(dst) + done, stage, n, stream), "weights upload");
                kvc::check(kvc_stream_synchronize(stream), "weights upload");
            }
        };
        try {
            for (const WeightRef& w : weight_refs()) {
                const auto it = man.find(w.name);
                if (it == man.end()) throw kvc::Error(KVC_ERR_ARG, "load_weights: missing tensor " + w.name);
                if (it->second.nbytes != elems(w.shape) * 2 || it->second.shape != w.shape)
                    throw kvc::Error(KVC_ERR_ARG, "load_weights: " + w.name + " has the wrong size or shape");
                read_into(it->second, w.dst);
            }
            const auto lh = man.find("lm_head.weight");
            bool tied = true;
            if (lh != man.end()) {
                const auto& e = man["model.embed_tokens.weight"];
                if (lh->second.nbytes != e.nbytes || lh->second.shape != e.shape)
                    throw kvc::Error(KVC_ERR_ARG, "load_weights: lm_head.weight has the wrong size or shape");
                // tied when the bytes equal the embedding's (the dump stores a copy)
                std::vector<char> a(chunk), b(chunk);
                for (size_t done = 0; done < e.nbytes && tied; done += chunk) {
                    const size_t n = std::min(chunk, e.nbytes - done);
                    bf.seekg((std::streamoff)(e.off + done)); bf.read(a.data(), (std::streamsize)n);
                    bf.seekg((std::streamoff)(lh->second.off + done)); bf.read(b.data(), (std::streamsize)n);
                    tied = std::memcmp(a.data(), b.data(), n) == 0;
                }
                if (!tied) {
                    if (!lm_head) lm_head = alloc(lh->second.nbytes);
                    read_into(lh->second, lm_head);
                }
            }
            if (tied) lm_head = nullptr;  // (an untied matrix from an earlier load stays allocated, unused)
        } catch (...) {
            kvc_host_free(stage);
            throw;
        }
        kvc_host_free(stage);
        kvc_graph_destroy(gexec);  // the captured step holds the old output matrix
        gexec = nullptr;
    }

    // Writes the model's tensors in the same format (lm_head.weight included, as the
    // reference's dump does for the tied Qwen2.5 models).
    void save_weights(const std::string& dir) {
        std::ofstream bf(dir + "/weights.bin", std::ios::binary);
        std::ofstream mf(dir + "/manifest.tsv");
        if (!bf || !mf) throw kvc::Error(KVC_ERR_ARG, "save_weights: cannot write into " + dir);
        auto refs = weight_refs();
        refs.push_back({"lm_head.weight", const_cast<void*>(lm_w()), {c.vocab, c.hidden}});
        size_t off = 0;
        std::vector<char> host;
        for (const WeightRef& w : refs) {
            const size_t nb = elems(w.shape) * 2;
            host.resize(nb);
            kvc::check(kvc_memcpy_d2h(host.data(), w.dst, nb, stream), "weights download");
            kvc::check(kvc_stream_synchronize(stream), "weights download");
            bf.write(host.data(), (std::streamsize)nb);
            std::string shape;
            for (size_t i = 0; i < w.shape.size(); ++i) shape += (i ? "," : "") + std::to_string(w.shape[i]);
            mf << w.name << '\t' << off << '\t' << nb << '\t' << shape << '\n';
            off += nb;
        }
        if (!bf || !mf) throw kvc::Error(KVC_ERR_ARG, "save_weights: write failed");
    }

    struct Request {
        std::vector<int> prompt;
        int gen_len = 0;
    };
    struct ServeStats {
        int steps = 0, finished = 0;
        long long tokens = 0, prompt_tokens = 0, graph_steps = 0, graph_captures = 0, chain_launches = 0;
        double wall_us = 0, prefill_us = 0, decode_us = 0;
    };

    // Continuous-batching greedy generation; out[i] receives request i's gen_len tokens.
    ServeStats serve(const std::vector<Request>& reqs, std::vector<std::vector<int>>& out) {
        using clk = std::chrono::steady_clock;
        ServeStats st;
        const long long graph_steps0 = graph_steps, graph_captures0 = graph_captures, chain0 = chain_launches;
        kvm.reset();
        out.assign(reqs.size(), {});
        std::vector<Sequence> seqs(reqs.size());
        std::deque<int> waiting;
        for (size_t i = 0; i < reqs.size(); ++i) {
            seqs[i].id = (int)i;
            seqs[i].prompt_len = (int)reqs[i].prompt.size();
            seqs[i].max_new_tokens = reqs[i].gen_len;
            waiting.push_back((int)i);
        }
        std::vector<int> run, in, nxt;
        int reserved = 0;  // worst-case blocks of the running sequences (engine.h:118-124)
        auto worst = [&](int i) { return blocks_needed(seqs[i].prompt_len + reqs[i].gen_len, c.block_size); };
        const auto t0 = clk::now();
        while (!waiting.empty() || !run.empty()) {
            for (size_t r = 0; r < run.size();) {  // retire
                Sequence& s = seqs[run[r]];
                if ((int)out[run[r]].size() >= reqs[run[r]].gen_len) {
                    kvm.free(s);
                    reserved -= worst(run[r]);
                    st.finished++;
                    run[r] = run.back();
                    run.pop_back();
                } else {
                    ++r;
                }
            }
            std::vector<int> admitted;
            while ((int)run.size() < c.max_batch && !waiting.empty()) {  // admit
                const int i = waiting.front();
                Sequence& s = seqs[i];
                if (reqs[i].gen_len < 1 || s.prompt_len < 1) throw kvc::Error(KVC_ERR_ARG, "serve: empty request");
                if (s.prompt_len > std::max(c.max_rows, c.prefill_rows))
                    throw kvc::Error(KVC_ERR_ARG, "serve: prompt longer than max_rows");
                if (reserved + worst(i) > c.num_blocks) break;
                if (!kvm.allocate_prompt(s)) break;
                reserved += worst(i);
                waiting.pop_front();
                admitted.push_back(i);
                run.push_back(i);
            }
            for (size_t a = 0; a < admitted.size();) {  // prefill the admitted prompts, stacked
                std::vector<Sequence*> ps;
                std::vector<const int*> pt;
                int rows = 0;
                size_t b = a;
                for (; b < admitted.size(); ++b) {
                    const int P = seqs[admitted[b]].prompt_len;
                    if (!ps.empty() && rows + P > c.prefill_rows) break;
                    ps.push_back(&seqs[admitted[b]]);
                    pt.push_back(reqs[admitted[b]].prompt.data());
                    rows += P;
                }
                std::vector<int> first(ps.size());
                const auto p0 = clk::now();
                prefill_batch(ps, pt, first.data());
                st.prefill_us += std::chrono::duration<double, std::micro>(clk::now() - p0).count();
                for (size_t j = 0; j < ps.size(); ++j) {
                    out[admitted[a + j]].push_back(first[j]);
                    st.prompt_tokens += ps[j]->prompt_len;
                    st.tokens++;
                }
                a = b;
            }
            std::vector<Sequence*> batch;
            in.clear();
            for (int i : run)
                if ((int)out[i].size() < reqs[i].gen_len) {
                    if (!kvm.append_token(seqs[i])) throw kvc::Error(KVC_ERR_NOMEM, "serve: pool exhausted");
                    batch.push_back(&seqs[i]);
                    in.push_back(out[i].back());
                }
            if (batch.empty()) {
                if (run.empty() && !waiting.empty())
                    throw kvc::Error(KVC_ERR_STATE, "serve: a request can never be admitted");
                continue;
            }
            nxt.resize(batch.size());
            const auto d0 = clk::now();
            decode(batch, in.data(), nxt.data());
            st.decode_us += std::chrono::duration<double, std::micro>(clk::now() - d0).count();
            st.steps++;
            for (size_t r = 0; r < batch.size(); ++r) {
                out[batch[r]->id].push_back(nxt[r]);
                st.tokens++;
            }
        }
        st.wall_us = std::chrono::duration<double, std::micro>(clk::now() - t0).count();
        st.graph_steps = graph_steps - graph_steps0;
        st.graph_captures = graph_captures - graph_captures0;
        st.chain_launches = chain_launches - chain0;
        return st;
    }
};
