// test_runner_paths.cpp -- ModelRunner::decode_step on its two decode paths.
//
// The host-planned path (work list appended to the step's one upload) and the
// device-lengths path (kvc_batched_paged_decode_split) must give the same
// attention output on the same pools, tables and inputs: within 2e-3 (fp16 K/V,
// fp32 accumulation; the two paths cut sequences into different chunks).  Both
// kernels are checked against the CPU restatement elsewhere; this program checks
// the runner's packing (offsets of tables and work list in the upload, the
// workspace sizing, growth of the metadata buffers) on a ragged GQA batch with
// sequences long enough to be split, over two layers with K/V writes.  Then the
// graph-replayed planned step (one capture, counts and metadata in device memory)
// against the eagerly launched one, step after step with different batches: the
// same kernels on the same plans, so the outputs must be bit-identical.  Last,
// prefill_batch (several prompts' rows through one planned causal launch per layer)
// against the query-tiled causal kernel run per prompt on the K/V it wrote.
#include <cmath>
#include <cstdio>
#include <vector>

#include "kvc/model_runner.h"

static std::vector<_Float16> fetch(const ModelRunner& r, int n) {
    std::vector<_Float16> h((size_t)n * r.n_heads * r.head_dim);
    kvc::check(kvc_memcpy_d2h(h.data(), r.dout, h.size() * sizeof(_Float16), r.stream), "d2h");
    kvc::check(kvc_stream_synchronize(r.stream), "sync");
    return h;
}

int main() {
    const int Hq = 14, Hkv = 2, D = 64, B = 16, NB = 4096, L = 2, maxB = 32;
    KVCacheManager kvm(NB, B, Hkv, D, KVC_F16, L);
    for (int l = 0; l < L; ++l) {
        kvc::check(kvc_fill_normal(kvm.k_layer(l), kvm.pool_elems(), KVC_F16, 11 + l, 1.0f, nullptr), "fill k");
        kvc::check(kvc_fill_normal(kvm.v_layer(l), kvm.pool_elems(), KVC_F16, 23 + l, 1.0f, nullptr), "fill v");
    }
    kvc::check(kvc_device_synchronize(), "sync");

    // ragged lengths 1 .. ~6000 tokens (several sequences need more than one chunk)
    std::vector<Sequence> seqs(maxB);
    std::vector<Sequence*> batch;
    unsigned x = 12345;
    for (int i = 0; i < maxB; ++i) {
        x = x * 1103515245u + 12345u;
        const double r = ((x >> 9) & 0x7FFFFF) / 8388608.0;
        seqs[i].id = i;
        seqs[i].prompt_len = seqs[i].cur_len = 1 + (int)(5999 * r * r * r);
        if (!kvm.allocate_prompt(seqs[i])) { std::printf("pool too small\n"); return 2; }
        batch.push_back(&seqs[i]);
    }
    std::vector<int> wpos(maxB);
    for (int i = 0; i < maxB; ++i) wpos[i] = seqs[i].cur_len - 1;  // rewrite each sequence's last row

    int worst = 0;
    for (int kv_write = 0; kv_write <= 1; ++kv_write) {
        for (int n : {maxB, 5}) {
            RunnerOptions po;
            po.n_kv_heads = Hkv; po.n_layers = L; po.dtype = KVC_F16; po.kv_write = kv_write;
            RunnerOptions so = po;
            so.decode_path = KVC_DECODE_DEVICE_LENGTHS;
            ModelRunner planned(Hq, D, B, maxB, NB, po), split(Hq, D, B, maxB, NB, so);
            std::vector<Sequence*> b(batch.begin(), batch.begin() + n);
            planned.decode_step(b, kvm, kv_write ? wpos.data() : nullptr);
            split.decode_step(b, kvm, kv_write ? wpos.data() : nullptr);
            const auto a = fetch(planned, n), c = fetch(split, n);
            double err = 0;
            bool finite = true;
            for (size_t i = 0; i < a.size(); ++i) {
                finite = finite && std::isfinite((double)a[i]);
                err = std::fmax(err, std::fabs((double)a[i] - (double)c[i]));
            }
            std::printf("kv_write=%d N=%d: max |planned - device-lengths| = %.3e (digests %s)\n", kv_write, n, err,
                        planned.digest == split.digest ? "equal" : "DIFFER");
            if (!(err <= 2e-3) || !finite || planned.digest != split.digest) worst = 1;
        }
    }
    for (int kv_write = 0; kv_write <= 1; ++kv_write) {
        RunnerOptions eo;
        eo.n_kv_heads = Hkv; eo.n_layers = L; eo.dtype = KVC_F16; eo.kv_write = kv_write;
        RunnerOptions go = eo;
        go.graph = true;
        ModelRunner eager(Hq, D, B, maxB, NB, eo), graph(Hq, D, B, maxB, NB, go);
        for (int n : {maxB, 5, 17, 1, maxB}) {
            std::vector<Sequence*> b(batch.begin() + (maxB - n) / 2, batch.begin() + (maxB - n) / 2 + n);
            std::vector<int> wp(wpos.begin() + (maxB - n) / 2, wpos.begin() + (maxB - n) / 2 + n);
            eager.decode_step(b, kvm, kv_write ? wp.data() : nullptr);
            const auto a = fetch(eager, n);
            graph.decode_step(b, kvm, kv_write ? wp.data() : nullptr);
            const auto c = fetch(graph, n);
            size_t diff = 0;
            for (size_t i = 0; i < a.size(); ++i) diff += (a[i] != c[i]);
            std::printf("graph kv_write=%d N=%d: %zu of %zu outputs differ from the eager step\n", kv_write, n, diff,
                        a.size());
            if (diff) worst = 1;
        }
        std::printf("graph steps replayed: %lld\n", graph.graph_steps);
        if (graph.graph_steps != 5) worst = 1;
    }
    {
        RunnerOptions fo;
        fo.n_kv_heads = Hkv; fo.n_layers = L; fo.dtype = KVC_F16; fo.kv_write = true; fo.prefill = true;
        KVCacheManager pk(NB, B, Hkv, D, KVC_F16, L);
        ModelRunner r(Hq, D, B, maxB, NB, fo);
        const int lens[] = {1, 16, 17, 130, 900, 45};
        std::vector<Sequence> ps(6);
        std::vector<Sequence*> pb;
        for (int i = 0; i < 6; ++i) {
            ps[i].id = i;
            ps[i].prompt_len = ps[i].cur_len = lens[i];
            if (!pk.allocate_prompt(ps[i])) { std::printf("pool too small\n"); return 2; }
            pb.push_back(&ps[i]);
        }
        r.prefill_batch(pb, pk);
        const int R = 1 + 16 + 17 + 130 + 900 + 45;
        std::vector<_Float16> got((size_t)R * Hq * D);
        kvc::check(kvc_memcpy_d2h(got.data(), r.pout, got.size() * 2, r.stream), "d2h");
        kvc::check(kvc_stream_synchronize(r.stream), "sync");
        int* dt = nullptr;
        void* one = nullptr;
        kvc::check(kvc_malloc((void**)&dt, 4096 * 4), "table");
        kvc::check(kvc_malloc(&one, (size_t)900 * Hq * D * 2), "out");
        double err = 0;
        int off = 0;
        for (int i = 0; i < 6; ++i) {  // the last layer's attention, prompt by prompt
            const int P = lens[i];
            kvc::check(kvc_memcpy_h2d(dt, ps[i].block_table.data(), ps[i].block_table.size() * 4, r.stream), "h2d");
            kvc::check(kvc_paged_causal_attn(static_cast<const char*>(r.pq) + (size_t)off * Hq * D * 2, one,
                                             pk.k_layer(L - 1), pk.v_layer(L - 1), dt, 0, P, Hq, Hkv, D, B,
                                             1.0f / std::sqrt((float)D), KVC_F16, nullptr, 0, r.stream),
                       "causal");
            std::vector<_Float16> ref((size_t)P * Hq * D);
            kvc::check(kvc_memcpy_d2h(ref.data(), one, ref.size() * 2, r.stream), "d2h");
            kvc::check(kvc_stream_synchronize(r.stream), "sync");
            for (size_t k = 0; k < ref.size(); ++k)
                err = std::fmax(err, std::fabs((double)ref[k] - (double)got[(size_t)off * Hq * D + k]));
            off += P;
        }
        kvc_free(dt); kvc_free(one);
        std::printf("prefill_batch vs per-prompt causal attention: max |diff| = %.3e\n", err);
        if (!(err <= 2e-3)) worst = 1;
    }
    std::printf(worst ? "=== RUNNER PATHS MISMATCH ===\n" : "=== RUNNER PATHS OK ===\n");
    return worst;
}
