// test_qwen_graph_regrow.cpp -- QwenModel's captured decode step after its split-K
// workspace moves.
//
// The step graph is captured with the workspace's address inside its kernel
// arguments.  Growing the workspace frees that address, so the model must drop the
// graph and capture it again on the next decode step; replaying the old graph
// would write partials into freed memory.  This program:
//   1. serves a first batch with graph replay (one capture),
//   2. grows the workspace (what a larger plan than the captured capacity does),
//   3. serves a second batch: the graph must be captured once more and every step
//      replayed, with the same tokens as a model that launches every step eagerly
//      (the eager steps are teacher-forced against the CPU restatement in
//      tests/test_gpu_qwen.py);
//   4. checks the host guard: a replay whose workspace differs from the captured
//      one is refused with KVC_ERR_STATE instead of being launched.
#include <cstdio>
#include <vector>

#include "kvc/qwen_model.h"

static std::vector<QwenModel::Request> requests(unsigned seed, int n, int vocab) {
    std::vector<QwenModel::Request> r(n);
    unsigned x = seed;
    auto next = [&] { x = x * 1103515245u + 12345u; return x >> 8; };
    for (auto& q : r) {
        q.prompt.resize(5 + next() % 120);
        for (int& t : q.prompt) t = (int)(next() % (unsigned)vocab);
        q.gen_len = 1 + (int)(next() % 24);
    }
    return r;
}

int main() {
    QwenConfig cfg;
    cfg.layers = 2; cfg.vocab = 4096; cfg.num_blocks = 512; cfg.max_batch = 4; cfg.max_rows = 256; cfg.seed = 11;
    QwenConfig eager_cfg = cfg;
    cfg.graph = 1;
    eager_cfg.graph = 0;
    int fails = 0;
    auto expect = [&](bool ok, const char* what) {
        std::printf("%s %s\n", ok ? "pass" : "FAIL", what);
        fails += !ok;
    };
    try {
        QwenModel g(cfg), e(eager_cfg);
        const auto a = requests(7, 6, cfg.vocab), b = requests(99, 9, cfg.vocab);
        std::vector<std::vector<int>> ga, ea, gb, eb;
        const auto sa = g.serve(a, ga);
        e.serve(a, ea);
        expect(sa.graph_captures == 1 && sa.graph_steps == sa.steps && sa.steps > 0, "first batch: one capture, every step replayed");
        expect(ga == ea, "first batch: replayed tokens equal eager tokens");

        const void* old_ws = g.ws;
        g.ensure_ws(g.ws_bytes * 4 + 1);
        expect(g.ws != old_ws && g.gexec == nullptr, "workspace growth drops the captured graph");

        const auto sb = g.serve(b, gb);
        e.serve(b, eb);
        expect(sb.graph_captures == 1 && sb.graph_steps == sb.steps && sb.steps > 0,
               "second batch: captured again on the new workspace, every step replayed");
        expect(gb == eb, "second batch: replayed tokens equal eager tokens");

        // a workspace swapped behind the graph's back is refused, not replayed
        void* other = nullptr;
        kvc::check(kvc_malloc(&other, g.ws_bytes), "other workspace");
        void* mine = g.ws;
        g.ws = other;
        bool refused = false;
        try {
            std::vector<std::vector<int>> tmp;
            g.serve(a, tmp);
        } catch (const kvc::Error& err) {
            refused = err.status == KVC_ERR_STATE;
        }
        g.ws = mine;
        kvc::check(kvc_stream_synchronize(g.stream), "sync");
        kvc_free(other);
        expect(refused, "replay with a different workspace fails with KVC_ERR_STATE");
    } catch (const kvc::Error& err) {
        std::printf("FAIL kvc error %d: %s\n", err.status, err.what());
        return 1;
    }
    std::printf(fails ? "%d check(s) failed\n" : "all checks passed\n", fails);
    return fails ? 1 : 0;
}
