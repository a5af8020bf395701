// demo_engine.cpp -- the end-to-end accounting checks of the reference's
// apps/demo_engine.cu:13-43 against the drop-in Engine: 256 synthetic requests
// (srand(123)), width 32, 512 blocks; tokens == sum(gen), finished == NREQ,
// peak <= pool.  `--host` runs scheduling only with a virtual clock (no GPU).
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "kvc/engine.h"

int main(int argc, char** argv) {
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host") == 0;
    EngineConfig cfg{/*n_heads*/ 8, /*head_dim*/ 64, /*block_size*/ 16, /*num_blocks*/ 512, /*max_batch*/ 32};
    if (host_only) {
        cfg.device = false;
        cfg.clock_mode = 1;
        cfg.c0 = 10.0;
    }
    Engine eng(cfg);
    srand(123);
    const int NREQ = 256;
    long long expected = 0;
    for (int i = 0; i < NREQ; ++i) {
        const int prompt = 8 + rand() % 120;
        const int gen = 16 + rand() % 200;
        eng.add_request(prompt, gen);
        expected += gen;
    }
    const EngineStats st = eng.run();
    std::printf("NREQ=%d iters=%d finished=%d tokens=%lld (expected %lld) peak=%d gpu_us=%.0f\n", NREQ, st.iters,
                st.finished, st.tokens, expected, st.peak_blocks, st.gpu_us);
    const bool ok = st.tokens == expected && st.finished == NREQ && st.peak_blocks <= cfg.num_blocks &&
                    (host_only || st.gpu_us > 0);
    std::printf(ok ? "=== ENGINE OK ===\n" : "=== ENGINE MISMATCH ===\n");
    return ok ? 0 : 1;
}
