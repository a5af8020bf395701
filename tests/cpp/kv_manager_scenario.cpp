// kv_manager_scenario.cpp -- KVCacheManager driven through a scripted scenario.
//
// A pool of 8 blocks x 4 tokens (Hkv 2, head_dim 8) serves three sequences.  Each
// step of the script applies one operation and states the whole observable state
// afterwards (the operation's result, every sequence's cur_len and table, the free
// count), so an accounting slip shows up at the step that made it.  The expected
// states follow from the manager's contract (kv_cache_manager.h:56-91 of the
// reference): prompts take ceil(len / BLOCK) blocks all-or-nothing, a token takes a
// new block only on a block boundary, an empty pool refuses without changing
// anything, and freed blocks go back LIFO in table order onto a stack that hands
// out 0, 1, 2, ... from a fresh pool.  `--host` runs the accounting without device
// pools; otherwise the pools must exist, be zero-filled and span the layout.
#include <cstdio>
#include <cstring>
#include <vector>

#include "kvc/kv_cache_manager.h"

namespace {

enum class Op { Prompt, Token, Free };

struct Step {
    Op op;
    int seq, arg;                       // sequence, prompt length (Prompt only)
    int result;                         // 1 true, 0 false, -1 no result (Free)
    int free_after;                     // free blocks after the step
    std::vector<std::vector<int>> tables;  // every sequence's table after the step
    std::vector<int> lens;              // every sequence's cur_len after the step
};

const char* name(Op op) { return op == Op::Prompt ? "allocate_prompt" : op == Op::Token ? "append_token" : "free"; }

}  // namespace

int main(int argc, char** argv) {
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host") == 0;
    const int NB = 8, BLOCK = 4, HKV = 2, D = 8;
    KVCacheManager kvm(NB, BLOCK, HKV, D, KVC_F32, 1, !host_only);
    std::vector<Sequence> seq(3);
    for (int i = 0; i < 3; ++i) seq[i].id = i;

    const std::vector<Step> script = {
        // seq 0: 5 tokens -> blocks 0,1 (3 slots left in block 1)
        {Op::Prompt, 0, 5, 1, 6, {{0, 1}, {}, {}}, {5, 0, 0}},
        {Op::Token, 0, 0, 1, 6, {{0, 1}, {}, {}}, {6, 0, 0}},
        {Op::Token, 0, 0, 1, 6, {{0, 1}, {}, {}}, {7, 0, 0}},
        {Op::Token, 0, 0, 1, 6, {{0, 1}, {}, {}}, {8, 0, 0}},
        // the 9th token crosses a block boundary: block 2
        {Op::Token, 0, 0, 1, 5, {{0, 1, 2}, {}, {}}, {9, 0, 0}},
        // seq 1: 20 tokens take the remaining 5 blocks
        {Op::Prompt, 1, 20, 1, 0, {{0, 1, 2}, {3, 4, 5, 6, 7}, {}}, {9, 20, 0}},
        // empty pool: a 1-token prompt and a boundary-crossing token are refused untouched
        {Op::Prompt, 2, 1, 0, 0, {{0, 1, 2}, {3, 4, 5, 6, 7}, {}}, {9, 20, 0}},
        {Op::Token, 1, 0, 0, 0, {{0, 1, 2}, {3, 4, 5, 6, 7}, {}}, {9, 20, 0}},
        // seq 0 returns 0,1,2 (pushed in table order, so 2 comes back first)
        // (free clears the table; cur_len is the caller's and stays)
        {Op::Free, 0, 0, -1, 3, {{}, {3, 4, 5, 6, 7}, {}}, {9, 20, 0}},
        {Op::Token, 1, 0, 1, 2, {{}, {3, 4, 5, 6, 7, 2}, {}}, {9, 21, 0}},
        {Op::Prompt, 2, 8, 1, 0, {{}, {3, 4, 5, 6, 7, 2}, {1, 0}}, {9, 21, 8}},
        {Op::Free, 1, 0, -1, 6, {{}, {}, {1, 0}}, {9, 21, 8}},
        {Op::Free, 2, 0, -1, 8, {{}, {}, {}}, {9, 21, 8}},
    };

    int fails = 0;
    for (size_t i = 0; i < script.size(); ++i) {
        const Step& st = script[i];
        Sequence& s = seq[st.seq];
        int got = -1;
        if (st.op == Op::Prompt) {
            s.prompt_len = st.arg;
            got = kvm.allocate_prompt(s);
        } else if (st.op == Op::Token) {
            got = kvm.append_token(s);
        } else {
            kvm.free(s);
        }
        bool ok = got == st.result && kvm.free_blocks() == st.free_after;
        for (int j = 0; j < 3; ++j) ok = ok && seq[j].block_table == st.tables[j] && seq[j].cur_len == st.lens[j];
        std::printf("step %2zu %-15s seq %d: %s\n", i, name(st.op), st.seq, ok ? "as expected" : "MISMATCH");
        if (!ok) {
            std::printf("    result %d (want %d), free %d (want %d)\n", got, st.result, kvm.free_blocks(), st.free_after);
            ++fails;
        }
    }

    // pool layout: slot (block, head, in-block) -> ((block*Hkv + head)*BLOCK + in)*D
    for (int b : {0, 3, 7})
        for (int h = 0; h < HKV; ++h)
            for (int in : {0, 2, 3})
                if (kvm.slot_offset(b, h, in) != (size_t)((b * HKV + h) * BLOCK + in) * D) {
                    std::printf("slot_offset(%d, %d, %d) = %zu\n", b, h, in, kvm.slot_offset(b, h, in));
                    ++fails;
                }
    if (kvm.pool_elems() != (size_t)NB * HKV * BLOCK * D) ++fails, std::printf("pool_elems %zu\n", kvm.pool_elems());

    if (!host_only) {
        if (!kvm.has_device()) {
            std::printf("device pools missing\n");
            ++fails;
        } else {
            std::vector<float> k(kvm.pool_elems(), 1.f), v(kvm.pool_elems(), 1.f);
            kvc::check(kvc_memcpy_d2h(k.data(), kvm.k_pool, k.size() * 4, nullptr), "k pool");
            kvc::check(kvc_memcpy_d2h(v.data(), kvm.v_pool, v.size() * 4, nullptr), "v pool");
            kvc::check(kvc_device_synchronize(), "sync");
            for (size_t i = 0; i < k.size(); ++i)
                if (k[i] != 0.f || v[i] != 0.f) {
                    std::printf("pool element %zu not zero-filled\n", i);
                    ++fails;
                    break;
                }
        }
    }
    std::printf(fails ? "%d mismatch(es)\n" : "scenario matches\n", fails);
    return fails ? 1 : 0;
}
