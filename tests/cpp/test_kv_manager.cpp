// test_kv_manager.cpp -- the checks of the reference's tests/test_kv_manager.cu:13-55,
// rewritten against the drop-in headers.  `--host` keeps the manager host-only
// (no device pools), so the accounting runs without a GPU.
#include <cstdio>
#include <cstring>

#include "kvc/kv_cache_manager.h"

static int g_fail = 0;
#define CHECK(cond, msg)                                  \
    do {                                                  \
        if (!(cond)) { std::printf("  [FAIL] %s\n", msg); ++g_fail; } \
        else         { std::printf("  [ ok ] %s\n", msg); }          \
    } while (0)

int main(int argc, char** argv) {
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host") == 0;
    KVCacheManager kvm(/*num_blocks*/ 8, /*block_size*/ 4, /*n_kv_heads*/ 2, /*head_dim*/ 8, KVC_F32, 1, !host_only);
    CHECK(kvm.free_blocks() == 8, "init free=8");
    CHECK(host_only || kvm.has_device(), "device pools allocated");

    Sequence a; a.id = 0; a.prompt_len = 5;
    CHECK(kvm.allocate_prompt(a), "A allocate_prompt ok");
    CHECK((int)a.block_table.size() == 2, "A has 2 blocks");
    CHECK(a.cur_len == 5, "A cur_len=5");
    CHECK(kvm.free_blocks() == 6, "free=6 after A");
    CHECK(kvm.slack(a) == 3, "A slack=3");
    kvm.append_token(a); kvm.append_token(a); kvm.append_token(a);
    CHECK((int)a.block_table.size() == 2, "A still 2 blocks at len=8");
    CHECK(kvm.slack(a) == 0, "A slack=0 at len=8");
    kvm.append_token(a);
    CHECK((int)a.block_table.size() == 3, "A grew to 3 blocks at len=9");
    CHECK(a.cur_len == 9 && a.num_generated() == 4, "A len=9 generated=4");
    CHECK(kvm.free_blocks() == 5, "free=5 after A grew");

    Sequence b; b.id = 1; b.prompt_len = 20;
    CHECK(kvm.allocate_prompt(b), "B allocate_prompt ok (uses last 5)");
    CHECK(kvm.free_blocks() == 0, "pool exhausted");
    Sequence c; c.id = 2; c.prompt_len = 1;
    CHECK(!kvm.allocate_prompt(c), "C allocate_prompt fails (OOM)");
    CHECK(c.block_table.empty(), "C untouched on OOM");
    CHECK(!kvm.append_token(b), "B append fails (no free block)");
    CHECK(b.cur_len == 20, "B cur_len unchanged on failed append");

    kvm.free(a);
    CHECK(a.block_table.empty(), "A table cleared");
    CHECK(kvm.free_blocks() == 3, "free=3 after releasing A");
    CHECK(kvm.append_token(b), "B append ok after free");
    CHECK(b.block_table.back() == 2, "B grew into A's last freed block (LIFO)");
    CHECK(kvm.slot_offset(3, 1, 2) == (((size_t)3 * 2 + 1) * 4 + 2) * 8, "slot_offset matches pool layout");

    std::printf(g_fail ? "\n=== %d CHECK(S) FAILED ===\n" : "\n=== ALL CHECKS PASSED ===\n", g_fail);
    return g_fail ? 1 : 0;
}
