// ref_gen_driver.cpp -- test infrastructure: runs the reference's own input
// generators on fixed arguments so that the Python restatements (workloads.hval,
// workloads.shuffle_perm) are pinned bit for bit against them:
//   hval          bench_throughput.cu:21-25 (deterministic K/V values in [-1, 1))
//   table shuffle main_paged.cu:28-37 (the seeded block-table permutation)
// Their bodies are not in this repository: oracle/Makefile (target `ref`) extracts
// them from /root/reference into _ref/ at build time, compiles this driver against
// them and deletes the extracted text.  Output: one line per value.
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <string_view>
#include <utility>
#include <vector>

#include "ref_hval.inc"

// the reference's shuffle loop, run on the identity permutation of nb blocks
static std::vector<int> ref_shuffle(int NB) {
    std::vector<int> perm(NB);
    std::iota(perm.begin(), perm.end(), 0);
#include "ref_shuffle.inc"
    }
    return perm;
}

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: ref_gen_driver hval|shuffle\n");
        return 2;
    }
    const std::string_view what = argv[1];
    if (what == "hval") {
        // a grid of (s, h, pos, d, salt) arguments, large values included (the hash wraps)
        const unsigned ss[] = {0, 1, 7, 127, 4096, 4000000000u};
        const unsigned hs[] = {0, 3, 31};
        const unsigned ps[] = {0, 1, 2047, 65535};
        const unsigned ds[] = {0, 5, 63, 127};
        const unsigned salts[] = {1, 2, 3};
        for (unsigned s : ss)
            for (unsigned h : hs)
                for (unsigned p : ps)
                    for (unsigned d : ds)
                        for (unsigned salt : salts) std::printf("%u %u %u %u %u %.9g\n", s, h, p, d, salt, hval(s, h, p, d, salt));
        return 0;
    }
    if (what == "shuffle") {
        for (int nb : {1, 2, 3, 16, 128, 1000}) {
            const std::vector<int> p = ref_shuffle(nb);
            std::printf("%d", nb);
            for (int x : p) std::printf(" %d", x);
            std::printf("\n");
        }
        return 0;
    }
    return 2;
}
