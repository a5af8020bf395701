// ref_alloc_driver.cpp -- runs the REFERENCE's own BlockAllocator / Sequence
// (compiled from /root/reference/src/include/block_alloc.h and sequence.h, the
// two host-only headers of the path that build with g++) over a script read
// from stdin, so tests can compare the oracle's and the product's free-list
// against the reference code itself.  Test infrastructure only.
//
// stdin:  first line "<total_blocks>", then one op per line:
//   A      -> alloc(), prints the block id (or -1)
//   F n    -> free_blocks(first n still-held blocks, in allocation order), prints free_count()
//   R      -> reset(), prints free_count()
//   N l b  -> blocks_needed(l, b), prints the result
//   D p c m-> Sequence{prompt_len=p, cur_len=c, max_new_tokens=m}.done(), prints 0/1
#include "block_alloc.h"
#include "sequence.h"
#include <iostream>
#include <string>
#include <vector>

int main() {
    int total = 0;
    if (!(std::cin >> total)) return 2;
    BlockAllocator a(total);
    std::vector<int> held;
    std::string op;
    while (std::cin >> op) {
        if (op == "A") {
            int b = a.alloc();
            if (b >= 0) held.push_back(b);
            std::cout << b << "\n";
        } else if (op == "F") {
            int n; std::cin >> n;
            if (n > (int)held.size()) n = (int)held.size();
            std::vector<int> fr(held.begin(), held.begin() + n);
            held.erase(held.begin(), held.begin() + n);
            a.free_blocks(fr);
            std::cout << a.free_count() << "\n";
        } else if (op == "R") {
            a.reset(); held.clear();
            std::cout << a.free_count() << "\n";
        } else if (op == "N") {
            int l, b; std::cin >> l >> b;
            std::cout << blocks_needed(l, b) << "\n";
        } else if (op == "D") {
            Sequence s; std::cin >> s.prompt_len >> s.cur_len >> s.max_new_tokens;
            std::cout << (s.done() ? 1 : 0) << "\n";
        } else {
            return 3;
        }
    }
    return 0;
}
