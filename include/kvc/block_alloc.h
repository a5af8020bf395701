// block_alloc.h -- host free-list of equal-size physical KV blocks.
//
// Drop-in for the reference's BlockAllocator / blocks_needed
// (src/include/block_alloc.h:10-43), same names and contract:
//   * a fresh allocator hands out 0, 1, 2, ... (LIFO stack initialised n-1..0),
//   * alloc() returns -1 when the pool is empty,
//   * free_blocks() pushes a sequence's table back in table order, so the last
//     block of a freed table is the next one handed out,
//   * reset() restores the fresh state.
// The exact order matters: block tables (and therefore every byte the decode
// kernels read) are bit-identical to the reference's for the same trace.
// Extension: shuffle() permutes the current free list (fragmented-pool
// workloads: blocks come out in a seeded random physical order).
#pragma once
#include <cstdint>
#include <utility>
#include <vector>

struct BlockAllocator {
    int total_blocks;
    std::vector<int> free_list;  // stack: back() is handed out next

    explicit BlockAllocator(int n) : total_blocks(n) { reset(); }

    int free_count() const { return (int)free_list.size(); }
    int used_count() const { return total_blocks - (int)free_list.size(); }

    int alloc() {
        if (free_list.empty()) return -1;
        const int b = free_list.back();
        free_list.pop_back();
        return b;
    }
    void free_blocks(const std::vector<int>& blocks) { free_blocks(blocks.data(), (int)blocks.size()); }
    void free_blocks(const int* blocks, int n) {
        for (int i = 0; i < n; ++i) free_list.push_back(blocks[i]);
    }
    void reset() {
        free_list.resize(total_blocks > 0 ? total_blocks : 0);
        for (int i = 0; i < (int)free_list.size(); ++i) free_list[i] = total_blocks - 1 - i;
    }
    // Seeded Fisher-Yates over the free list (splitmix64 stream).
    void shuffle(uint64_t seed) {
        uint64_t x = seed;
        auto next = [&x] {
            uint64_t z = (x += 0x9E3779B97F4A7C15ull);
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            return z ^ (z >> 31);
        };
        for (int i = (int)free_list.size() - 1; i > 0; --i) std::swap(free_list[i], free_list[next() % (uint64_t)(i + 1)]);
    }
};

// Blocks needed to hold seq_len tokens: ceil(seq_len / block).
static inline int blocks_needed(int seq_len, int block) { return (seq_len + block - 1) / block; }
