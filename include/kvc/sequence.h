// sequence.h -- one request as the Engine tracks it (reference src/include/sequence.h:12-27).
// The members are those the Engine loop and KVCacheManager read and write: the KV
// lengths at admission and now (their difference is what the stop rule compares with
// max_new_tokens), the block table the manager fills, the lifecycle state, and the
// arrival timestamp that the latency report subtracts from the finishing clock.
#pragma once
#include <vector>

enum class SeqStatus { Waiting, Running, Finished };

struct Sequence {
    int id = -1;
    int prompt_len = 0;            // tokens in the cache once admitted
    int cur_len = 0;               // tokens in the cache now
    int max_new_tokens = 0;        // the stop rule's budget of generated tokens
    double arrival_us = 0;         // clock (us) at which the request entered the queue
    std::vector<int> tokens;       // token ids (the scheduling benchmarks leave it empty)
    std::vector<int> block_table;  // physical block id of each logical block, in order
    SeqStatus status = SeqStatus::Waiting;

    int num_generated() const { return cur_len - prompt_len; }
    bool done() const { return num_generated() >= max_new_tokens; }
    bool is_finished() const { return status == SeqStatus::Finished; }
};
