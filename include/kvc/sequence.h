// sequence.h -- runtime state of one sequence (reference src/include/sequence.h:12-27).
// Logical state only: token progress, block table, status, stop rule, arrival
// time.  Physical blocks belong to KVCacheManager, scheduling to Engine.
#pragma once
#include <vector>

enum class SeqStatus { Waiting, Running, Finished };

struct Sequence {
    int id = -1;
    int prompt_len = 0;        // KV length after prefill
    int cur_len = 0;           // KV length = prompt + generated tokens
    int max_new_tokens = 0;    // stop after this many generated tokens
    double arrival_us = 0;     // arrival time (us); latency = finish - arrival
    std::vector<int> tokens;   // token ids (unused by the scheduling benchmarks)
    std::vector<int> block_table;  // logical block -> physical block
    SeqStatus status = SeqStatus::Waiting;

    int num_generated() const { return cur_len - prompt_len; }
    bool done() const { return num_generated() >= max_new_tokens; }
    bool is_finished() const { return status == SeqStatus::Finished; }
};
