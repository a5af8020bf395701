// kv_cache_manager.h -- the single owner of paged KV memory.
//
// Drop-in for the reference's KVCacheManager (src/include/kv_cache_manager.h:27-92):
// same block-granular primitives and accounting --
//   allocate_prompt  all-or-nothing, ceil(prompt/BLOCK) blocks, cur_len = prompt
//   append_token     grows the table only on a block boundary; on an empty pool
//                    returns false and leaves cur_len unchanged
//   free             returns the table to the free list in table order
//   slack            table capacity minus cur_len
//   slot_offset      element offset ((phys*Hkv + h)*BLOCK + in)*D
// and the same device layout per layer slice: [num_blocks, Hkv, BLOCK, D].
// Extensions (trailing constructor arguments with defaults): element type
// (KVC_F32 as the reference, or KVC_F16), n_layers slices laid out
// [n_layers][num_blocks][Hkv][BLOCK][D] (one allocation per K and V, as the
// reference's model path does, qwen_serve.cu:84-86), and a host-only mode
// (allocate_device = false) that keeps the accounting without a GPU.
#pragma once
#include <cstddef>
#include <stdexcept>
#include <string>

#include "../kvc_abi.h"
#include "block_alloc.h"
#include "sequence.h"

namespace kvc {
struct Error : std::runtime_error {
    int status;
    Error(int st, const std::string& what) : std::runtime_error(what), status(st) {}
};
inline void check(int st, const char* what) {
    if (st != KVC_OK) throw Error(st, std::string(what) + ": " + kvc_last_error());
}
inline int dtype_size(int dtype) { return dtype == KVC_F16 ? 2 : 4; }
}  // namespace kvc

struct KVCacheManager {
    int num_blocks, block_size, n_kv_heads, head_dim;
    int dtype = KVC_F32;
    int n_layers = 1;
    BlockAllocator alloc;
    float* k_pool = nullptr;  // base of the K allocation (reinterpret for KVC_F16)
    float* v_pool = nullptr;

    KVCacheManager(int num_blocks_, int block_size_, int n_kv_heads_, int head_dim_, int dtype_ = KVC_F32,
                   int n_layers_ = 1, bool allocate_device = true)
        : num_blocks(num_blocks_), block_size(block_size_), n_kv_heads(n_kv_heads_), head_dim(head_dim_),
          dtype(dtype_), n_layers(n_layers_ > 0 ? n_layers_ : 1), alloc(num_blocks_) {
        if (num_blocks <= 0 || block_size <= 0 || n_kv_heads <= 0 || head_dim <= 0)
            throw kvc::Error(KVC_ERR_ARG, "KVCacheManager: sizes must be positive");
        if (dtype != KVC_F32 && dtype != KVC_F16) throw kvc::Error(KVC_ERR_ARG, "KVCacheManager: bad dtype");
        if (!allocate_device) return;
        const size_t bytes = total_bytes_per_pool();
        void *k = nullptr, *v = nullptr;
        kvc::check(kvc_malloc(&k, bytes), "KVCacheManager K pool");
        if (kvc_malloc(&v, bytes) != KVC_OK) {
            kvc_free(k);
            kvc::check(KVC_ERR_NOMEM, "KVCacheManager V pool");
        }
        k_pool = static_cast<float*>(k);
        v_pool = static_cast<float*>(v);
        kvc::check(kvc_memset(k_pool, 0, bytes, nullptr), "KVCacheManager zero K");
        kvc::check(kvc_memset(v_pool, 0, bytes, nullptr), "KVCacheManager zero V");
        kvc::check(kvc_device_synchronize(), "KVCacheManager init");
    }
    ~KVCacheManager() {
        kvc_free(k_pool);
        kvc_free(v_pool);
    }
    KVCacheManager(const KVCacheManager&) = delete;
    KVCacheManager& operator=(const KVCacheManager&) = delete;

    // Elements of one layer slice of one pool (reference pool_elems()).
    size_t pool_elems() const { return (size_t)num_blocks * n_kv_heads * block_size * head_dim; }
    size_t layer_bytes() const { return pool_elems() * kvc::dtype_size(dtype); }
    size_t total_bytes_per_pool() const { return layer_bytes() * n_layers; }
    bool has_device() const { return k_pool != nullptr; }
    void* k_layer(int l) const { return reinterpret_cast<char*>(k_pool) + (size_t)l * layer_bytes(); }
    void* v_layer(int l) const { return reinterpret_cast<char*>(v_pool) + (size_t)l * layer_bytes(); }

    int free_blocks() const { return alloc.free_count(); }
    int used_blocks() const { return alloc.used_count(); }

    // Restore the free list; device contents are left as they are.
    void reset() { alloc.reset(); }

    int slack(const Sequence& s) const { return (int)s.block_table.size() * block_size - s.cur_len; }

    bool allocate_prompt(Sequence& s) {
        const int need = blocks_needed(s.prompt_len, block_size);
        if (alloc.free_count() < need) return false;
        for (int i = 0; i < need; ++i) s.block_table.push_back(alloc.alloc());
        s.cur_len = s.prompt_len;
        return true;
    }

    bool append_token(Sequence& s) {
        if (blocks_needed(s.cur_len + 1, block_size) > (int)s.block_table.size()) {
            const int b = alloc.alloc();
            if (b < 0) return false;
            s.block_table.push_back(b);
        }
        ++s.cur_len;
        return true;
    }

    void free(Sequence& s) {
        alloc.free_blocks(s.block_table);
        s.block_table.clear();
    }

    size_t slot_offset(int phys, int kv_head, int in_block) const {
        return (((size_t)phys * n_kv_heads + kv_head) * block_size + in_block) * head_dim;
    }
};
