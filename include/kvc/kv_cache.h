// kv_cache.h -- reference-named kernel launchers over the C ABI (kvc_abi.h).
//
// Same names, argument order and layouts as the reference's
// src/include/kv_cache.h:2-34 (fp32, MHA, null stream) and the fp16 GQA
// launchers of src/include/qwen_kernels.h:15-37, so existing call sites compile
// unchanged.  Differences a caller can see:
//   * each launcher returns the kvc_status (0 = ok) instead of void; the last
//     failure message is kvc_last_error();
//   * launch_batched_paged and launch_batched_paged_flash are one entry point: the
//     online fp32 softmax with split-K is the only implementation; the kernel plans
//     its chunks from the device lengths, so `cap` only raises its planning budget
//     (shapes without that path give a sequence longer than `cap` NaN outputs, never
//     a partial attention, and a report kvc_check_device_errors returns);
//   * launch_flash_decode allocates nothing per call: its partials live in a
//     grow-only library workspace (pass your own through kvc_flash_decode).
// Optional trailing arguments select a stream (hipStream_t as void*).
#pragma once
#include <hip/hip_fp16.h>

#include "../kvc_abi.h"

inline int launch_append(const float* k_new, const float* v_new, float* k_cache, float* v_cache, int pos, int H,
                         int D, int S, kvc_stream_t stream = nullptr) {
    return kvc_append(k_new, v_new, k_cache, v_cache, pos, H, D, S, KVC_F32, stream);
}

inline int launch_decode(const float* q, const float* k_cache, const float* v_cache, float* out, int cur_len, int H,
                         int D, int S, float scale, kvc_stream_t stream = nullptr) {
    return kvc_decode(q, k_cache, v_cache, out, cur_len, H, D, S, scale, KVC_F32, stream);
}

inline int launch_paged(const float* q, const float* k_pool, const float* v_pool, const int* block_table, float* out,
                        int cur_len, int H, int D, int BLOCK, float scale, kvc_stream_t stream = nullptr) {
    return kvc_paged_decode(q, k_pool, v_pool, block_table, out, cur_len, H, D, BLOCK, scale, KVC_F32, stream);
}

inline int launch_batched_decode(const float* q, const float* k_cache, const float* v_cache, const int* cur_len,
                                 float* out, int N, int H, int D, int MAXS, int cap, float scale,
                                 kvc_stream_t stream = nullptr) {
    return kvc_batched_decode(q, k_cache, v_cache, cur_len, out, N, H, H, D, MAXS, cap, scale, KVC_F32, nullptr, 0,
                              stream);
}

inline int launch_batched_paged(const float* q, const float* k_pool, const float* v_pool, const int* table_all,
                                const int* tab_off, const int* cur_len, float* out, int N, int H, int D, int BLOCK,
                                int cap, float scale, kvc_stream_t stream = nullptr) {
    return kvc_batched_paged_decode(q, k_pool, v_pool, table_all, tab_off, cur_len, out, N, H, H, D, BLOCK, cap, scale,
                                    KVC_F32, nullptr, 0, stream);
}

inline int launch_batched_paged_flash(const float* q, const float* k_pool, const float* v_pool, const int* table_all,
                                      const int* tab_off, const int* cur_len, float* out, int N, int H, int D,
                                      int BLOCK, int cap, float scale, kvc_stream_t stream = nullptr) {
    return launch_batched_paged(q, k_pool, v_pool, table_all, tab_off, cur_len, out, N, H, D, BLOCK, cap, scale,
                                stream);
}

inline int launch_flash_decode(const float* q, const float* k_cache, const float* v_cache, float* out, int cur_len,
                               int H, int D, int S, float scale, int num_splits, kvc_stream_t stream = nullptr) {
    return kvc_flash_decode(q, k_cache, v_cache, out, cur_len, H, D, S, scale, num_splits, KVC_F32, nullptr, 0,
                            stream);
}

// ---- fp16 / GQA family (qwen_kernels.h:15-37) --------------------------------
inline int qk_write_kv(const half* k, const half* v, half* k_pool, half* v_pool, const int* block_table_dev,
                       int start_pos, int L, int Hkv, int D, int BLOCK, kvc_stream_t stream = nullptr) {
    return kvc_write_kv(k, v, k_pool, v_pool, block_table_dev, start_pos, L, Hkv, D, BLOCK, KVC_F16, stream);
}

inline int qk_batched_write_kv(const half* k, const half* v, half* k_pool, half* v_pool, const int* table_all,
                               const int* tab_off, const int* wpos, int N, int Hkv, int D, int BLOCK,
                               kvc_stream_t stream = nullptr) {
    return kvc_batched_write_kv(k, v, k_pool, v_pool, table_all, tab_off, wpos, N, Hkv, D, BLOCK, KVC_F16, stream);
}

inline int qk_paged_causal_attn(const half* q, half* out, const half* k_pool, const half* v_pool,
                                const int* block_table_dev, int q_pos_base, int Nq, int Hq, int Hkv, int D, int BLOCK,
                                float scale, kvc_stream_t stream = nullptr) {
    return kvc_paged_causal_attn(q, out, k_pool, v_pool, block_table_dev, q_pos_base, Nq, Hq, Hkv, D, BLOCK, scale,
                                 KVC_F16, nullptr, 0, stream);
}

// As the reference, any N and BLOCK and no length bound: the kernel plans its own
// chunks from the device lengths (cap 0 = unknown; a batch of more sequences than one
// launch plans runs as consecutive launches, a shape without that path reads the
// longest length from the device).  With cap 0 the planning budget holds a mean length
// of up to 63 of the largest chunks (64 blocks for one- or two-head units, 1024 blocks
// on the matrix cores); past it the rows are NaN and kvc_check_device_errors reports
// it.  `cap`, after the stream, states a longer bound.
inline int qk_batched_paged_decode_attn(const half* q, half* out, const half* k_pool, const half* v_pool,
                                        const int* table_all, const int* tab_off, const int* cur_len, int N, int Hq,
                                        int Hkv, int D, int BLOCK, float scale, kvc_stream_t stream = nullptr,
                                        int cap = 0) {
    return kvc_batched_paged_decode(q, k_pool, v_pool, table_all, tab_off, cur_len, out, N, Hq, Hkv, D, BLOCK, cap,
                                    scale, KVC_F16, nullptr, 0, stream);
}
