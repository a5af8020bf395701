// qwen_kernels.h -- the reference's decoder-step kernel names over the C ABI.
//
// Same names, argument order and meaning as src/include/qwen_kernels.h:7-47 of the
// reference, so its model call sites (qwen_serve.cu, qwen_infer.cu) compile against
// this header unchanged.  The four attention-path launchers (qk_write_kv,
// qk_batched_write_kv, qk_paged_causal_attn, qk_batched_paged_decode_attn) live in
// kv_cache.h, included here.  Differences a caller can see:
//   * every launcher returns the kvc_status (0 = ok) instead of void; the last
//     failure message is kvc_last_error();
//   * row widths (H, N, n, D) are multiples of 8: the kernels move 16-byte vectors;
//   * qk_embed_gather reads any non-negative id as a row (the reference does not
//     bound it either); negative ids give zero rows;
//   * the stream is a hipStream_t (as void*); qk_rope_pos takes one as an optional
//     trailing argument (the reference's runs on the null stream).
// The qkcuda_* forms read their position from device memory, so a captured graph
// replays at advancing positions (qwen_infer.cu:135-214).
#pragma once
#include <climits>

#include "../kvc_abi.h"
#include "kv_cache.h"

// qwen_kernels.h:7 -- out[L, H] = embed[ids[r], :]
inline int qk_embed_gather(half* out, const half* embed, const int* ids, int L, int H, kvc_stream_t stream = nullptr) {
    return kvc_embed_gather(out, embed, ids, L, H, INT_MAX, stream);
}

// qwen_kernels.h:8 -- out = in * rsqrt(mean(in^2) + eps) * w, per row of H
inline int qk_rmsnorm(half* out, const half* in, const half* w, int L, int H, float eps,
                      kvc_stream_t stream = nullptr) {
    return kvc_rmsnorm(out, in, w, L, H, eps, stream);
}

// qwen_kernels.h:9 -- x[L, N] += bias[N]
inline int qk_add_bias(half* x, const half* bias, int L, int N, kvc_stream_t stream = nullptr) {
    return kvc_add_bias(x, bias, L, N, stream);
}

// qwen_kernels.h:10 -- x[n] += y[n]
inline int qk_add_residual(half* x, const half* y, int n, kvc_stream_t stream = nullptr) {
    return kvc_add_residual(x, y, n < 0 ? 0 : (size_t)n, stream);
}

// qwen_kernels.h:11 -- rotate-half rotary embedding of x [L, n_heads, D] at positions pos_base + r
inline int qk_rope(half* x, int L, int n_heads, int D, int pos_base, float theta, kvc_stream_t stream = nullptr) {
    return kvc_rope(x, nullptr, pos_base, L, n_heads, D, theta, stream);
}

// qwen_kernels.h:12 -- out = silu(gate) * up
inline int qk_silu_mul(half* out, const half* gate, const half* up, int n, kvc_stream_t stream = nullptr) {
    return kvc_silu_mul(out, gate, up, n < 0 ? 0 : (size_t)n, stream);
}

// qwen_kernels.h:22 -- *d_idx = first index of the maximum of fp32 logits[0, n)
inline int qk_argmax(const float* logits, int n, int* d_idx, kvc_stream_t stream = nullptr) {
    return kvc_argmax(logits, 1, n, d_idx, stream);
}

// qwen_kernels.h:24 -- rotary embedding of row r at position pos[r] (device array)
inline int qk_rope_pos(half* x, int n_rows, int n_heads, int D, const int* pos, float theta,
                       kvc_stream_t stream = nullptr) {
    return kvc_rope(x, pos, 0, n_rows, n_heads, D, theta, stream);
}

// qwen_kernels.h:42 -- qk_rope at positions *pos_base + r (device memory)
inline int qkcuda_rope(half* x, int L, int n_heads, int D, int* pos_base, float theta,
                       kvc_stream_t stream = nullptr) {
    return kvc_rope_dev(x, pos_base, L, n_heads, D, theta, stream);
}

// qwen_kernels.h:43-44 -- qk_write_kv at positions *start_pos + r (device memory)
inline int qkcuda_write_kv(const half* k, const half* v, half* k_pool, half* v_pool, const int* block_table_dev,
                           int* start_pos, int L, int Hkv, int D, int BLOCK, kvc_stream_t stream = nullptr) {
    return kvc_write_kv_dev(k, v, k_pool, v_pool, block_table_dev, start_pos, L, Hkv, D, BLOCK, KVC_F16, stream);
}

// qwen_kernels.h:45-47 -- qk_paged_causal_attn with the first query at *q_pos_base
// (device memory); the kernel plans its chunks from that position.  Outside stream
// capture the partials go to the library's per-stream workspace (up to 512 queries at
// the matrix-core shapes, 1024 otherwise).  The reference captures this call in a graph
// (qwen_infer.cu:145-162, one query per step); under capture nothing may be allocated,
// so it takes the allocation-free entry point, whose partials live in a 4 MiB static
// device array per GPU: about 17 queries of the 14q/2kv D 64 shape at most (larger calls
// are refused with KVC_ERR_UNSUPPORTED), and captured calls that overlap on one GPU race.
inline int qkcuda_paged_causal_attn(const half* q, half* out, const half* k_pool, const half* v_pool,
                                    const int* block_table_dev, int* q_pos_base, int Nq, int Hq, int Hkv, int D,
                                    int BLOCK, float scale, kvc_stream_t stream = nullptr) {
    int capturing = 0;
    const int rc = kvc_stream_is_capturing(stream, &capturing);
    if (rc) return rc;
    if (capturing)
        return kvc_paged_causal_attn_dev_noalloc(q, out, k_pool, v_pool, block_table_dev, q_pos_base, Nq, Hq, Hkv, D,
                                                 BLOCK, scale, KVC_F16, stream);
    return kvc_paged_causal_attn_dev(q, out, k_pool, v_pool, block_table_dev, q_pos_base, Nq, Hq, Hkv, D, BLOCK,
                                     scale, KVC_F16, nullptr, 0, stream);
}
