/* kvc_abi.h -- C ABI of the MI355X (gfx950) paged-decode library libkvcache_amd.so.
 *
 * Drop-in boundary for the decode hot path of kimxinw/kvcache.  Every kernel
 * entry point mirrors one reference launcher (argument order kept, cited as
 * reference file:line) and extends it with:
 *   - an element type `dtype` (KVC_F32 as the reference, or KVC_F16),
 *   - separate query / KV head counts (Hq, Hkv) for grouped-query attention,
 *   - an explicit HIP stream (`stream` is a hipStream_t; NULL = null stream),
 *   - caller-provided workspace for split-K partials (NULL = a grow-only buffer
 *     owned by the library, one per (device, stream), allocated on first need;
 *     calls on one stream are ordered by it, calls on different streams never
 *     share partials; refused with KVC_ERR_STATE while the stream is capturing),
 *   - an int status instead of void: 0 = KVC_OK, otherwise a KVC_ERR_* code,
 *     with a readable message from kvc_last_error().
 * No function throws across this boundary.  All launches are asynchronous on
 * `stream`; every pointer argument named *_pool, *_cache, q, out, k, v, table*
 * or *len* is a device pointer unless stated otherwise.
 *
 * Layouts (elements of dtype):
 *   contiguous cache [H(kv), S, D] (single sequence) or [N, Hkv, MAXS, D];
 *   paged pool       [num_blocks, Hkv, BLOCK, D]  (reference kv_cache_manager.h:30);
 *   q / out          [N, Hq, D];
 *   table_all        concatenated block tables, sequence s starts at tab_off[s].
 *
 * Deployment: run with HIP_FORCE_DEV_KERNARG=1 in the environment (set before HIP
 * initialises; the Python binding sets it when unset).  Every decode workgroup reads
 * its parameter block from the kernel-argument segment; where the HIP runtime's
 * default places that segment in host memory, each read crosses PCIe (MI355X, same
 * box: config-2 decode 37.4 vs 33.5 us per launch, one config-4 layer 8.0 vs 6.0 us).
 */
#ifndef KVC_ABI_H
#define KVC_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kvc_stream_t; /* a hipStream_t */

enum kvc_status {
    KVC_OK = 0,
    KVC_ERR_ARG = 1,         /* bad shape / null pointer / out-of-range argument */
    KVC_ERR_UNSUPPORTED = 2, /* shape the kernels do not implement (e.g. head_dim) */
    KVC_ERR_HIP = 3,         /* a HIP runtime call failed */
    KVC_ERR_NOMEM = 4,       /* device or pinned allocation failed / pool exhausted */
    KVC_ERR_WORKSPACE = 5,   /* caller workspace smaller than required */
    KVC_ERR_STATE = 6        /* call not valid in the object's current state */
};
enum kvc_dtype { KVC_F32 = 0, KVC_F16 = 1 };
/* How an engine step launches decode: host-planned work list (kvc_decode_plan +
 * kvc_batched_paged_decode_planned) or device lengths (kvc_batched_paged_decode_split). */
enum kvc_decode_path { KVC_DECODE_PLANNED = 0, KVC_DECODE_DEVICE_LENGTHS = 1 };

/* ---- library ---------------------------------------------------------- */
int         kvc_version(void);                 /* 100*major + minor */
const char* kvc_status_string(int status);
const char* kvc_last_error(void);               /* last failure on this host thread */
int         kvc_device_count(int* count);
/* Tuning knobs (process-wide): "fused_merge" (how split partials are merged:
 * -1 automatic, 0 a separate merge kernel, 1 the last-arriving chunk merges
 * behind agent-scope fences, 2 the last-arriving chunk merges partials written
 * and read with coherent atomic accesses), "target_units" (automatic split:
 * workgroups to aim for),
 * "min_chunk_bytes" (automatic split: least K+V bytes per workgroup),
 * "waves_per_block" (0 automatic, 4 or 8 waves cooperating on one chunk),
 * "batch" (2, 4 or 8 wave-loads per double-buffered batch when a wave serves at
 * most two query heads), "last_chunk_first" (1: dispatch later chunks first),
 * "mfma" (grouped-query heads on the matrix cores: -1 automatic, 0 off, 1 on),
 * "wg_per_cu" (cap on decode workgroups per CU through reserved LDS: -1
 * automatic, 0 none, n), "split_first" (planner: chunks of split sequences
 * before whole sequences), "mfma_min_chunk" (planner, grouped-query heads on the
 * matrix cores: tokens below which a sequence stays in one unit, default 1024),
 * "self_plan" (device-length decode with the automatic split: 1 = the kernel
 * derives the planner's units from the device lengths, 0 = a chunk x sequence x
 * head grid sized by cap), "self_grid" (self-planned launches: 0 = one workgroup
 * per resident slot, n = at most n workgroups, each then serving several units),
 * "self_prefetch_kib" (self-planned paged launches: about this many KiB of K and V,
 * the first blocks of every sequence, are read ahead while the kernel plans;
 * default 32768, 0 = none), "self_prefetch_min_len" (... of the sequences of at
 * least this many tokens, default 256; at most a quarter of each is read ahead),
 * "self_prefetch_xcd" (1: each KV head's slice is read ahead on the XCD whose
 * units read it), "self_lead_tokens" (self-planned launches on the VALU kernel: a
 * sequence of at most this many tokens is attended whole while the kernel plans the
 * others, default 320, 0 = none; at most the largest chunk).
 * The matrix-core path takes fp16 K/V, head_dim 64 or 128, 3..16 query heads per
 * KV head and, paged, a power-of-two BLOCK >= 16; other shapes use the VALU
 * kernels. */
int         kvc_set_tuning(const char* key, int value);
int         kvc_get_tuning(const char* key, int* value);

/* ---- device memory / stream / event plumbing (thin HIP wrappers) ------- */
int kvc_malloc(void** dptr, size_t bytes);
int kvc_free(void* dptr);
int kvc_host_alloc(void** hptr, size_t bytes);  /* pinned host memory */
int kvc_host_free(void* hptr);
int kvc_memcpy_h2d(void* dst, const void* src, size_t bytes, kvc_stream_t stream);
int kvc_memcpy_d2h(void* dst, const void* src, size_t bytes, kvc_stream_t stream);
int kvc_memcpy_d2d(void* dst, const void* src, size_t bytes, kvc_stream_t stream);
int kvc_memset(void* dst, int value, size_t bytes, kvc_stream_t stream);
int kvc_stream_create(kvc_stream_t* stream);    /* default priority */
int kvc_stream_destroy(kvc_stream_t stream);
int kvc_stream_synchronize(kvc_stream_t stream);
int kvc_device_synchronize(void);
int kvc_event_create(void** ev);
int kvc_event_destroy(void* ev);
int kvc_event_record(void* ev, kvc_stream_t stream);
int kvc_event_synchronize(void* ev);
/* work queued on `stream` after this call waits for `ev` (no host synchronisation): orders a copy
 * stream and a compute stream */
int kvc_stream_wait_event(kvc_stream_t stream, void* ev);
int kvc_event_elapsed_ms(float* ms, void* start, void* stop); /* synchronizes on stop */
/* HIP graphs (stream capture): the launches made on `stream` between begin and end
 * are recorded, not run; end instantiates them as one executable graph, launch
 * replays it on a stream (the reference captures its decode step as a CUDA graph,
 * qwen_infer.cu:135-214).  Only graph-safe entry points may be captured: those that
 * allocate nothing and take per-step counts from device memory (the *_dev and
 * dev_rows forms below). */
/* No counterpart in the reference; a measurement aid for the practical ceiling of the
 * decode's access pattern.  Reads the K/V bytes that kvc_batched_paged_decode_planned
 * reads for the same work list (kvc_decode_plan for Hq/Hkv/D/BLOCK/dtype), unit by unit in
 * the same grid order, with the same 16-byte-per-lane loads and buffer descriptors, and
 * computes nothing from them (sink: n_units ints, written only in the unlikely event
 * that a unit's xor of its bytes equals a fixed constant).  The chunks of the plan must
 * span at most 64 blocks (every plan of the one/two-head shapes does); BLOCK must hold a
 * power-of-two number of 1 KiB loads per KV head. */
int kvc_read_probe_planned(const void* k_pool, const void* v_pool, const int* table_all, int table_len,
                           const int* work, int n_units, int Hq, int Hkv, int D, int BLOCK, int dtype, int* sink,
                           kvc_stream_t stream);
/* No counterpart in the reference; a measurement aid: one launch of an empty kernel of
 * `blocks` (1..65535) one-wave workgroups on `stream`.  Timed back to back it gives the
 * launch floor that every decode launch pays. */
int kvc_empty_launch(int blocks, kvc_stream_t stream);
/* 1 in *capturing when `stream` is being captured into a graph (0 for the null stream). */
int kvc_stream_is_capturing(kvc_stream_t stream, int* capturing);
/* Device-side failure reports.  A device-length decode launch that cannot attend a
 * sequence whole -- a length past the stated cap on the explicit-split grid, a batch past
 * the self-planned record budget, a contiguous length past MAXS -- writes NaN in that
 * sequence's output rows (never a partial attention) and stores a report in a per-device
 * word of pinned host memory.  kvc_check_device_errors synchronizes `stream` and returns
 * KVC_ERR_ARG (message in kvc_last_error) when such a report is pending, KVC_OK otherwise;
 * it clears the report.  The next device-length decode call on the device
 * (kvc_batched_decode*, kvc_batched_paged_decode*, kvc_paged_causal_attn_dev) also returns
 * a report that has reached the host by then, without launching, and clears it.  No
 * counterpart in the reference, whose launchers return void (kv_cache.h:2-34). */
int kvc_check_device_errors(kvc_stream_t stream);
int kvc_graph_begin(kvc_stream_t stream);
int kvc_graph_end(kvc_stream_t stream, void** graph_exec);
int kvc_graph_launch(void* graph_exec, kvc_stream_t stream);
int kvc_graph_destroy(void* graph_exec);

/* One packed per-step upload: copies `bytes` from (preferably pinned) host
 * memory to the device with a single async copy on `stream`.  Replaces the
 * three blocking cudaMemcpy of model_runner.h:70-72. */
int kvc_step_upload(void* dst_device, const void* src_host, size_t bytes, kvc_stream_t stream);

/* Deterministic N(0, stddev^2) fill of n elements of dtype (synthetic K/V/q). */
int kvc_fill_normal(void* dst, size_t n, int dtype, uint64_t seed, float stddev, kvc_stream_t stream);

/* ---- K/V append ------------------------------------------------------- */
/* launch_append (kv_cache.h:2-4, kv_cache.cu:5-19): k_new/v_new [H,D] -> cache[h,pos,:] of [H,S,D]. */
int kvc_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
               int pos, int H, int D, int S, int dtype, kvc_stream_t stream);

/* qk_write_kv (qwen_kernels.h:15-16, qwen_kernels.cu:111-126): L tokens k/v [L,Hkv,D]
 * into the paged pool at positions start_pos..start_pos+L-1 of one block table. */
int kvc_write_kv(const void* k, const void* v, void* k_pool, void* v_pool,
                 const int* block_table, int start_pos, int L, int Hkv, int D, int BLOCK,
                 int dtype, kvc_stream_t stream);

/* qkcuda_write_kv (qwen_kernels.h:43-44, qwen_kernels.cu:128-143): kvc_write_kv with the
 * start position read from device memory (*dev_start_pos), so a captured graph can be
 * replayed at advancing positions.  Rows whose position is negative are skipped. */
int kvc_write_kv_dev(const void* k, const void* v, void* k_pool, void* v_pool,
                     const int* block_table, const int* dev_start_pos, int L, int Hkv, int D, int BLOCK,
                     int dtype, kvc_stream_t stream);

/* qk_batched_write_kv (qwen_kernels.h:30-32, qwen_kernels.cu:270-290): one token per
 * sequence, k/v [N,Hkv,D] -> pool at position wpos[r] of table table_all+tab_off[r].
 * Rows with wpos[r] < 0 are skipped. */
int kvc_batched_write_kv(const void* k, const void* v, void* k_pool, void* v_pool,
                         const int* table_all, const int* tab_off, const int* wpos,
                         int N, int Hkv, int D, int BLOCK, int dtype, kvc_stream_t stream);

/* Slot-mapped write (no reference counterpart; the scheduler precomputes
 * slot = phys*BLOCK + pos%BLOCK per row): k/v [rows,Hkv,D] -> pool; slot < 0 skips. */
int kvc_write_kv_slots(const void* k, const void* v, void* k_pool, void* v_pool,
                       const int* slot_map, int rows, int Hkv, int D, int BLOCK,
                       int dtype, kvc_stream_t stream);

/* ---- decode attention --------------------------------------------------- */
/* launch_decode (kv_cache.h:5-6, decode_attn.cu:5-52): one sequence, contiguous [H,S,D]. */
int kvc_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
               int cur_len, int H, int D, int S, float scale, int dtype, kvc_stream_t stream);

/* launch_paged (kv_cache.h:9-11, paged.cu:7-62): one sequence, pool [NB,H,BLOCK,D].
 * Bit-identical to kvc_decode on the same logical data. */
int kvc_paged_decode(const void* q, const void* k_pool, const void* v_pool,
                     const int* block_table, void* out, int cur_len,
                     int H, int D, int BLOCK, float scale, int dtype, kvc_stream_t stream);

/* launch_batched_decode (kv_cache.h:15-17, batched.cu:49-88,132-138): caches
 * [N,Hkv,MAXS,D], lengths cur_len[N] (device), cap = max length (host; 0: MAXS bounds
 * every length).  A length past MAXS gets NaN rows and a device error report
 * (kvc_check_device_errors). */
int kvc_batched_decode(const void* q, const void* k_cache, const void* v_cache,
                       const int* cur_len, void* out, int N, int Hq, int Hkv, int D,
                       int MAXS, int cap, float scale, int dtype,
                       void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* launch_batched_paged / launch_batched_paged_flash (kv_cache.h:20-27,
 * batched.cu:97-147,157-207) and qk_batched_paged_decode_attn (qwen_kernels.h:35-37,
 * qwen_kernels.cu:293-335): one query per sequence over its pages [0,cur_len[s]).
 * Bit-identical to kvc_batched_decode on the same logical data (at BLOCK 16 or 32).
 * cap: the caller's bound on every cur_len, or 0 (unknown).
 *  - Shapes with a self-planned path (tuning "self_plan"; a power-of-two BLOCK of at
 *    least 1024 / (D * element bytes) tokens) plan from the device lengths; cap only
 *    raises the planning budget.  Batches of more than 1024 sequences (512 on the matrix
 *    cores) run as consecutive launches of that many.  The budget holds 64 partial
 *    records per (sequence, head): a batch whose mean length passes 63 x the largest
 *    chunk (64,512 tokens for one- or two-head units at BLOCK 16) with cap 0 gets NaN
 *    rows and a device error report (kvc_check_device_errors); stating cap avoids it.
 *  - Other shapes with cap 0 read the longest length from the device (one
 *    synchronisation; refused with KVC_ERR_STATE under stream capture); with cap > 0 a
 *    sequence longer than cap gets NaN rows and a device error report -- never a
 *    silent partial attention. */
int kvc_batched_paged_decode(const void* q, const void* k_pool, const void* v_pool,
                             const int* table_all, const int* tab_off, const int* cur_len,
                             void* out, int N, int Hq, int Hkv, int D, int BLOCK, int cap,
                             float scale, int dtype,
                             void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* Same as kvc_batched_paged_decode with an explicit split size: each sequence is
 * cut into chunks of split_tokens tokens (a multiple of BLOCK; 0 = automatic),
 * chunks run in parallel and are merged by log-sum-exp.  Long-context split-K
 * (flash_decode.cu:103-126 generalised to paged, batched, GQA). */
int kvc_batched_paged_decode_split(const void* q, const void* k_pool, const void* v_pool,
                                   const int* table_all, const int* tab_off, const int* cur_len,
                                   void* out, int N, int Hq, int Hkv, int D, int BLOCK, int cap,
                                   float scale, int dtype, int split_tokens,
                                   void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* kvc_batched_decode with an explicit split size (any positive token count). */
int kvc_batched_decode_split(const void* q, const void* k_cache, const void* v_cache,
                             const int* cur_len, void* out, int N, int Hq, int Hkv, int D,
                             int MAXS, int cap, float scale, int dtype, int split_tokens,
                             void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* Workspace (bytes) needed by the batched calls for a batch of N sequences whose
 * longest is cap tokens, with split_tokens as given (0 = the automatic choice).
 * BLOCK = 0 for the contiguous calls. */
size_t kvc_decode_workspace_size(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int split_tokens, int dtype);
/* The split size the automatic choice picks for this shape (BLOCK = 0: contiguous). */
int kvc_decode_auto_split(int N, int Hq, int Hkv, int D, int BLOCK, int cap, int dtype);

/* Planned decode for host-known lengths (the serving path: the scheduler knows
 * every length when it builds the step).  kvc_decode_plan cuts each sequence into
 * near-equal block-aligned chunks and writes the units (chunks of split sequences
 * first, each group longest first) into `work` (host memory; work == NULL only
 * reports *n_units / *n_records), kvc_decode_plan_entry_ints() ints per unit:
 * {s, kv_head_slot | chunk << 16, j0, j1, chunks | inline_ids << 16, record group,
 * counter, table index of the chunk's first block}, followed on the grouped-query
 * matrix-core path (64-int entries) by up to 56 of the chunk's block ids copied
 * from host_table_all (may be NULL: then none are inlined).  host_tab_off (N+1,
 * may be NULL: tables packed in sequence order) locates each sequence's table in
 * table_all.  target_tokens = 0 picks the chunk size.  capacity is in units.  The
 * caller copies the work list to the device (e.g. inside its per-step upload) and
 * runs kvc_batched_paged_decode_planned with the same shape and tables; every
 * block-id read is bounded by table_len (ints in table_all).  Partials of split
 * sequences are merged by the last chunk to finish, inside the same kernel.
 * A plan depends on the tuning knobs ("mfma", "waves_per_block", "mfma_min_chunk"): plan and launch
 * under the same settings.  Units naming a sequence or KV head outside N / Hkv
 * are skipped. */
int kvc_decode_plan_entry_ints(int Hq, int Hkv, int D, int BLOCK, int dtype);
int kvc_decode_plan(const int* host_lens, const int* host_tab_off, const int* host_table_all, int host_table_len,
                    int N, int Hq, int Hkv, int D, int BLOCK, int dtype, int target_tokens, int* work, int capacity,
                    int* n_units, int* n_records);
size_t kvc_decode_planned_workspace_size(int Hq, int Hkv, int D, int BLOCK, int dtype, int n_records);
int kvc_batched_paged_decode_planned(const void* q, const void* k_pool, const void* v_pool,
                                     const int* table_all, int table_len, void* out,
                                     int N, int Hq, int Hkv, int D, int BLOCK, float scale,
                                     int dtype, const int* work, int n_units, int n_records,
                                     void* workspace, size_t workspace_bytes, kvc_stream_t stream);
/* The model step's per-layer pair qk_batched_write_kv + qk_batched_paged_decode_attn
 * (qwen_kernels.h:15-16,30-37; qwen_serve.cu:130-160) in one planned launch: row
 * s of k_new / v_new ([N][Hkv][D]) belongs at position wpos[s] of sequence s, a
 * position inside its attended length (the step's new token, wpos = len - 1).
 * The unit whose chunk holds it attends over the new row taken from k_new/v_new
 * and stores the row into the pools, so the result and the pools afterwards
 * equal those of the write followed by the decode.  wpos[s] outside [0, len) is
 * not written. */
int kvc_batched_paged_append_decode_planned(const void* q, const void* k_new, const void* v_new, const int* wpos,
                                            void* k_pool, void* v_pool, const int* table_all, int table_len,
                                            void* out, int N, int Hq, int Hkv, int D, int BLOCK, float scale,
                                            int dtype, const int* work, int n_units, int n_records,
                                            void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* The chunk target (tokens) kvc_decode_plan uses for these lengths and target_tokens:
 * sequences up to 1.5x this length stay whole, longer ones are cut into near-equal
 * block-aligned chunks of about this length.  Units run split chunks first, then
 * longest first in 64 length buckets of target/42 tokens each. */
int kvc_decode_plan_chunk(const int* host_lens, int N, int Hq, int Hkv, int D, int BLOCK, int dtype,
                          int target_tokens, int* chunk_tokens);

/* Upper bound on the units (and partial records) of any plan of N sequences holding
 * at most total_tokens tokens: the capacity a graph-safe launch is sized for. */
int kvc_decode_plan_capacity(int N, long long total_tokens, int Hq, int Hkv, int D, int BLOCK, int dtype,
                             int* max_units);

/* Graph-safe form of the two planned launches above (no counterpart in the
 * reference, whose graph variants read positions through device pointers,
 * qwen_kernels.cu:83-99,128-143,187-226): the step's {N, n_units, n_records} are
 * read from dev_counts[0..2] in device memory, so one captured launch serves every
 * step.  N_cap, units_cap and records_cap are capacities: the grid is units_cap
 * workgroups (those past the step's n_units exit at once), `work` holds units_cap
 * entries, the workspace is sized for records_cap.  k_new == NULL: no append. */
int kvc_batched_paged_decode_planned_dev(const void* q, const void* k_new, const void* v_new, const int* wpos,
                                        void* k_pool, void* v_pool, const int* table_all, int table_len, void* out,
                                        int N_cap, int Hq, int Hkv, int D, int BLOCK, float scale, int dtype,
                                        const int* work, int units_cap, int records_cap, const int* dev_counts,
                                        void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* qk_paged_causal_attn (qwen_kernels.h:19-21, qwen_kernels.cu:146-181): the prompt
 * (prefill) attention of one sequence.  Query i of q [Nq, Hq, D] sits at position
 * q_pos_base + i and attends causally to positions 0 .. q_pos_base + i of the
 * paged pools through block_table; out is [Nq, Hq, D].  Runs the batched decode
 * kernels with query i as a sequence of length q_pos_base + i + 1 sharing the one
 * table (grouped-query heads on the matrix cores, long prefixes split and merged).
 * workspace as for the batched decode (NULL: library-owned). */
int kvc_paged_causal_attn(const void* q, void* out, const void* k_pool, const void* v_pool, const int* block_table,
                          int q_pos_base, int Nq, int Hq, int Hkv, int D, int BLOCK, float scale, int dtype,
                          void* workspace, size_t workspace_bytes, kvc_stream_t stream);
size_t kvc_paged_causal_attn_workspace_size(int q_pos_base, int Nq, int Hq, int Hkv, int D, int BLOCK, int dtype);

/* qkcuda_paged_causal_attn (qwen_kernels.h:45-47, qwen_kernels.cu:187-226): as
 * kvc_paged_causal_attn with the first query's position read from device memory
 * (*dev_q_pos_base), for captured graphs.  The kernel plans its own chunks from that
 * position (no host-side length); Nq <= 512 on the matrix-core path, 1024 otherwise,
 * and BLOCK a power of two whose block of one KV head holds at least 1 KiB
 * (BLOCK * D * element size >= 1024: BLOCK >= 16 for fp16 D 32, >= 8 for fp16 D 64);
 * other shapes are refused with KVC_ERR_UNSUPPORTED. */
int kvc_paged_causal_attn_dev(const void* q, void* out, const void* k_pool, const void* v_pool,
                              const int* block_table, const int* dev_q_pos_base, int Nq, int Hq, int Hkv, int D,
                              int BLOCK, float scale, int dtype, void* workspace, size_t workspace_bytes,
                              kvc_stream_t stream);
size_t kvc_paged_causal_attn_dev_workspace_size(int Nq, int Hq, int Hkv, int D, int BLOCK, int dtype);

/* No counterpart in the reference: kvc_paged_causal_attn_dev for callers that cannot
 * allocate (code under HIP graph capture -- the reference captures
 * qkcuda_paged_causal_attn, qwen_infer.cu:145-162 --, tight serving loops, harnesses
 * that forbid allocation).  It allocates nothing: its split-K partials and counters
 * live in a static device array of 4 MiB per GPU (kvc_paged_causal_attn_dev_workspace_size
 * must not exceed it: about 17 queries of the 14q/2kv, D 64 shape; larger sizes are
 * refused with KVC_ERR_UNSUPPORTED).  Every call on a GPU shares that GPU's array,
 * so calls that overlap on one GPU (other streams, other threads) race.  The array's
 * device address is resolved on the first call on each GPU. */
int kvc_paged_causal_attn_dev_noalloc(const void* q, void* out, const void* k_pool, const void* v_pool,
                                      const int* block_table, const int* dev_q_pos_base, int Nq, int Hq, int Hkv,
                                      int D, int BLOCK, float scale, int dtype, kvc_stream_t stream);

/* ---- decoder-step operations around the attention path (a Qwen2-shaped layer) ----
 * fp16 activations and weights, fp32 arithmetic; row widths multiples of 8.
 * qk_embed_gather (qwen_kernels.h:7): out[L,H] = embed[ids[r]] (ids outside [0,V) give zeros).
 * qk_rmsnorm (:8): out = in * rsqrt(mean(in^2) + eps) * w per row of H.
 * qk_add_bias (:9): x[L,N] += bias[N].   qk_add_residual (:10): x[n] += y[n].
 * qk_silu_mul (:12): out = silu(gate) * up.
 * qk_rope / qk_rope_pos (:11,24): x [L, n_heads, D], rotate-half rotary embedding at
 *   position pos[r] (pos != NULL) or pos_base + r, frequencies theta^(-2t/D).
 * qk_argmax (:22): out[r] = first index of the maximum of fp32 logits[r, 0..V).
 * kvc_linear: the linear layers (cuBLAS in the reference, rocBLAS here):
 *   y[M,N] = x[M,K] w[N,K]^T, fp16 inputs, fp32 accumulation, y fp16 or fp32. */
int kvc_embed_gather(void* out, const void* embed, const int* ids, int L, int H, int V, kvc_stream_t stream);
/* graph-safe gather: rows [0, *dev_rows) of at most L_cap (row count in device memory) */
int kvc_embed_gather_dev(void* out, const void* embed, const int* ids, const int* dev_rows, int L_cap, int H, int V,
                         kvc_stream_t stream);
int kvc_rmsnorm(void* out, const void* in, const void* w, int L, int H, float eps, kvc_stream_t stream);
int kvc_add_bias(void* x, const void* bias, int L, int N, kvc_stream_t stream);
int kvc_add_residual(void* x, const void* y, size_t n, kvc_stream_t stream);
int kvc_silu_mul(void* out, const void* gate, const void* up, size_t n, kvc_stream_t stream);
int kvc_rope(void* x, const int* pos, int pos_base, int L, int n_heads, int D, float theta, kvc_stream_t stream);
/* qkcuda_rope (qwen_kernels.h:42, qwen_kernels.cu:83-99): positions *dev_pos_base + r. */
int kvc_rope_dev(void* x, const int* dev_pos_base, int L, int n_heads, int D, float theta, kvc_stream_t stream);
int kvc_argmax(const float* logits, int L, int V, int* out, kvc_stream_t stream);
int kvc_linear(void* y, const void* x, const void* w, int M, int N, int K, int out_dtype, kvc_stream_t stream);

/* ---- decode-step linear layers over at most 32 rows (one per running sequence) ----
 * Weight-streaming matrix-core kernels with the surrounding ops fused; each replaces a
 * cuBLAS GEMM plus the elementwise kernels after it in the reference's decode step
 * (qwen_serve.cu:127-175).  fp16 rows and weights ([out, in] row-major), fp32
 * accumulation, results rounded to fp16 where the op-by-op path stores them.
 * 1 <= M <= 32; K a multiple of 32; norm_w != NULL applies RMSNorm(x) * norm_w
 * (qk_rmsnorm, qwen_kernels.h:8) to the rows first (K <= 1024 then; kvc_rows_qkv,
 * kvc_rows_swiglu and kvc_rows_lm_head need K <= 1024 in any case).
 * Workspace (split-K partials, arrival counters, argmax candidates): 256-byte aligned,
 * kvc_rows_workspace_size(N, K) bytes, ZERO-FILLED before its first use; every call
 * leaves its counters zero again, so one workspace serves all calls of a stream.
 * kvc_rows_linear: y[M,N] = A W^T (fp16), or y += A W^T when residual != 0 (qk_add,
 *   qwen_kernels.h:10); N a multiple of 32; y must not alias x.
 * kvc_rows_qkv: q|k|v = A [wq;wk;wv]^T + [bq;bk;bv] (w_qkv [(Hq+2Hkv)D, H]), then the
 *   rotary embedding of q and k at position pos[r] (qk_rope_pos, qwen_kernels.h:24);
 *   q [M, Hq*D], k and v [M, Hkv*D]; D a multiple of 32.
 * kvc_rows_swiglu: act[M,I] = silu(A wg^T) * (A wu^T) (qk_silu_mul, qwen_kernels.h:12),
 *   w_gate_up = [wg; wu] as [2I, H]; I a multiple of 16.
 * kvc_rows_lm_head: logits[M,V] = A w^T in fp32 (logits may be NULL) and tokens[r] =
 *   first index of the row maximum (qk_argmax, qwen_kernels.h:22); V a multiple of 32.
 * dev_rows != NULL (graph-safe launches): the row count is read from device memory and
 *   M is its capacity (<= 32).
 * kvc_rows_set_tuning: overrides, -1 = automatic: K splits of layers with K > 1024,
 *   column groups (32 outputs) per workgroup, kernel shape 0..3 (4 waves x 7 k steps,
 *   8 waves x 4, 4 or 8 waves x 4 with K split).  The workspace size depends on them. */
size_t kvc_rows_workspace_size(int N, int K);
int kvc_rows_linear(void* y, const void* x, const void* w, int M, int N, int K, const void* norm_w, float eps,
                    int residual, const int* dev_rows, void* workspace, size_t workspace_bytes, kvc_stream_t stream);
int kvc_rows_qkv(void* q, void* k, void* v, const void* x, const void* norm_w, float eps, const void* w_qkv,
                 const void* b_qkv, const int* pos, int M, int H, int Hq, int Hkv, int D, float theta,
                 const int* dev_rows, kvc_stream_t stream);
int kvc_rows_swiglu(void* act, const void* x, const void* norm_w, float eps, const void* w_gate_up, int M, int I,
                    int H, const int* dev_rows, kvc_stream_t stream);
int kvc_rows_lm_head(float* logits, int* tokens, const void* x, const void* norm_w, float eps, const void* w, int M,
                     int V, int H, const int* dev_rows, void* workspace, size_t workspace_bytes,
                     kvc_stream_t stream);
int kvc_rows_set_tuning(int splits, int groups_per_wg, int shape);

/* The linear layers between two attention launches of a decode step as ONE launch:
 * the tail of layer l -- x += att W_o^T; act = silu(n W_g^T) * (n W_u^T) with
 * n = RMSNorm(x) * ln2; x += act W_d^T -- then the head of layer l + 1 -- q|k|v =
 * rotary(RMSNorm(x) * ln1 [wq;wk;wv]^T + b) at positions pos -- in the fused kernels'
 * shapes and rounding, phases separated by grid barriers inside the launch
 * (qwen_serve.cu:127-175 runs them as GEMMs plus one kernel per elementwise op; no
 * single counterpart in the reference).  Results equal kvc_rows_linear (o_proj,
 * residual), kvc_rows_swiglu, kvc_rows_linear (down_proj, residual) and kvc_rows_qkv
 * run in order, bit for bit.  The tail is skipped when w_o is NULL, the head when
 * w_qkv is NULL.  Layouts: x [M,H], att [M,Hq*D], act [M,I] (scratch), w_o [H,Hq*D],
 * w_gate_up [2I,H], w_down [H,I], w_qkv [(Hq+2Hkv)D,H], b_qkv [(Hq+2Hkv)D], q/k/v as
 * kvc_rows_qkv; fp16; M <= 32; H a multiple of 32 (<= 1024), I of 32, D of 32.
 * workspace (tail): kvc_rows_chain_workspace_size(H, I) bytes, 256-byte aligned,
 * ZERO-FILLED before first use and then used by kvc_rows_chain calls of one stream
 * only (the launches keep their barrier counters consistent from one to the next, not
 * zero: do not share it with the other kvc_rows_* calls).  The grid (at most one workgroup per CU) must be resident at once:
 * KVC_ERR_UNSUPPORTED when the device is too small or a shape falls outside the
 * kernel's.  A barrier wait that gives up (workgroups not all resident, e.g. another
 * stream's kernels holding CUs) ends the launch without finishing it and reports
 * through the device error word: the next kvc_rows_chain call with a tail, or
 * kvc_check_device_errors, returns KVC_ERR_STATE (and the call clears the counters).
 * Not graph-safe in the sense of the *_dev entry points (M is fixed at capture). */
typedef struct kvc_layer_chain {
    int M, H, Hq, Hkv, D, I;
    float eps, theta;
    void* x;
    const void *att, *w_o, *ln2, *w_gate_up;
    void* act;
    const void* w_down;
    void *q, *k, *v;
    const void *ln1, *w_qkv, *b_qkv;
    const int* pos;
} kvc_layer_chain;
size_t kvc_rows_chain_workspace_size(int H, int I);
int kvc_rows_chain(const kvc_layer_chain* chain, void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* ---- Qwen2-shaped decoder served with continuous batching (include/kvc/qwen_model.h;
 * the model track of the reference, qwen_serve.cu:60-210) ----
 * Random N(0, init_std) fp16 weights from `seed` (norm weights 1, lm_head tied to the
 * embedding); greedy decoding; requests admitted FIFO up to max_batch running. */
typedef struct kvc_qwen_config {
    int layers, hidden, n_heads, n_kv_heads, head_dim, inter, vocab;
    float eps, theta, init_std;
    int block_size, num_blocks, max_batch, max_rows;  /* max_rows: longest prompt */
    uint64_t seed;                                      /* 0: default */
    int step_path;  /* 0: fused decode-step kernels when a step has <= 32 rows; 1: one kernel per op */
    int graph;      /* 1: fused steps replay one captured HIP graph (0: eager launches) */
    int prefill_rows;  /* prompt rows stacked into one prefill forward (0: 4096) */
    int chain;      /* 1: eager fused steps run the linear layers between two attention launches as one
                       launch (kvc_rows_chain) where the device and shapes allow; 0: one launch each */
} kvc_qwen_config;
typedef struct kvc_qwen_stats {
    int steps, finished;
    long long tokens, prompt_tokens;
    double wall_us, prefill_us, decode_us;   /* host clock around the whole run / prefills / decode steps */
    long long graph_steps;                   /* decode steps that replayed the captured graph */
    long long graph_captures;                /* step graphs captured (again after a workspace growth) */
    long long chain_launches;                /* layer-chain launches (kvc_rows_chain) of the decode steps */
} kvc_qwen_stats;
typedef struct kvc_qwen kvc_qwen;
int  kvc_qwen_create(const kvc_qwen_config* cfg, kvc_qwen** out);
void kvc_qwen_destroy(kvc_qwen* h);
/* device address and size of a weight: "embed", "norm", or per layer "ln1", "wq", "bq",
 * "wk", "bk", "wv", "bv", "wo", "ln2", "wg", "wu", "wd" ([out, in] row-major fp16) */
int  kvc_qwen_tensor(kvc_qwen* h, const char* name, int layer, void** ptr, size_t* bytes);
/* requests i: prompt tokens [prompt_off[i], prompt_off[i+1]), gen_len[i] >= 1 tokens
 * generated (the first from the prompt's last position); out_tokens gets them in
 * request order (sum of gen_len ints). */
int  kvc_qwen_serve(kvc_qwen* h, int n_req, const int* prompt_off, const int* prompt_tokens, const int* gen_len,
                    int* out_tokens, kvc_qwen_stats* stats);
/* weights in the reference's dump format (QwenWeights::load, qwen_loader.h:21-76; written by
 * tools/dump_weights.py:29-66): <dir>/manifest.tsv ("name\toffset\tnbytes\tshape_csv"
 * per line, Hugging Face names) over <dir>/weights.bin (fp16, [out, in] row-major).
 * Load: every tensor of the configured shape must be present (others are ignored);
 * lm_head.weight, if it differs from the embedding, is used untied.  Save: writes all
 * tensors, lm_head.weight included. */
int  kvc_qwen_load_weights(kvc_qwen* h, const char* dir);
int  kvc_qwen_save_weights(kvc_qwen* h, const char* dir);
/* one prompt: its first generated token and the fp32 logits of its last position (vocab floats) */
int  kvc_qwen_prefill_logits(kvc_qwen* h, const int* tokens, int P, float* logits_host, int* token);

/* launch_flash_decode (kv_cache.h:32-34, flash_decode.cu:103-126): one sequence,
 * contiguous [H,S,D], num_splits clamped to [1, cur_len]; split j covers
 * [j*ceil(L/ns), ...) and the partials are merged by log-sum-exp.  Unlike the
 * reference it allocates nothing: partials go to `workspace`. */
int kvc_flash_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                     int cur_len, int H, int D, int S, float scale, int num_splits, int dtype,
                     void* workspace, size_t workspace_bytes, kvc_stream_t stream);
size_t kvc_flash_decode_workspace_size(int H, int D, int num_splits);

/* ---- block free-list (block_alloc.h:10-43), host only ------------------- */
typedef struct kvc_block_allocator kvc_block_allocator;
int  kvc_block_allocator_create(int total_blocks, kvc_block_allocator** out);
void kvc_block_allocator_destroy(kvc_block_allocator* a);
int  kvc_block_allocator_alloc(kvc_block_allocator* a);   /* block id, or -1 when empty */
void kvc_block_allocator_free(kvc_block_allocator* a, const int* blocks, int n);
void kvc_block_allocator_reset(kvc_block_allocator* a);
int  kvc_block_allocator_free_count(const kvc_block_allocator* a);
int  kvc_block_allocator_used_count(const kvc_block_allocator* a);
/* Permute the current free list with a seeded Fisher-Yates shuffle so later
 * allocations come out in a random physical order (fragmented pool workloads). */
void kvc_block_allocator_shuffle(kvc_block_allocator* a, uint64_t seed);
int  kvc_blocks_needed(int seq_len, int block);           /* block_alloc.h:41-43 */

/* ---- serving loop: Engine (engine.h) and static baseline (scheduler.h) --- */
typedef struct kvc_engine_config {
    int n_heads;       /* query heads (EngineConfig.n_heads, engine.h:25) */
    int n_kv_heads;    /* KV heads; 0 = n_heads (MHA, as the reference) */
    int head_dim;
    int block_size;
    int num_blocks;    /* pool blocks per layer slice */
    int max_batch;
    int n_layers;      /* KV layer slices [n_layers, num_blocks, Hkv, BLOCK, D]; 0 = 1 */
    int dtype;         /* KVC_F32 (reference) or KVC_F16 */
    int kv_write;      /* 0: reference step (attend over cur_len, grow after, engine.h:132-137);
                          1: per layer write K/V at cur_len then attend over cur_len+1
                             (qwen_serve.cu:130-160) */
    int clock_mode;    /* 0: clock advances by the measured GPU step time (engine.h:132-133);
                          1: virtual clock, step cost = c0 + c1*N + c2*sum(len) us */
    double virt_c0, virt_c1, virt_c2;
    int device;        /* 1: own device pools and launch kernels; 0: scheduling only (no GPU) */
    int split_tokens;  /* device-lengths decode: split size; 0 = automatic */
    int decode_path;   /* KVC_DECODE_PLANNED (0, default) or KVC_DECODE_DEVICE_LENGTHS */
    int prefill;       /* 1: admitted prompts run qk_write_kv + qk_paged_causal_attn per layer; the
                          GPU time advances the measured clock (the virtual clock ignores it) */
    uint64_t seed;     /* seed of the synthetic q/k/v fill */
    int graph;         /* 1: planned decode steps replay one captured HIP graph (counts in device memory) */
} kvc_engine_config;

typedef struct kvc_engine_stats {     /* EngineStats (engine.h:33-45) + p50 + digest */
    int iters;
    long long tokens;
    double gpu_us;          /* sum of step times (measured or virtual) */
    double wall_us;         /* scheduler clock at the end = makespan */
    long long slot_steps;
    long long useful_steps;
    int peak_blocks;
    int finished;
    double avg_latency_us;
    double p50_latency_us;
    double p99_latency_us;
    uint64_t step_digest;   /* FNV-1a 64 over every step's packed metadata */
    double host_wall_us;    /* real elapsed time of the whole run on the host clock */
    double prefill_us;      /* GPU time of prompt processing (part of gpu_us) */
} kvc_engine_stats;

typedef struct kvc_request { int id; double arrival_us; int prompt_len; int gen_len; } kvc_request;

typedef struct kvc_engine kvc_engine;
int  kvc_engine_create(const kvc_engine_config* cfg, kvc_engine** out);
void kvc_engine_destroy(kvc_engine* e);
int  kvc_engine_reset(kvc_engine* e);
/* Requests must be added in non-decreasing arrival order (engine.h:87). */
int  kvc_engine_add_request(kvc_engine* e, int prompt_len, int max_new_tokens, double arrival_us);
/* One iteration; *more = 0 once every request has finished.  Returns KVC_ERR_STATE if the
 * head of the queue can never be admitted (its worst case exceeds the pool). */
int  kvc_engine_step(kvc_engine* e, int* more);
int  kvc_engine_run(kvc_engine* e, kvc_engine_stats* out);
int  kvc_engine_stats_get(const kvc_engine* e, kvc_engine_stats* out);
/* No counterpart in the reference: what the last decode step ran, for checking it from
 * outside.  n = its batch; lens[n], tab_off[n+1] and table[] (table_cap ints at least)
 * are the packed metadata it uploaded (model_runner.h:61-69 order); wpos/slots (may be
 * NULL) each row's write position and pool slot (-1: none); dev[6] = the runner's
 * q [L][max_batch][Hq][D], new K and V [L][max_batch][Hkv][D] and out [max_batch][Hq][D]
 * (the last layer's) buffers and the K and V pools [L][num_blocks][Hkv][BLOCK][D]. */
int  kvc_engine_last_step(const kvc_engine* e, int* n, int* lens, int* tab_off, int* table, int table_cap,
                          int* wpos, int* slots, void** dev);
/* run_static (scheduler.h:33-89) over the engine's pool and runner. */
int  kvc_run_static(kvc_engine* e, const kvc_request* reqs, int n, int max_batch, kvc_engine_stats* out);

#ifdef __cplusplus
}
#endif
#endif /* KVC_ABI_H */
