/*
 * grm_hip_router.h -- C ABI of libgrm_hip_router.so, the MI355X (gfx950)
 * GRM graft route library.
 *
 * Part 1 keeps the reference sidecar ABI symbol-for-symbol, so the
 * reference's ctypes bindings load this library unchanged:
 *   MLA: scripts/grm_mla_cuda_probe.py:286-547 (C source), :575-626 (ctypes)
 *   GQA: scripts/grm_gqa_cuda_probe.py:297-606 (C source), :634-697 (ctypes)
 * Part 2 adds the entry points the reference has no counterpart for (node
 * ids and scores out, bf16/fp16/int8 storage, ragged CSR banks, device-side
 * append/evict); their comments say so.
 *
 * Conventions (both parts, as the reference, scripts/grm_mla_cuda_probe.py:60-66):
 *   return 0 on success, -1 on invalid arguments, 1000 + hipError_t on a HIP
 *   runtime error, -3 when a bank's capacity would be exceeded.
 *   grm_hip_last_error() returns a message for the calling thread's last
 *   failure.
 *   Top-k order: score descending, node id ascending; non-finite scores are
 *   never ranked; unfilled result slots hold UINT64_MAX (ids) / NaN (scores).
 *   topk must satisfy 1 <= topk <= 16 and topk <= live nodes.
 *   Every call is synchronous with respect to its outputs; calls on one bank
 *   must not overlap (one bank per thread, as the reference).
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct MlaDeviceArena MlaDeviceArena;
typedef struct GqaDeviceArena GqaDeviceArena;

/* Element types of banks and queries (extension). */
enum {
  GRM_DTYPE_F32 = 0,
  GRM_DTYPE_BF16 = 1,
  GRM_DTYPE_F16 = 2,
  GRM_DTYPE_I8 = 3
};

/* ======================================================= reference MLA ABI */

/* Replaces grm_mla_cuda_arena_create, scripts/grm_mla_cuda_probe.py:286-336.
 * rows_host [nodes][dim] fp32; node id of row i is i. */
int grm_mla_cuda_arena_create(const float* rows_host, int nodes, int dim,
                              MlaDeviceArena** out_arena);

/* Replaces grm_mla_cuda_arena_route, scripts/grm_mla_cuda_probe.py:437-464.
 * queries_host [query_count][dim] fp32; out_topk_host [query_count][topk]
 * row ids; elapsed_ms_host = device time of queries [warmup, query_count). */
int grm_mla_cuda_arena_route(MlaDeviceArena* arena, const float* queries_host,
                             int query_count, int dim, int warmup, int topk,
                             uint64_t* out_topk_host, float* elapsed_ms_host);

/* Replaces grm_mla_cuda_arena_route_device, scripts/grm_mla_cuda_probe.py:473-488.
 * d_queries is a device pointer to [query_count][dim] fp32. */
int grm_mla_cuda_arena_route_device(MlaDeviceArena* arena,
                                    const float* d_queries, int query_count,
                                    int dim, int warmup, int topk,
                                    uint64_t* out_topk_host,
                                    float* elapsed_ms_host);

/* Replaces grm_mla_cuda_upload_queries, scripts/grm_mla_cuda_probe.py:493-514. */
int grm_mla_cuda_upload_queries(const float* host_buf, size_t num_floats,
                                float** out_device_ptr);

/* Replaces grm_mla_cuda_free_device_ptr, scripts/grm_mla_cuda_probe.py:515-520. */
int grm_mla_cuda_free_device_ptr(float* device_ptr);

/* Replaces grm_mla_cuda_arena_destroy, scripts/grm_mla_cuda_probe.py:522-525. */
int grm_mla_cuda_arena_destroy(MlaDeviceArena* arena);

/* Replaces grm_mla_cublas_route (one-shot create/route/destroy),
 * scripts/grm_mla_cuda_probe.py:527-547.  No BLAS library is involved. */
int grm_mla_cublas_route(const float* rows_host, const float* queries_host,
                         int nodes, int dim, int query_count, int warmup,
                         int topk, uint64_t* out_topk_host,
                         float* elapsed_ms_host);

/* ======================================================= reference GQA ABI */

/* Replaces grm_gqa_cuda_arena_create, scripts/grm_gqa_cuda_probe.py:297-365.
 * keys_host [nodes][kv_heads][key_tokens][head_dim] fp32 (zero-padded dense
 * bank); node id of node i is i. */
int grm_gqa_cuda_arena_create(const float* keys_host, int nodes, int kv_heads,
                              int key_tokens, int head_dim,
                              GqaDeviceArena** out_arena);

/* Replaces grm_gqa_cuda_arena_route, scripts/grm_gqa_cuda_probe.py:484-514.
 * queries_host [query_count][query_heads][query_tokens][head_dim] fp32. */
int grm_gqa_cuda_arena_route(GqaDeviceArena* arena, const float* queries_host,
                             int query_count, int query_heads,
                             int query_tokens, int warmup, int topk,
                             uint64_t* out_topk_host, float* elapsed_ms_host);

/* Replaces grm_gqa_cuda_arena_route_device, scripts/grm_gqa_cuda_probe.py:525-536. */
int grm_gqa_cuda_arena_route_device(GqaDeviceArena* arena,
                                    const float* d_queries, int query_count,
                                    int query_heads, int query_tokens,
                                    int warmup, int topk,
                                    uint64_t* out_topk_host,
                                    float* elapsed_ms_host);

/* Replaces grm_gqa_cuda_upload_queries, scripts/grm_gqa_cuda_probe.py:547-567. */
int grm_gqa_cuda_upload_queries(const float* host_buf, size_t num_floats,
                                float** out_device_ptr);

/* Replaces grm_gqa_cuda_free_device_ptr, scripts/grm_gqa_cuda_probe.py:569-574. */
int grm_gqa_cuda_free_device_ptr(float* device_ptr);

/* Replaces grm_gqa_cuda_arena_destroy, scripts/grm_gqa_cuda_probe.py:576-579. */
int grm_gqa_cuda_arena_destroy(GqaDeviceArena* arena);

/* Replaces grm_gqa_cublas_route, scripts/grm_gqa_cuda_probe.py:581-606. */
int grm_gqa_cublas_route(const float* keys_host, const float* queries_host,
                         int nodes, int kv_heads, int key_tokens,
                         int query_count, int query_heads, int query_tokens,
                         int head_dim, int warmup, int topk,
                         uint64_t* out_topk_host, float* elapsed_ms_host);

/* ============================================= extensions (no counterpart) */

/* Message for the calling thread's most recent failure ("" if none).
 * No counterpart: the reference sidecar reports codes only. */
const char* grm_hip_last_error(void);

/* Library/device description: writes a short JSON object (device name,
 * compute units, library version) into out.  No counterpart. */
int grm_hip_runtime_info(char* out, size_t out_cap);

/* MLA node bank (no counterpart: the reference rebuilds and re-uploads the
 * whole bank on every mutation, core/graft_arena.py:1164-1198).
 * rows_host [nodes][dim] of row_dtype (GRM_DTYPE_F32 or GRM_DTYPE_BF16 as
 * uint16 bit patterns); node_ids [nodes] or NULL (0..nodes-1); capacity is
 * the slot count to reserve (>= nodes; 0 means nodes). */
int grm_mla_hip_bank_create(const void* rows_host, int row_dtype,
                            uint64_t nodes, int dim, const uint64_t* node_ids,
                            uint64_t capacity, MlaDeviceArena** out_arena);

/* MLA route returning node ids and scores (no counterpart: the reference
 * returns row ids only).  queries [query_count][dim] of query_dtype
 * (F32 or BF16 bits); queries_on_device selects a device pointer.
 * out_ids_host / out_scores_host are [query_count][topk]; scores may be NULL.
 * elapsed_ms_host may be NULL: no device time is taken then, and the call
 * sees its kernel's completion through per-block flags in host memory
 * rather than a stream event (the same results, sooner). */
int grm_mla_hip_route(MlaDeviceArena* arena, const void* queries,
                      int query_dtype, int queries_on_device, int query_count,
                      int dim, int warmup, int topk, uint64_t* out_ids_host,
                      float* out_scores_host, float* elapsed_ms_host);

/* Allocation-free variant of grm_mla_hip_route for callers that cannot
 * allocate device or host memory (tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the
 * reference.  Queries are device memory [query_count][dim] (F32 or BF16
 * bits); results go to device memory: d_out_ids [query_count][topk] and
 * d_out_scores (may be NULL), unfilled slots UINT64_MAX / NaN.  Every query
 * runs the single-query kernel (the batched matrix-core path is not used).
 * The per-block lists live in a fixed 256 KiB device array inside the
 * library (one per GPU, held until the process ends); a route whose grid
 * blocks x topk exceed its 16384 entries is refused with -1.  The call
 * allocates nothing and returns once the outputs are written.  Calls on
 * one GPU share that array, so they are serialised: a per-device lock is
 * held from the first launch until the bank's stream has drained.  The
 * work runs on the bank's own stream and the call synchronizes it, so it
 * cannot be recorded into a caller's HIP graph. */
int grm_mla_hip_route_noalloc(MlaDeviceArena* arena, const void* d_queries,
                              int query_dtype, int query_count, int dim,
                              int topk, uint64_t* d_out_ids,
                              float* d_out_scores);

/* Append `count` rows with node ids (no counterpart).  The upload and the
 * device-side placement run on the bank's side stream; the next route waits
 * for them.  out_epoch (may be NULL) receives the bank epoch after the call.
 * Appending an id that is already live returns -1. */
int grm_mla_hip_append(MlaDeviceArena* arena, const void* rows_host,
                       int row_dtype, uint64_t count, const uint64_t* node_ids,
                       uint64_t* out_epoch);

/* Evict live node ids (tombstone: the slot stops ranking at once and is
 * reused by later appends).  Unknown ids return -1 and evict nothing.
 * No counterpart. */
int grm_mla_hip_evict(MlaDeviceArena* arena, const uint64_t* node_ids,
                      uint64_t count, uint64_t* out_epoch);

/* Wait for pending side-stream mutations.  No counterpart. */
int grm_mla_hip_sync(MlaDeviceArena* arena);

/* Bank description: [live, capacity, slots in use, epoch, dim, dtype].
 * No counterpart. */
int grm_mla_hip_bank_info(MlaDeviceArena* arena, uint64_t* out6);

/* Route counters since create: [queries screened by the batched
 * matrix-core path, of those routed again on the single-query path (no
 * certificate), queries through the single-query kernel, screen passes].
 * No counterpart. */
int grm_mla_hip_route_stats(MlaDeviceArena* arena, uint64_t* out4);

/* Device time (ms, from events on the route stream) of the matrix-core
 * screen kernels in the timed segment of the last batched route; 0 when
 * the last route was not batched.  No counterpart. */
int grm_mla_hip_screen_ms(MlaDeviceArena* arena, float* ms);

/* Test entry, no counterpart and on no route path: runs the batched
 * route's matrix-core screen over every slot of a small bf16 bank
 * (capacity x 256 <= 2^26) for query_count queries (at most one screen
 * pass, <= 256) and writes each screened score s~ of (query q, slot s) to
 * out_values[q * high_water + s], the query's screen bound B to
 * out_bounds[q] (+inf where it is not established), and the slots' node
 * ids to out_slot_ids (optional; high_water entries).  The certificate of
 * the batched route rests on |s~ - law score| <= B for every pair.
 * Allocates its own buffers. */
int grm_mla_hip_probe_screen(MlaDeviceArena* arena, const void* queries_host,
                             int query_dtype, int query_count,
                             float* out_values_host, double* out_bounds_host,
                             uint64_t* out_slot_ids_host);

/* MLA route key from a device-resident latent block [tokens][dim] (row
 * stride row_stride elements, 0 = dim; latent_dtype F32, BF16 or F16): the
 * unit-norm token mean of core/kv_graft.py:131-142 (latent_centroid), written
 * as dim floats to d_out (normalize = 0 writes the plain mean).  Replaces
 * the forward pass's host round trip before route_topk_device
 * (core/grm_cuda_router.py:491-539).  Waits for completion.  No counterpart. */
int grm_mla_hip_latent_query(MlaDeviceArena* arena, const void* d_latent, int latent_dtype,
                             uint64_t tokens, uint64_t row_stride, int normalize,
                             float* d_out);

/* ---- Store route on the device (cpp/grm_runtime_c.h:176-181, 381-424) ----
 * Per-node route filter bits, as route_filter_bits (cpp/grm_runtime.cpp:
 * 2793-2838: kind at bit 0, scope 16, durability 32, mutability 48, one
 * bit per known value).  A slot reused by a later append starts at 0.
 * Ids must be live.  Counterpart of the filter bits kept by
 * grm_store_set_route_metadata. */
int grm_mla_hip_set_filter_bits(MlaDeviceArena* arena, const uint64_t* node_ids,
                                const uint64_t* bits, uint64_t count);

/* One query routed over the nodes that pass the route filters
 * (cpp/grm_runtime.cpp:3074-3104 with known values): for each category c
 * set in filter_categories (bits 0..3), a node's bits must meet the 16-bit
 * mask at shift 16c of filter_mask.  Ids and scores as grm_mla_hip_route.
 * The lexical bonus is added above this call (graftrepository_amd.
 * store_route), giving grm_store_route_filtered's law. */
int grm_mla_hip_route_filtered(MlaDeviceArena* arena, const void* query, int query_dtype,
                               int query_on_device, int topk, uint64_t filter_mask,
                               uint32_t filter_categories, uint64_t* out_ids_host,
                               float* out_scores_host, float* elapsed_ms_host);

/* Exact law scores (cpp/grm_runtime.cpp:3518-3545) of listed live nodes for
 * one host query (F32 or BF16): float, NaN where not finite.  No
 * counterpart (the store scores every entry on the CPU). */
int grm_mla_hip_score_nodes(MlaDeviceArena* arena, const void* query_host, int query_dtype,
                            const uint64_t* node_ids, uint64_t count, float* out_scores_host);

/* Form that key on the bank's route stream and route it (one query) in the
 * same call: ids and scores as grm_mla_hip_route.  No counterpart. */
int grm_mla_hip_route_latent(MlaDeviceArena* arena, const void* d_latent, int latent_dtype,
                             uint64_t tokens, uint64_t row_stride, int topk,
                             uint64_t* out_ids_host, float* out_scores_host,
                             float* elapsed_ms_host);

/* Ragged GQA node bank over CSR token offsets (no counterpart: the reference
 * zero-pads every node to the longest, core/graft_arena.py:2979-3042).
 * keys_host: node i's block [kv_heads][L_i][head_dim] starts at value
 * offset tok_offsets[i] * kv_heads * head_dim, L_i = tok_offsets[i+1] -
 * tok_offsets[i]; key_dtype F32, BF16, F16 (bit patterns) or I8.
 * For I8, scales_host holds one scale per (kv head, token, group of
 * group_size values) in the same node-major order, scale_dtype F32 or F16;
 * values dequantise as fp16(code * scale) (core/graft_quant.py:136-144).
 * capacity_nodes / capacity_tokens reserve room for appends (0 = exact). */
int grm_gqa_hip_bank_create(const void* keys_host, int key_dtype,
                            const void* scales_host, int scale_dtype,
                            int group_size, const uint64_t* tok_offsets,
                            uint64_t nodes, int kv_heads, int head_dim,
                            const uint64_t* node_ids, uint64_t capacity_nodes,
                            uint64_t capacity_tokens,
                            GqaDeviceArena** out_arena);

/* GQA route returning node ids and scores (no counterpart).  queries
 * [query_count][query_heads][query_tokens][head_dim] of query_dtype
 * (F32 or BF16 bits).  Stacked routing layers are expressed by folding the
 * layer axis into the head axes of both bank and query.  elapsed_ms_host
 * may be NULL: no device time is taken then, and screen-and-refine routes
 * see completion through the finalize blocks' flags in host memory rather
 * than a stream event (the same results, sooner). */
int grm_gqa_hip_route(GqaDeviceArena* arena, const void* queries,
                      int query_dtype, int queries_on_device, int query_count,
                      int query_heads, int query_tokens, int warmup, int topk,
                      uint64_t* out_ids_host, float* out_scores_host,
                      float* elapsed_ms_host);

/* Append `count` nodes; node j has tok_counts[j] tokens and its blocks are
 * consecutive in keys_host (and scales_host for I8).  Side-stream upload as
 * grm_mla_hip_append.  No counterpart. */
int grm_gqa_hip_append(GqaDeviceArena* arena, const void* keys_host,
                       const void* scales_host, const uint64_t* tok_counts,
                       uint64_t count, const uint64_t* node_ids,
                       uint64_t* out_epoch);

/* Evict live node ids (tombstone; token space is reclaimed by
 * grm_gqa_hip_compact).  No counterpart. */
int grm_gqa_hip_evict(GqaDeviceArena* arena, const uint64_t* node_ids,
                      uint64_t count, uint64_t* out_epoch);

/* Compact the token arena on the device (drops evicted nodes' tokens).
 * No counterpart. */
int grm_gqa_hip_compact(GqaDeviceArena* arena);

/* Wait for pending side-stream mutations.  No counterpart. */
int grm_gqa_hip_sync(GqaDeviceArena* arena);

/* Bank description: [live nodes, node capacity, tokens in use, token
 * capacity, epoch, kv_heads, head_dim, key dtype].  No counterpart. */
int grm_gqa_hip_bank_info(GqaDeviceArena* arena, uint64_t* out8);

/* Route counters since create: [route calls, query passes routed by
 * screen and refine, passes routed by bound and verify, queries routed by
 * the exact path].  An fp32 bank's passes are screened through its fp16
 * key copy.  No counterpart. */
int grm_gqa_hip_route_stats(GqaDeviceArena* arena, uint64_t* out4);

/* Test entry, no counterpart and on no route path: the screen of the
 * bound-and-verify path for one query [query_heads][query_tokens][head_dim]
 * (R * query_tokens <= 64 columns per kv head, R = heads / kv_heads) over
 * every node with key tokens.  Writes, for every slot of the node
 * capacity, the largest screened value per (slot, kv head g, column
 * cg = r * query_tokens + t) in the screen's scaled units to
 * out_maxima[(slot * kv + g) * R * query_tokens + cg]; the bound
 * parameters {coef, eabs, scale, kcap} of each column to
 * out_colinfo[(g * R * query_tokens + cg) * 4 ..]; the key norm bound K of
 * each slot to out_knorm; the slots' node ids to out_slot_ids (optional).
 * For a node with K < kcap, |maximum - scale * max_t |q . k_t|| <=
 * coef * K + eabs (the screen bound both screen paths rest on).
 * Allocates its own query buffer. */
int grm_gqa_hip_probe_screen(GqaDeviceArena* arena, const void* query_host,
                             int query_dtype, int query_heads, int query_tokens,
                             float* out_maxima_host, float* out_colinfo_host,
                             double* out_knorm_host, uint64_t* out_slot_ids_host);

/* ---- GQA store route on the device (cpp/grm_runtime.cpp:6898-6961) ----
 * Per-node route filter bits, as grm_mla_hip_set_filter_bits (a slot taken
 * by a later append starts at 0).  Ids must be live. */
int grm_gqa_hip_set_filter_bits(GqaDeviceArena* arena, const uint64_t* node_ids,
                                const uint64_t* bits, uint64_t count);

/* One query [query_heads][query_tokens][head_dim] routed over the nodes that
 * pass the route filters (semantics of grm_mla_hip_route_filtered): node
 * ids and raw law scores (cpp/grm_runtime.cpp:2980-3029), (score desc, id
 * asc).  route_gqa_raw's filtered ranking before any lexical bonus. */
int grm_gqa_hip_route_filtered(GqaDeviceArena* arena, const void* query, int query_dtype,
                               int query_on_device, int query_heads, int query_tokens, int topk,
                               uint64_t filter_mask, uint32_t filter_categories,
                               uint64_t* out_ids_host, float* out_scores_host,
                               float* elapsed_ms_host);

/* Exact raw law scores of listed live nodes for one host query (F32 or
 * BF16): float, NaN where not finite.  No counterpart (the store scores
 * every entry on the CPU). */
int grm_gqa_hip_score_nodes(GqaDeviceArena* arena, const void* query_host, int query_dtype,
                            int query_heads, int query_tokens, const uint64_t* node_ids,
                            uint64_t count, float* out_scores_host);

/* ---- The store's route calls over a device bank ---------------------------
 * A device store holds route entries (one route key, lexical keys, route
 * metadata per node) in an MLA or a GQA bank of this library and answers
 * the reference store's route calls with their names, argument lists and
 * output conventions (cpp/grm_runtime_c.h:176-181, 381-436, 499): 0 on
 * success, nonzero with grm_store_last_error() on failure; out_count
 * receives min(results, out_cap).  Nodes need no grm_store_add_node here:
 * the CPU store keeps nodes and payloads, this store their route entries.
 * An entry with several keys (set_route_multi / set_route_list) scores the
 * maximum of its keys' finite law scores (cpp/grm_runtime.cpp:3518-3545,
 * 3031-3051); its keys are scored exactly on every route.
 * Limits: topk <= 16; MLA keys of the store's dim, GQA keys of whole
 * [kv_heads][L][head_dim] blocks; calls on one handle are serialized. */
typedef struct grm_store_handle grm_store_handle;

/* Create an MLA store of `dim`-value fp32 route keys with room for
 * `capacity` entries (row_dtype GRM_DTYPE_F32), or a GQA store with room
 * for capacity_nodes entries and capacity_tokens key tokens.  Replace the
 * reference's grm_store_create_mla / _gqa (cpp/grm_runtime_c.h:70-106) for
 * the route path. */
int grm_hip_store_create_mla(int dim, uint64_t capacity, int row_dtype,
                             grm_store_handle** out_handle);
int grm_hip_store_create_gqa(int kv_heads, int head_dim, uint64_t capacity_nodes,
                             uint64_t capacity_tokens, grm_store_handle** out_handle);
/* cpp/grm_runtime_c.h:108 (grm_store_destroy) */
void grm_hip_store_destroy(grm_store_handle* handle);

/* cpp/grm_runtime_c.h:381-385 */
int grm_store_set_route(grm_store_handle* handle, uint64_t node_id, const float* route_key,
                        uint64_t route_len, const char* lexical_keys);
/* cpp/grm_runtime_c.h:386-391 */
int grm_store_set_route_multi(grm_store_handle* handle, uint64_t node_id,
                              const float* route_keys, uint64_t key_count, uint64_t route_len,
                              const char* lexical_keys);
/* cpp/grm_runtime_c.h:392-399 */
int grm_store_set_route_list(grm_store_handle* handle, uint64_t node_id,
                             const float* route_values, uint64_t value_count,
                             const uint64_t* route_offsets, uint64_t key_count,
                             const char* lexical_keys);
/* cpp/grm_runtime_c.h:400-401 */
int grm_store_clear_route(grm_store_handle* handle, uint64_t node_id);
/* cpp/grm_runtime_c.h:176-181 */
int grm_store_set_route_metadata(grm_store_handle* handle, uint64_t node_id, const char* kind,
                                 const char* scope, const char* durability,
                                 const char* mutability);
/* cpp/grm_runtime_c.h:402-409 */
int grm_store_route(grm_store_handle* handle, const float* query, uint64_t query_len,
                    const char* lexical_keys, uint64_t topk, uint64_t* out_node_ids,
                    uint64_t out_cap, uint64_t* out_count);
/* cpp/grm_runtime_c.h:410-421 */
int grm_store_route_filtered(grm_store_handle* handle, const float* query, uint64_t query_len,
                             const char* lexical_keys, const char* kind_filters,
                             const char* scope_filters, const char* durability_filters,
                             const char* mutability_filters, uint64_t topk,
                             uint64_t* out_node_ids, uint64_t out_cap, uint64_t* out_count);
/* cpp/grm_runtime_c.h:422-435 */
int grm_store_route_gqa(grm_store_handle* handle, const float* query, uint64_t query_heads,
                        uint64_t query_tokens, uint64_t head_dim, const char* lexical_keys,
                        const char* kind_filters, const char* scope_filters,
                        const char* durability_filters, const char* mutability_filters,
                        uint64_t topk, uint64_t* out_node_ids, uint64_t out_cap,
                        uint64_t* out_count);
/* cpp/grm_runtime_c.h:499 (the calling thread's last message) */
const char* grm_store_last_error(grm_store_handle* handle);

/* Many new entries at once (no counterpart: the reference sets routes one
 * node at a time): keys back to back, key_lens[i] values for node i;
 * lexical_keys[i] '\n'-joined (NULL array: none); metadata[4*i + c] the
 * kind, scope, durability, mutability of node i (NULL array or empty
 * values: the entry defaults). */
int grm_hip_store_set_routes(grm_store_handle* handle, uint64_t count, const uint64_t* node_ids,
                             const float* keys, const uint64_t* key_lens,
                             const char* const* lexical_keys, const char* const* metadata);

/* The store route with its fp32 route scores (no counterpart: the reference
 * returns ids only).  MLA stores ignore query_heads / query_tokens (the
 * query holds the store's dim values); GQA stores take
 * [query_heads][query_tokens][head_dim]. */
int grm_hip_store_route_scored(grm_store_handle* handle, const float* query,
                               uint64_t query_heads, uint64_t query_tokens,
                               const char* lexical_keys, const char* kind_filters,
                               const char* scope_filters, const char* durability_filters,
                               const char* mutability_filters, uint64_t topk,
                               uint64_t* out_node_ids, float* out_scores, uint64_t out_cap,
                               uint64_t* out_count);

/* [dialect (0 MLA, 1 GQA), entries, dim or kv_heads, 0 or head_dim].
 * No counterpart. */
int grm_hip_store_info(grm_store_handle* handle, uint64_t* out4);

/* ---- Packed graft payloads (core/graft_quant.py:177-268) ----------------
 * A packed tensor is int8 codes (values in row-major order, grouped along
 * the last axis) and one fp32 scale per group of group_size values.  It
 * unpacks as fp16(fp32(code) * scale) (core/graft_quant.py:136-144; any
 * storage depth <= 8).  The reference dequantises on the host and uploads
 * fp16 (unpack_node, core/graft_arena.py:3479-3492); these entry points
 * take the packed form to the device and write the fp16 bit patterns there.
 * n_values must be a multiple of group_size.  Both wait for completion;
 * elapsed_ms (may be NULL) receives the device time. */

/* Device codes and scales to device fp16.  No counterpart (the reference
 * has no device unpack). */
int grm_hip_payload_dequant(const void* d_codes, const void* d_scales, uint64_t n_values,
                            uint32_t group_size, void* d_out_f16, float* elapsed_ms);

/* Host codes and scales uploaded in chunks and unpacked to device fp16.
 * Replaces the host dequant + fp16 upload of unpack_node
 * (core/graft_arena.py:3479-3492). */
int grm_hip_payload_upload(const void* h_codes, const void* h_scales, uint64_t n_values,
                           uint32_t group_size, void* d_out_f16, float* elapsed_ms);

/* Device memory for payload outputs (no counterpart; the reference's
 * equivalents are the sidecars' upload_queries / free_device_ptr). */
int grm_hip_device_alloc(uint64_t bytes, void** out_ptr);
int grm_hip_device_free(void* ptr);
int grm_hip_copy_to_host(void* host, const void* device, uint64_t bytes);
int grm_hip_copy_to_device(void* device, const void* host, uint64_t bytes);

/* ---- Synthetic workload keys (host only) --------------------------------
 * Rows [row0, row0 + rows) of the synthetic INT8 key stream: each row's dim
 * values are normal quantiles (normal_table[65536], the caller's table of
 * Phi^-1((u + 0.5) / 65536)) indexed by 16-bit words of a splitmix64
 * counter stream keyed by `key`, quantised by the packed graft format's
 * law (core/graft_quant.py:93-131) with one group per row and the scale
 * stored as fp16.  Writes codes [rows][dim] int8 and scales_f16 [rows]
 * (fp16 bits) on `threads` host threads.  No counterpart in the reference;
 * it builds benchmark and test banks and is on no route path.  dim must be
 * a multiple of 4. */
int grm_hip_synth_int8_rows(uint64_t key, uint64_t row0, uint64_t rows, int dim,
                            const float* normal_table, int threads, int8_t* codes,
                            uint16_t* scales_f16);

#ifdef __cplusplus
}
#endif
