/*
 * kunserve_hip.h — C ABI of the MI355X (gfx950) paged-KV attention path.
 *
 * This library replaces the GPU side of the KV-cache operators that the
 * KunServe host layer reaches through libflash_pybinding.so:
 *
 *   torch.ops.swapping_ops.swap            kunserve/worker.py:673-681
 *   LlamaOp.local_copy_blocks              kunserve/worker.py:818-823
 *   LlamaOp.kv_exchange (pack / scatter)   kunserve/worker.py:514-532,
 *                                          kunserve/flash_backend.py:857-1022
 *   LlamaOp.pforward, attention stage      kunserve/worker.py:298-312
 *       (K/V append into pages, paged decode attention for q_len == 1 rows,
 *        chunked-prefill causal attention for prefill rows)
 *
 * Conventions
 *   - Every function returns 0 on success and a negative KUNSERVE_E* code on
 *     failure; kunserve_last_error() returns a message for the calling thread.
 *   - Pointers named *_dev are device pointers, *_host are host pointers.
 *   - All device work is enqueued on the given stream; no function
 *     synchronises the device or the stream, and no function allocates
 *     device memory: scratch space is passed in by the caller. The one
 *     exception is the kunserve_pmm_* group, whose purpose is to create and
 *     remap device memory; it runs while the engine is paused.
 *   - KV data is fp16 or bf16 (kunserve_kv_pool.dtype; q, outputs and new
 *     K/V share it). Element (page, layer, kv_head, slot, dim) of the K (or
 *     V) pool lives at
 *        page*page_stride + layer*layer_stride + kv_head*head_stride
 *        + slot*token_stride + dim                      (in elements)
 *     The default strides are those of the [num_pages, num_layers,
 *     num_kv_heads, page_size, head_dim] pool of kunserve/worker.py:168-176.
 *   - Page tables are CSR: pages of sequence b are
 *     indices[indptr[b] .. indptr[b+1]), token t of sequence b lives in page
 *     indices[indptr[b] + t / page_size] at slot t % page_size
 *     (kunserve/block_manager.py:786-795).
 */
#ifndef KUNSERVE_HIP_H
#define KUNSERVE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kunserve_stream_t; /* == hipStream_t */

enum {
  KUNSERVE_OK = 0,
  KUNSERVE_EINVAL = -1,     /* bad argument (shape, stride, alignment, NULL) */
  KUNSERVE_ERANGE = -2,     /* page / block id outside the pool              */
  KUNSERVE_ENOSPC = -3,     /* caller buffer (plan, workspace) too small     */
  KUNSERVE_EUNSUPPORTED = -4, /* head_dim / page_size / GQA not compiled   */
  KUNSERVE_EHIP = -5        /* a HIP runtime call failed                     */
};

/* Element types of pools and activations. */
enum {
  KUNSERVE_DTYPE_F16 = 0,
  KUNSERVE_DTYPE_BF16 = 1
};

/* Paged KV pool (separate K and V pools with identical strides). */
typedef struct {
  void* k;                 /* device, 16-bit elements of type dtype */
  void* v;
  int64_t num_pages;       /* page ids must lie in [0, num_pages)            */
  int64_t page_stride;     /* elements between consecutive pages             */
  int64_t layer_stride;
  int64_t head_stride;
  int64_t token_stride;    /* elements between consecutive slots of a page   */
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t page_size;       /* tokens per page; power of two, >= 4            */
  int32_t head_dim;        /* 64, 128 or 256                                 */
  int32_t dtype;           /* KUNSERVE_DTYPE_*: pool, q, out, new K/V alike   */
} kunserve_kv_pool;

/* Per-step page table in CSR form, device resident. */
typedef struct {
  const int32_t* indptr_dev;   /* [num_seqs + 1]                             */
  const int32_t* indices_dev;  /* [indptr[num_seqs]] page ids                */
  const int32_t* kv_len_dev;   /* [num_seqs] tokens in the cache after append */
  int32_t num_seqs;
} kunserve_page_table;

/* Strided activation tensor [num_tokens, num_heads, head_dim] (head_dim
 * contiguous), of the pool's dtype. */
typedef struct {
  void* data;              /* device */
  int64_t token_stride;    /* elements */
  int64_t head_stride;     /* elements */
} kunserve_tensor3;

/* ---------------------------------------------------------------- misc */

/* Library ABI version (major*100 + minor): 300. Major 2 gave
 * kunserve_prefill_plan_bound and kunserve_prefill_plan a head_dim argument
 * and kunserve_prefill_plan_info its head_dim field; major 3 gave
 * kunserve_paged_decode(_noalloc) the q_token_dev argument and
 * kunserve_paged_prefill the q_start_dev argument (mixed steps in place). */
int32_t kunserve_version(void);

/* Message of the last error raised on the calling thread ("" if none). */
const char* kunserve_last_error(void);

/* ------------------------------------------------------- block copy (A8) */

/* LlamaOp.local_copy_blocks (kunserve/worker.py:818-823): for each i,
 * block dst_ids[i] := block src_ids[i] for K and V, all layers, same device.
 * Ids are device int32 arrays of length n. A block is num_layers slabs of
 * num_kv_heads*page_size*head_dim elements. Source and destination sets
 * must not overlap (the kernel copies all pairs concurrently). */
int kunserve_copy_blocks(const kunserve_kv_pool* pool,
                         const int32_t* src_ids_dev, const int32_t* dst_ids_dev,
                         int64_t n, kunserve_stream_t stream);

/* kv_exchange phase 1 "pack" (kunserve/flash_backend.py:930-985): gather
 * layers [layer_begin, layer_end) of pages page_ids[0..n) into a contiguous
 * scratch buffer laid out [layer_end-layer_begin][n][2 (K,V)][num_kv_heads]
 * [page_size][head_dim] (16-bit elements, densely packed). */
int kunserve_kv_pack(const kunserve_kv_pool* pool, int32_t layer_begin,
                     int32_t layer_end, const int32_t* page_ids_dev, int64_t n,
                     void* scratch_dev, int64_t scratch_bytes,
                     kunserve_stream_t stream);

/* kv_exchange phase 3 "scatter": inverse of kunserve_kv_pack — write the
 * scratch layout into pages page_ids[0..n) (fused page ids on the receiver,
 * kunserve/block_manager.py:755-763). */
int kunserve_kv_scatter(const kunserve_kv_pool* pool, int32_t layer_begin,
                        int32_t layer_end, const int32_t* page_ids_dev,
                        int64_t n, const void* scratch_dev,
                        int64_t scratch_bytes, kunserve_stream_t stream);

/* Bytes of scratch that kunserve_kv_pack / kunserve_kv_scatter need. */
int64_t kunserve_kv_pack_bytes(const kunserve_kv_pool* pool, int32_t num_layers,
                               int64_t n);

/* Bandwidth calibration (no reference counterpart): streams `bytes` (a
 * multiple of 256 KiB) with the launch shape of the block copy. mode 0
 * reads src_dev only (dst_dev must hold 16 bytes), mode 1 writes dst_dev
 * only, mode 2 copies src_dev to dst_dev. The benchmark times these to
 * give the block copy's ceiling on the part it runs on. */
int kunserve_hbm_probe(int32_t mode, const void* src_dev, void* dst_dev,
                       int64_t bytes, kunserve_stream_t stream);

/* Access-pattern calibration (no reference counterpart): reads a decode
 * launch's K/V slabs (slab_bytes each: one page's tokens of one head, a
 * multiple of 1 KiB up to 16 KiB) in the partition kernel's workgroup
 * shape and dispatch order (num_items, a multiple of 8, are the plan's
 * work records: 8 XCD lanes interleaved, an item's heads on one XCD), with
 * no page-table lookups and no arithmetic. The workgroup of item i and
 * head h reads counts_dev[i] slabs at byte offsets
 * slab_offsets_dev[i * max_slabs + j] + h * head_stride_bytes from k_dev and
 * v_dev, and writes the XOR of every 32-bit word it read to sink_dev[i *
 * num_heads + h]. max_slabs is at most 1026 (the decode's longest
 * partition in pages); counts above max_slabs are read as max_slabs; the
 * offsets are device data the library cannot check, so the caller keeps
 * every slab inside both pools. The benchmark times it beside the decode
 * launch. */
int kunserve_decode_slab_probe(const void* k_dev, const void* v_dev,
                               const int64_t* slab_offsets_dev,
                               const int32_t* counts_dev, int32_t num_items,
                               int32_t max_slabs, int64_t head_stride_bytes,
                               int32_t num_heads, int32_t slab_bytes,
                               uint32_t* sink_dev, kunserve_stream_t stream);

/* ------------------------------------------------------------ swap (A7) */

/* torch.ops.swapping_ops.swap (kunserve/worker.py:646-650,673-681):
 * for each i, copy whole block src_ids[i] -> dst_ids[i] for K and V.
 * is_swap_in != 0: host (pinned) pool -> device pool; else device -> host.
 * Ids are host arrays. Block b of a pool is the contiguous byte range
 * [b*block_bytes, (b+1)*block_bytes). Pinned host pools (hipHostMalloc)
 * are read or written in place by one copy kernel per pool; the ids are
 * staged in a pinned slot the library keeps per device (reused once the
 * copies that read it have completed, a host wait only when 64 swaps are in
 * flight). Host memory the device cannot map falls back to one DMA copy per
 * run of consecutive ids. Enqueued on `stream`; does not synchronise. */
int kunserve_swap_blocks(const int64_t* src_ids_host,
                         const int64_t* dst_ids_host, int64_t n,
                         int32_t is_swap_in, void* k_cache_dev,
                         void* v_cache_dev, int64_t num_gpu_blocks,
                         void* k_swap_host, void* v_swap_host,
                         int64_t num_cpu_blocks, int64_t block_bytes,
                         kunserve_stream_t stream);

/* --------------------------------------------------- K/V append (A5 i) */

/* Append new tokens' K and V into the pool for one layer. Row b owns new
 * tokens [q_indptr[b], q_indptr[b+1]) of k_new / v_new ([num_tokens,
 * num_kv_heads, head_dim]); token i of row b goes to position
 * kv_len[b] - q_len[b] + i, i.e. page indices[indptr[b] + pos/page_size],
 * slot pos % page_size (kunserve/request.py:447-462). */
int kunserve_append_kv(const kunserve_kv_pool* pool, int32_t layer,
                       const kunserve_page_table* table,
                       const int32_t* q_indptr_dev, int32_t num_tokens,
                       const kunserve_tensor3* k_new,
                       const kunserve_tensor3* v_new,
                       kunserve_stream_t stream);

/* Fused attention prologue of a step: rotary position embedding of q (in
 * place, all num_qo_heads heads) and of k_new, then the append of the
 * rotated k and of v_new into the pages, as kunserve_append_kv. Token i of
 * row b sits at position kv_len[b] - q_len[b] + i (kunserve/request.py:
 * 447-462). inv_freq_dev holds head_dim / 2 fp32 frequencies (Llama:
 * theta^(-2j / head_dim)); the angle of pair j is the fp32 product
 * position * inv_freq[j]. Pairs are (j, j + head_dim / 2) ("rotate half"),
 * or (2j, 2j + 1) when interleave is non-zero. fp32 rotation, one rounding.
 * No reference counterpart: the rotation sits inside the native LlamaOp,
 * whose source the reference does not ship; this is the prologue that
 * LlamaOp.pforward runs before attention (kunserve/worker.py:298-312). */
int kunserve_rope_append_kv(const kunserve_kv_pool* pool, int32_t layer,
                            const kunserve_page_table* table,
                            const int32_t* q_indptr_dev, int32_t num_tokens,
                            kunserve_tensor3* q, int32_t num_qo_heads,
                            const kunserve_tensor3* k_new,
                            const kunserve_tensor3* v_new,
                            const float* inv_freq_dev, int32_t interleave,
                            kunserve_stream_t stream);

/* ---------------------------------------------- decode attention (A4) */

typedef struct {
  int32_t num_work;      /* work records: 8 XCD lanes of partitions,
                            interleaved, padded with seq -1 records      */
  int32_t num_merge;     /* sequences split over more than one partition  */
  int32_t num_slots;     /* partial-result slots used                     */
  int32_t part_tokens;   /* partition length in tokens                    */
  int32_t group_size;    /* q heads handled per workgroup                 */
  int32_t plan_ints;     /* int32 entries of the plan buffer in use       */
} kunserve_decode_plan_info;

/* Upper bound of the plan buffer length (int32 entries) for these lengths. */
int64_t kunserve_decode_plan_bound(const int32_t* kv_len_host,
                                   int32_t num_seqs);

/* Host-side plan, shared by every layer of one step (decode rows only).
 * Splits each sequence into partitions of part_tokens (0 = choose from
 * num_cus: the longest power of two in [256, 4096] whose longest work item
 * is at most 3/4 of one CU's share of the launch and that gives every CU
 * at least 4 workgroups, or whole rows for a short launch whose rows are
 * at most two minimum partitions), orders the work, and writes it to
 * plan_host (int32, upload it to the device as-is). */
int kunserve_decode_plan(const int32_t* kv_len_host, int32_t num_seqs,
                         int32_t num_qo_heads, int32_t num_kv_heads,
                         int32_t num_cus, int32_t part_tokens,
                         int32_t* plan_host, int64_t plan_capacity,
                         kunserve_decode_plan_info* info);

/* Workspace bytes needed by kunserve_paged_decode for this plan. */
int64_t kunserve_decode_workspace_bytes(const kunserve_decode_plan_info* info,
                                        int32_t num_qo_heads,
                                        int32_t head_dim);

/* o[t, h, :] = softmax(q[t, h, :] . K[b, g(h)]^T * sm_scale) . V[b, g(h)]
 * over the kv_len[b] tokens of sequence b in layer `layer`, with
 * g(h) = h / (num_qo_heads / num_kv_heads) and t = q_token[b], or t = b
 * when q_token_dev is NULL. q and out are [num_tokens, num_qo_heads,
 * head_dim] of the pool dtype (fp16 or bf16); fp32 accumulation. q_token
 * (device int32 [num_seqs]) lets the decode rows of a mixed step
 * (kunserve/flash_backend.py:1870-1950, rows of request.py:654-670) read q
 * and write out in place, among the step's prefill tokens. */
int kunserve_paged_decode(const kunserve_kv_pool* pool, int32_t layer,
                          const kunserve_page_table* table,
                          const int32_t* q_token_dev,
                          const kunserve_tensor3* q, kunserve_tensor3* out,
                          int32_t num_qo_heads, float sm_scale,
                          const int32_t* plan_dev,
                          const kunserve_decode_plan_info* info,
                          void* workspace_dev, int64_t workspace_bytes,
                          kunserve_stream_t stream);

/* kunserve_paged_decode without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The split partials live in a static device array of
 * kunserve_paged_decode_noalloc_max_bytes() (32 MiB) that each device the
 * library runs on holds until the process ends; plans whose
 * kunserve_decode_workspace_bytes exceed it fail with KUNSERVE_ENOSPC. The
 * call allocates nothing. Every call on one device shares that array:
 * calls that overlap on one device (concurrent streams) race, so serialise
 * them. Results equal kunserve_paged_decode's bit for bit. */
int64_t kunserve_paged_decode_noalloc_max_bytes(void);
int kunserve_paged_decode_noalloc(const kunserve_kv_pool* pool, int32_t layer,
                                  const kunserve_page_table* table,
                                  const int32_t* q_token_dev,
                                  const kunserve_tensor3* q, kunserve_tensor3* out,
                                  int32_t num_qo_heads, float sm_scale,
                                  const int32_t* plan_dev,
                                  const kunserve_decode_plan_info* info,
                                  kunserve_stream_t stream);

/* ------------------------------------- chunked-prefill attention (A5 ii) */

typedef struct {
  int32_t num_tiles;     /* workgroups of the launch (incl. padding)        */
  int32_t tile_q;        /* q rows per tile                                */
  int32_t plan_ints;     /* int32 entries of the plan buffer in use       */
  int32_t num_qo_heads;  /* heads the plan was made for                    */
  int32_t max_kv_len;    /* longest kv_len among the planned rows          */
  int32_t num_merge;     /* (tile, head) items whose KV range is split     */
  int32_t num_slots;     /* partial-result slots of the split items        */
  int32_t kv_chunk;      /* split length in tokens (0: nothing split)      */
  int32_t head_dim;      /* head_dim the plan was made for                 */
} kunserve_prefill_plan_info;

/* Upper bound of the prefill plan length (int32 entries); -1 for a bad
 * argument or a head_dim other than 64, 128 and 256. */
int64_t kunserve_prefill_plan_bound(const int32_t* q_indptr_host,
                                    int32_t num_seqs, int32_t num_qo_heads,
                                    int32_t head_dim);

/* Host-side plan: tiles the ragged q rows (q_len[b] = q_indptr[b+1] -
 * q_indptr[b]) of every q head into tiles of tile_q rows (256 for head_dim
 * 64 and 128, 128 for 256; other head dims: KUNSERVE_EUNSUPPORTED), and orders the
 * (row, tile, head) items so that items reading the same K/V (same row and
 * KV head) run back to back on one XCD (one L2), longest first. When the
 * items cannot fill num_cus CUs twice over (0: 256 CUs), each item's KV
 * range is split into chunks of kv_chunk tokens; split items write fp32
 * partials to the workspace and are merged within kunserve_paged_prefill.
 * Layout: num_tiles records of 6 ints (row or -1 for padding, first q row,
 * q head, KV begin, KV end, partial slot or -1), then num_merge records of
 * 5 ints (row, first q row, q head, first slot, splits). */
int kunserve_prefill_plan(const int32_t* q_indptr_host,
                          const int32_t* kv_len_host, int32_t num_seqs,
                          int32_t num_qo_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t num_cus, int32_t* plan_host,
                          int64_t plan_capacity,
                          kunserve_prefill_plan_info* info);

/* Workspace bytes needed by kunserve_paged_prefill for this plan (0 when
 * nothing is split). */
int64_t kunserve_prefill_workspace_bytes(const kunserve_prefill_plan_info* info);

/* Causal attention of the q_len[b] new rows of each sequence against its
 * kv_len[b] cached tokens (new ones already appended): q row i of
 * sequence b sees positions [0, kv_len[b] - q_len[b] + i]. q and out are
 * [num_tokens, num_qo_heads, head_dim] of the pool dtype; row i of
 * sequence b is token q_start[b] + i, or q_indptr[b] + i when q_start_dev
 * is NULL (q_len[b] = q_indptr[b+1] - q_indptr[b] either way). q_start
 * (device int32 [num_seqs]) lets the prefill rows of a mixed step
 * (kunserve/flash_backend.py:1870-1950) read q and write out in place,
 * among the step's decode tokens. fp16 or bf16 MFMA for Q.K^T and P.V,
 * fp32 accumulation and softmax. head_dim 64, 128 or 256
 * (KUNSERVE_EUNSUPPORTED otherwise); the plan must have been made for the
 * pool's head_dim. */
int kunserve_paged_prefill(const kunserve_kv_pool* pool, int32_t layer,
                           const kunserve_page_table* table,
                           const int32_t* q_indptr_dev,
                           const int32_t* q_start_dev,
                           const kunserve_tensor3* q, kunserve_tensor3* out,
                           int32_t num_qo_heads, float sm_scale,
                           const int32_t* plan_dev,
                           const kunserve_prefill_plan_info* info,
                           void* workspace_dev, int64_t workspace_bytes,
                           kunserve_stream_t stream);

/* MFMA calibration (no reference counterpart): each of num_workgroups
 * workgroups runs 8 waves (two per SIMD) of `iterations` rounds of two
 * independent 32x32x16 MFMAs (dtype KUNSERVE_DTYPE_F16 or _BF16) on
 * per-lane operands read once from operands_dev (num_workgroups * 8192
 * elements), and writes one float per thread to sink_dev (num_workgroups *
 * 512 floats). One launch issues num_workgroups * 16 * iterations MFMAs of
 * 32,768 flop. The benchmark times random and constant operands to give the
 * prefill kernel's ceiling on the part it runs on: the operands' bits set
 * the power the matrix cores draw, and so the clock the part holds. */
int kunserve_mfma_probe(int32_t dtype, const void* operands_dev, float* sink_dev,
                        int32_t num_workgroups, int32_t iterations,
                        kunserve_stream_t stream);

/* ------------------------------------------- fused page-id space (A6) */

/* When N instances fuse into an N-stage pipeline (KunServe's balloon), each
 * instance runs G = num_layers / N layers and its block manager numbers
 * pages in the fused space (kunserve/block_manager.py:231-269):
 *   - layer group i (layers [i*G, (i+1)*G)) of base page b is fused page
 *     i * P + b, P = base pages before fusion (convert_to_pipeline_format,
 *     :250-253; a stale request of rank r keeps r * P + b, :755-760);
 *   - extend pages (the dropped weight memory, pages P.. of the pool) are
 *     fused ids from P * N on (add_ex_fusion_blocks, :262-269), each of G
 *     layers: extend page P + q holds fused pages P*N + q*N + i, i < N;
 *   - pforward then receives max_num_pages = P*N + E
 *     (kunserve/flash_backend.py:2433-2440).
 * kunserve_fused_pool describes the same memory as a pool of
 * num_pages * N pages of G layers, and kunserve_fused_page_ids turns fused
 * ids into its page indices. Every other entry point then works unchanged
 * on the fused pool, with stage-local layer indices. Nothing is copied:
 * fused page r * P + b of stage r reads the bytes page b held before the
 * fusion. Requires page_stride == num_layers * layer_stride. Host only. */
int kunserve_fused_pool(const kunserve_kv_pool* pool, int64_t base_pages,
                        int32_t fusion_size, kunserve_kv_pool* fused);

/* Fused ids [0, num_fused_pages) -> page indices of the fused pool
 * (num_fused_pages = P*N + E). KUNSERVE_ERANGE on an id outside. Host only. */
int kunserve_fused_page_ids(const int32_t* fused_ids_host, int64_t n,
                            int64_t base_pages, int32_t fusion_size,
                            int64_t num_fused_pages, int32_t* pages_host);

/* ------------------------------------ parameter memory remap (pmm_drop) */

/* KV pools whose tail can be extended by the memory of dropped weight
 * layers, and given back (LlamaOp.pmm_drop / pmm_restore,
 * kunserve/worker.py:454-501, kunserve/flash_backend.py:716-725; the remap
 * is described at kunserve/llm_engine.py:553-558). The K and V pools are
 * address ranges reserved for base + max_extend pages of page_bytes each,
 * of which the first num_pages are mapped; a kunserve_kv_pool built on them
 * must carry that num_pages. These calls are synchronous on the host:
 * drop and restore wait for all work on the device to finish before they
 * move memory, and must not run concurrently with each other or with work
 * submitted from other threads. */
typedef struct kunserve_pmm kunserve_pmm;

/* Reserves the two ranges on `device` and maps base_pages of fresh device
 * memory at the start of each. page_bytes must be a multiple of the
 * device's mapping granularity (4 KiB on MI355X). */
int kunserve_pmm_create(int32_t device, int64_t page_bytes,
                        int64_t base_pages, int64_t max_extend_pages,
                        kunserve_pmm** out);

/* Allocates a weight segment of `bytes` (a multiple of 2 * page_bytes)
 * and maps it at an address of its own, returned in *address, where the
 * caller keeps one layer's weights. */
int kunserve_pmm_add_segment(kunserve_pmm* pmm, int64_t bytes,
                             int32_t* segment_id, void** address);

/* Drops a weight segment: its first half becomes K pages
 * [num_pages, num_pages + n) and its second half the V pages of the same
 * ids, n = bytes / (2 * page_bytes); the new page count is returned. The
 * segment's address stops being valid; the new pages hold its bytes
 * unchanged (the extend blocks of kunserve/block_manager.py:262-269). */
int kunserve_pmm_drop(kunserve_pmm* pmm, int32_t segment_id,
                      int64_t* num_pages);

/* Undoes the most recent drop: the pool's last n pages become the segment
 * again, at its original address and holding what those pages held. */
int kunserve_pmm_restore(kunserve_pmm* pmm, int32_t* segment_id,
                         int64_t* num_pages);

/* Current K and V pool bases (fixed for the handle's life) and page
 * count. */
int kunserve_pmm_pools(const kunserve_pmm* pmm, void** k, void** v,
                       int64_t* num_pages);

/* Waits for the device, unmaps and frees every pool page and segment. */
void kunserve_pmm_destroy(kunserve_pmm* pmm);

#ifdef __cplusplus
}
#endif

#endif /* KUNSERVE_HIP_H */
