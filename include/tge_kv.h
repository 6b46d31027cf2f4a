/*
 * tge_kv.h — C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * Replaces, behind a thin C boundary, what the reference engine does on the
 * CPU for its KV cache (AegeanWorks/Aegean-TGE, paths relative to its root):
 *   - the per-token K/V store          src/models/qwen2.cpp:2073-2093,
 *                                       1681-1702, 2308-2329, 88-120
 *   - GQA decode attention + split-K    include/tge/cpu/kernels.hpp:207-288
 *     (KernelSet::attention_head /      include/tge/core/dispatch.hpp:31-33
 *      attention_group + merge)         src/models/qwen2.cpp:1243-1522
 *   - the query-block prefill kernel    include/tge/cpu/kernels.hpp:290-317
 *                                       src/models/qwen2.cpp:1524-1571
 *   - the block table                   include/tge/models/block_table.hpp
 * Conventions (the reference's, restated for a C boundary):
 *   - every entry point returns an int status (TGE_OK = 0); no exception or
 *     C++ type crosses it. TGE_ERR_INVALID is the reference's
 *     std::invalid_argument (kernel argument checks, attention_scalar.cpp:
 *     11-44); TGE_ERR_RUNTIME its std::runtime_error (model/BlockTable misuse,
 *     qwen2.cpp:2036-2044, block_table.hpp:25-123).
 *   - outputs are left untouched when a call fails (backend.hpp:87-89).
 *   - all pointers are borrowed. Pointers documented "device" address HIP
 *     device memory; "host" pointers are read during the call only.
 *   - `stream` is a hipStream_t (NULL = the default stream). Work is
 *     enqueued asynchronously; the caller synchronises.
 *
 * Storage: K/V live in device pages of TGE_PAGE_TOKENS tokens, one pool per
 * layer, addressed by physical page id. The in-page order is chosen for the
 * CDNA4 matrix cores and documented below (tge_kv_k_index / tge_kv_v_index);
 * tge_kv_gather turns pages back into the reference's flat row-major rows.
 */
#ifndef TGE_KV_H
#define TGE_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGE_PAGE_TOKENS 16 /* block_table.hpp:19 kBlockTokens */

enum tge_status {
  TGE_OK = 0,
  TGE_ERR_INVALID = -1,     /* bad argument (std::invalid_argument) */
  TGE_ERR_RUNTIME = -2,     /* misuse of model/table state (std::runtime_error) */
  TGE_ERR_UNAVAILABLE = -3, /* no usable gfx950 device, or forced off */
  TGE_ERR_DEVICE = -4,      /* a HIP runtime call failed */
  TGE_ERR_CAPACITY = -5     /* out of device/host memory (a full
                               BlockTable is TGE_ERR_RUNTIME, as the
                               reference throws) */
};

enum tge_kv_format {
  TGE_KV_F16 = 1, /* IEEE half bits, the reference's float_to_half recipe */
  TGE_KV_I8 = 2   /* int8 codes, one scale per 32 values (store_kv_q8) */
};

enum tge_scale_format {
  TGE_SCALE_F16 = 0, /* scale stored as float_to_half(fp32 scale) */
  TGE_SCALE_F32 = 1  /* scale stored as the fp32 value (reference layout) */
};

/* Text for a status code; the last error message of the calling thread. */
const char* tge_status_string(int status);
const char* tge_last_error(void);

/*
 * Backend bring-up, never throws, idempotent (reference gpu::init(),
 * backend.hpp:52-54). Returns TGE_OK when a gfx950 device is usable.
 * Setting the environment variable TGE_FORCE_UNAVAILABLE=1 makes it report
 * TGE_ERR_UNAVAILABLE (for fallback tests).
 */
int tge_backend_init(void);
/* Name of the device's architecture (e.g. "gfx950"), or "" when none. */
const char* tge_backend_arch(void);

/* ---------------------------------------------------------------------------
 * Page pool. Device memory for `layers` x `pages` x `kv_heads` page blocks.
 * Each page block holds TGE_PAGE_TOKENS tokens of one KV head at the block
 * width W = 64 (head_dim <= 64), 128 (head_dim <= 128) or 256 (head_dim <=
 * 256), dims from head_dim on stored as zeros, its parts back to back (one
 * contiguous run of memory per block):
 *   K part, then V part: 16 * W elements each (f16 bits or int8 codes)
 *   I8 only, K scales, then V scales: 16 * W/32 scales each (f16 bits or
 *   fp32)
 * Block (page, kv_head) of a layer is block number page*kv_heads + kv_head.
 * Element (token t, dim d) of a block's part sits at:
 *   K: tge_kv_k_index(t, d, format)  V: tge_kv_v_index(t, d, format)
 *   scale of (t, block b = d/32): tge_kv_scale_index(t, b, W)
 * head_dim: a multiple of 4 up to 256 (F16) or of 32 up to 256 (I8, whose
 * scales cover 32-dim blocks). The reference takes any head_dim > 0
 * (attention_scalar.cpp:11-14; int8 % 32, qwen2.cpp:406-409); heads wider
 * than 256 are not supported here. q, k, v and out rows always have the
 * model's head_dim.
 * ------------------------------------------------------------------------ */
typedef struct tge_kv_pool tge_kv_pool;

typedef struct {
  int layers;
  int pages;        /* physical pages per layer (BlockTable capacity) */
  int kv_heads;
  int head_dim;
  int format;       /* enum tge_kv_format */
  int scale_format; /* enum tge_scale_format, I8 only */
} tge_kv_pool_desc;

/* One layer of a pool: the parts of block 0; the parts of block n sit
 * n * block_bytes further on. */
typedef struct {
  void* k;        /* device, K part of block 0 (the layer's base address) */
  void* v;        /* V part of block 0 */
  void* k_scales; /* NULL for F16 */
  void* v_scales;
  size_t kv_block_bytes;    /* bytes of one K (or V) part */
  size_t scale_block_bytes; /* bytes of one scale part (0 for F16) */
  size_t block_bytes;       /* bytes of a whole page block: the block stride */
  int block_dims;           /* the block width W (64, 128 or 256) */
} tge_kv_layer_view;

int tge_kv_pool_create(const tge_kv_pool_desc* desc, tge_kv_pool** out);
void tge_kv_pool_destroy(tge_kv_pool* pool);
int tge_kv_pool_layer(const tge_kv_pool* pool, int layer,
                      tge_kv_layer_view* out);
/* Device bytes the pool holds. */
size_t tge_kv_pool_bytes(const tge_kv_pool* pool);
/* Copy page src's blocks (every layer, every KV head) over page dst: the copy
 * of copy-on-write prefix sharing. The reference copies a prefix's flat rows
 * into the new slot instead (prime_cache_from_table, qwen2.cpp:1973-2026).
 * Asynchronous on `stream`. */
int tge_kv_copy_page(tge_kv_pool* pool, int src_page, int dst_page, void* stream);

/* In-page element index of (token, dim) in a K or V part of the given
 * format (TGE_KV_F16 or TGE_KV_I8; -1 for another value), and of the scale
 * of (token, 32-dim block) in blocks of width W (the third argument, 64, 128
 * or 256; the pool's tge_kv_layer_view.block_dims). A part is a sequence of
 * 16-byte pieces of PE = 8 (F16) or 16 (I8) elements; piece i of lane l
 * (l = 0..63) sits at element (i*64 + l)*PE, so a 64-lane wave reads a part
 * with one 1-KiB contiguous load per piece. Lane l holds elements j = 0 ..
 * 8*W/32-1 of its matrix-core operand, element j in piece j/PE at position
 * j%PE:
 *   K: lane = ((d/4)&3)*16 + t,   j = (d/32)*8 + ((d/16)&1)*4 + (d&3)
 *   V: lane = (t/4)*16 + (d&15),  j = (d/32)*8 + ((d/16)&1)*4 + (t&3)
 *   index = ((j/PE)*64 + lane)*PE + j%PE   (the same for every W)
 *   scale: ((t/4)*NP + b)*4 + (t&3), NP = W/32 */
int tge_kv_k_index(int token, int dim, int format);
int tge_kv_v_index(int token, int dim, int format);
int tge_kv_scale_index(int token, int block, int head_dim);

/* ---------------------------------------------------------------------------
 * Batch: the sessions one step works on. A plan is built once per step on the
 * host and uploaded once; every layer's append and attention then reuse it.
 *
 * Session s owns n_new[s] new tokens at positions ctx[s] .. ctx[s]+n_new[s]-1
 * (appended first, then attended causally: new token i sees positions
 * 0 .. ctx[s]+i, the store-then-attend order of qwen2.cpp:2073-2095).
 * Its block table lists physical page ids in logical order:
 * page_ids[table_offsets[s] .. table_offsets[s+1]) and must cover
 * ceil((ctx+n_new)/16) pages. Rows of q/k/v/out are the sessions' new tokens
 * in session order (session s starts at row sum(n_new[0..s-1])), the
 * per-token row order of forward_batch (qwen2.cpp:1613-1747).
 *   q, out: [rows][q_heads*head_dim] fp32     k, v: [rows][kv_heads*head_dim] fp32
 * ------------------------------------------------------------------------ */
typedef struct tge_batch tge_batch;

typedef struct {
  int n_sessions;
  const int* ctx;           /* host [n_sessions] */
  const int* n_new;         /* host [n_sessions], >= 1 */
  const int* table_offsets; /* host [n_sessions+1] */
  const int* page_ids;      /* host [table_offsets[n_sessions]] */
  int q_heads;              /* multiple of the pool's kv_heads, at most 128
                               query heads per KV head (64 at head_dim
                               > 128) */
} tge_batch_desc;

int tge_batch_create(tge_batch** out);
void tge_batch_destroy(tge_batch* batch);

/* Validates the description against `pool`, builds the work lists and
 * uploads tables and plan (one host-to-device copy on `stream`). A failure
 * leaves the batch unplanned; TGE_ERR_CAPACITY when device or pinned host
 * memory runs out (a later, smaller plan allocates again). */
int tge_batch_plan(tge_batch* batch, const tge_kv_pool* pool,
                   const tge_batch_desc* desc, void* stream);

/* Plan statistics: total new-token rows, decode work items and the largest
 * number of splits of one (session, KV head); a plan whose rows exceed a
 * decode unit reports 0 work items and 0 splits. */
int tge_batch_info(const tge_batch* batch, int* rows, int* work_items,
                   int* max_splits);

/* Kernel timing of attention calls (no counterpart in the reference: it is
 * for benchmarks and telemetry). Enabling clears the record; while enabled,
 * each decode or prefill attention call on `batch` records HIP timing events
 * on its stream before the paged attention kernel, between it and the split
 * merge kernel, and after the merge. tge_batch_kernel_times waits for every
 * recorded call and returns their number and the summed durations in
 * microseconds; merge_us sums only the calls that launched the split merge
 * kernel (a call whose plan has no split pieces adds nothing to it). Calls
 * issued back to back keep the launch latency of the host out of the
 * bracketed intervals. */
int tge_batch_set_profiling(tge_batch* batch, int enable);

/* Static sparse attention for the batch's attention calls (SparseConfig,
 * qwen2.hpp:30-35; set_sparse_config, qwen2.cpp:182-189; kernels
 * attention_head_static_sparse_*_avx2, attention_avx2.cpp:263-490): a query
 * whose span exceeds sink + window attends to positions < sink, every
 * stride-th position from sink on, and the last `window` positions (the
 * kept set of build_sparse_index, qwen2.cpp:192-220); shorter spans stay
 * dense. enabled 0 turns it off. stride < 2, sink < 0 or window < 1 ->
 * TGE_ERR_RUNTIME (the reference's runtime_error). With stride > 16 the
 * decode kernel skips pages holding no kept position. The reference applies
 * it to f32/f16 caches only (uses_sparse, qwen2.cpp:1313-1317); here any
 * pool format. Persists across plans. */
int tge_batch_set_sparse(tge_batch* batch, int enabled, int sink, int window,
                         int stride);
int tge_batch_kernel_times(const tge_batch* batch, int* calls, float* attention_us,
                           float* merge_us);

/*
 * Fused quantize-and-scatter of every new token's K and V rows into its page
 * slot (the store sites above). F16: bits of the reference float_to_half
 * (kernels.hpp:358-386). I8: per 32 values, codes and scale exactly as
 * quantize_kv_block (qwen2.cpp:88-104); the scale is stored as fp32 or as
 * float_to_half(scale) per the pool's scale_format.
 */
int tge_kv_append(const tge_batch* batch, tge_kv_pool* pool, int layer,
                  const float* k, const float* v, void* stream);

/*
 * Decode attention for every session of the batch (n_new small: decode and
 * speculative verify; the reference's attention_head / attention_group
 * plugins, kernels.hpp:231,285, under the schedules of qwen2.cpp:1243-1467
 * and 1705-1747). Each (session, kv head) is one stream of pages read once
 * for its whole query-head group; the streams are laid end to end and cut
 * into one share per resident workgroup (balanced by pages, per-piece cost
 * and the workgroup's dispatch rank on its CU), and a stream cut into
 * several pieces is merged by a reduction pass (merge_gqa_chunks,
 * qwen2.cpp:1469-1522).
 * softmax scale = 1/sqrt(head_dim) (qwen2.cpp:1278). Requires
 * n_new*group <= 64 for every session.
 */
int tge_decode_attention(const tge_batch* batch, const tge_kv_pool* pool,
                         int layer, const float* q, float* out, void* stream);

/*
 * tge_kv_append followed by tge_decode_attention, in one call: the
 * store-then-attend order of forward / forward_batch (qwen2.cpp:2073-2095,
 * 1681-1747). A small step (every session's rows fit a decode unit, at
 * most 48 rows per session at head_dim 128, at most 4096 page blocks in the
 * step; with a static sparse subset and int8 pages with fp32 scales, at most
 * 16 rows per session and head_dim 128) runs as one kernel: the workgroup
 * that reads a segment's new positions stores the new rows of its KV head
 * first (the same bits as tge_kv_append), and a context cut into several
 * pieces is merged by the last piece to finish. A larger
 * step runs the decode kernel and its merge, the decode kernel taking the
 * new rows from k and v: each wave encodes the rows of the pages it reads
 * (the same bits as tge_kv_append), writes them into its on-chip copy of
 * such a page as it lands and stores them into the pool after its last
 * page. Where its variant cannot (head_dim above 128, more than 32 rows per
 * unit, more new rows on one wave's pages than it holds, a static sparse
 * subset) the append runs first, as its own launch. Outputs equal those of
 * the two calls within the attention tolerance (the same math, other page
 * splits; bit for bit on a large step).
 */
int tge_decode_step(const tge_batch* batch, tge_kv_pool* pool, int layer, const float* q,
                    const float* k, const float* v, float* out, void* stream);

/* Workgroups of the one-kernel step tge_decode_step launches for the
 * current plan, and the most pieces one (session, KV head) context is cut
 * into; 0 and 0 when the step runs the append and decode kernels. No
 * counterpart in the reference: for benchmarks and tests. */
int tge_batch_step_info(const tge_batch* batch, int* workgroups, int* max_pieces);

/* 1 in *stores when tge_decode_step runs the current plan (and sparse
 * setting) as a decode launch that stores the new rows itself (no append
 * launch), else 0. No counterpart in the reference: for benchmarks and
 * tests. */
int tge_batch_decode_stores_rows(const tge_batch* batch, int* stores);

/*
 * tge_decode_attention for callers that cannot allocate memory (tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Not for stream capture: the plan is built on the host and
 * copied from host memory at each call, so a captured copy would replay
 * stale contents; a call on a stream that is capturing returns
 * TGE_ERR_INVALID before anything is enqueued. It plans the step from `desc` on the
 * host (the decode plan of tge_batch_plan; dense attention, no sparse
 * subset) and runs the same kernels, so its output equals that of
 * tge_batch_plan + tge_decode_attention on the same description bit for
 * bit. The plan image and the split-K partials live in a static device
 * array of 32 MiB per GPU, held until the process ends: at most 4 MiB of
 * plan (sessions, block tables, work lists) and 28 MiB of partials; a
 * larger step returns TGE_ERR_CAPACITY before anything runs. It calls no
 * device or pinned-host allocation. Every call on one GPU shares that
 * array, so calls that overlap on one GPU (different streams, or threads)
 * race; calls on one stream are ordered. q, out and the pool are as in
 * tge_decode_attention; the K/V rows of the step must already be appended.
 */
int tge_decode_attention_static(const tge_batch_desc* desc, const tge_kv_pool* pool,
                                int layer, const float* q, float* out, void* stream);

/*
 * Chunked-prefill block attention (attention_block_head_avx2,
 * attention_avx2.cpp:660-864): each new token attends causally to every
 * prior page and the chunk itself, on f16 MFMA (Q rounded to f16 as in
 * decode; I8 pools run the same kernel where the reference takes its
 * per-token i8 path, qwen2.cpp:1535-1538). Tiles of up to 128
 * (query, head) rows of one KV head's query group (64 at head_dim > 128,
 * and for steps whose 128-row tiles would leave compute units idle);
 * long prefixes are split and merged like decode.
 */
int tge_prefill_attention(const tge_batch* batch, const tge_kv_pool* pool,
                          int layer, const float* q, float* out, void* stream);

/*
 * Attention for a mixed step (continuous batching: forward_batch rows of
 * many sessions, some decoding, some prefilling a chunk; qwen2.cpp:1613-1747
 * handles any mix per token), in one call on one plan: sessions with
 * n_new*group <= 64 take the decode path, the others the block-prefill path.
 * A dense step is one kernel launch (decode shares and prefill tiles as
 * roles of one kernel, split contexts merged inside the launch); with a
 * static sparse subset the two kinds run as two launches. A step of only
 * one kind is exactly tge_decode_attention or tge_prefill_attention.
 */
int tge_batch_attention(const tge_batch* batch, const tge_kv_pool* pool,
                        int layer, const float* q, float* out, void* stream);

/*
 * Device gather of one session's positions [0, count) back to the flat
 * row-major layout of the reference cache (gather_blocks_row_major,
 * kv_block_layout.hpp:64-84, applied per element): k_rows/v_rows receive
 * [count][kv_heads*head_dim] elements (f16 bits or int8 codes), scales
 * [count][kv_heads*head_dim/32] (I8 only; may be NULL otherwise).
 */
int tge_kv_gather(const tge_batch* batch, const tge_kv_pool* pool, int layer,
                  int session, int count, void* k_rows, void* v_rows,
                  void* k_scales, void* v_scales, void* stream);

/* ---------------------------------------------------------------------------
 * Kernel level: the reference's GPU placement predicate and its
 * attention_group plugin slot (KernelSet::attention_group,
 * include/tge/core/dispatch.hpp:31-33), for a caller that keeps the
 * reference's own schedule (Qwen2::attention_gqa, qwen2.cpp:1382-1467: KV
 * heads x position chunks, then merge_gqa_chunks) and routes each chunk
 * here instead of to attention_group_avx2.
 * ------------------------------------------------------------------------ */
#define TGE_GQA_MIN_SPAN 256 /* GpuThresholds::kGqaMinSpan, backend.hpp:49 */

/* gpu::eligible_gqa (backend.hpp:170-174 with want_gqa_gpu :124-126, the
 * predicate Qwen2::wants_gpu_gqa wraps, qwen2.cpp:786-795): 1 when the GPU
 * was requested, more than one thread runs the schedule, the span reaches
 * TGE_GQA_MIN_SPAN, the caller follows the grouped schedule (uses_gqa) and
 * the attention is dense; else 0. A pure function (no device call): backend
 * readiness is tge_backend_init's, as the reference's dispatcher adds
 * use_gpu(). */
int tge_eligible_gqa(int requested, int span, int threads, int follows_schedule,
                     int dense_only);

/* AttentionGroupArgs (kernels.hpp:262-283) over pages. The group_heads query
 * heads of KV head `kv_head` (rows of `queries`, [group_heads][head_dim]
 * fp32, device) attend to positions [first, first + count) of one session
 * of layer `layer`, whose block table is page_ids (device, logical order,
 * covering position first + count - 1). Per head the outputs are the
 * reference group kernel's running online-softmax state (attention_group_
 * scalar, attention_scalar.cpp:117-199): maxima[h] the largest score,
 * sums[h] = sum of exp(score - max), accumulators[h][d] = sum of
 * exp(score - max) * v[d], for the caller's chunk merge (merge_gqa_chunks,
 * qwen2.cpp:1469-1522); count 0 gives (-inf, 0, 0). Scores are
 * (q . k) * scale in fp32; K and V are dequantised in fp32. Rejects
 * (TGE_ERR_INVALID) null pointers, a layer or KV head outside the pool,
 * first < 0, count < 0 and group_heads outside 1..128. A page id outside
 * the pool is not read: that call's outputs become NaN. Asynchronous on
 * `stream`. */
typedef struct {
  const tge_kv_pool* pool;
  int layer;
  int kv_head;
  const int* page_ids;  /* device */
  int first;
  int count;
  const float* queries; /* device [group_heads][head_dim] */
  int group_heads;
  float scale;          /* the reference passes 1/sqrt(head_dim) */
  float* maxima;        /* device [group_heads] */
  float* sums;          /* device [group_heads] */
  float* accumulators;  /* device [group_heads][head_dim] */
} tge_attention_group_args;

int tge_attention_group(const tge_attention_group_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Fused bias + RoPE + append: the per-token sequence before the store in
 * forward / forward_batch / prefill_run (qwen2.cpp:2062-2093, 1665-1702,
 * 2286-2329): q += q_bias; k += k_bias; v += v_bias; apply_rope(q);
 * apply_rope(k) (NeoX halves, qwen2.cpp:1196-1230); store k and v. One
 * launch does it for every row of the plan; the rotated q goes to q_out
 * (which may be q itself) for the attention call. Row i's position is its
 * plan position (ctx + j of its session) and indexes the tables. head_dim
 * must be a multiple of 16 here (TGE_ERR_INVALID otherwise): each NeoX
 * half is whole runs of 8 dims.
 * ------------------------------------------------------------------------ */
typedef struct {
  const float* q;        /* [rows][q_heads*head_dim] or NULL (K/V only) */
  float* q_out;          /* [rows][q_heads*head_dim]; may equal q */
  const float* k;        /* [rows][kv_dim], before bias and RoPE */
  const float* v;        /* [rows][kv_dim], before bias */
  const float* q_bias;   /* [q_heads*head_dim] or NULL */
  const float* k_bias;   /* [kv_dim] or NULL */
  const float* v_bias;   /* [kv_dim] or NULL */
  const float* rope_cos; /* device [positions][head_dim/2]: rope_cos_ of */
  const float* rope_sin; /* qwen2.cpp:608-681 (tge_rope_tables builds them) */
  int rope_positions;    /* rows of the tables; every plan position < this */
  int rope_fma;          /* 1: apply_rope_avx2 rounding (the default CPU
                            path), 0: apply_rope_scalar rounding */
} tge_rope_append_args;

int tge_kv_append_rope(const tge_batch* batch, tge_kv_pool* pool, int layer,
                       const tge_rope_append_args* args, void* stream);

/* Host: the rotary tables of qwen2.cpp:608-681 for positions [0, positions):
 * freq_i = theta^(-2i/head_dim) / factor_i (factors NULL: all ones),
 * angle = position * freq_i, cos/sin(angle) * attn_factor, in float with
 * the C library's powf/cosf/sinf. Outputs are host [positions][head_dim/2]. */
int tge_rope_tables(int head_dim, int positions, float theta, float attn_factor,
                    const float* factors, float* cos_out, float* sin_out);

/* ---------------------------------------------------------------------------
 * Block table (block_table.hpp:21-130), host-side page-id allocator.
 * allocate: LIFO free list (a fresh table hands out 0,1,2,...); release at
 * refcount 0 returns the page to the free list; misuse -> TGE_ERR_RUNTIME.
 * ------------------------------------------------------------------------ */
typedef struct tge_block_table tge_block_table;

int tge_block_table_create(int blocks, int block_tokens, tge_block_table** out);
void tge_block_table_destroy(tge_block_table* table);
int tge_block_table_allocate(tge_block_table* table, int* block);
int tge_block_table_share(tge_block_table* table, int block);
int tge_block_table_release(tge_block_table* table, int block);
int tge_block_table_refcount(const tge_block_table* table, int block, int* out);
int tge_block_table_free_count(const tge_block_table* table);
int tge_block_table_capacity(const tge_block_table* table);
int tge_block_table_remember_prefix(tge_block_table* table, uint64_t hash,
                                    int block);
/* -1 on a miss (find_prefix). */
int tge_block_table_find_prefix(const tge_block_table* table, uint64_t hash);
/* slot_for (block_table.hpp:77-82); hash_tokens FNV-1a (:85-98). */
int tge_slot_for(int logical_pos, int block_tokens, int* block, int* offset);
int tge_hash_tokens(const int* tokens, int count, uint64_t* out);

/* ---------------------------------------------------------------------------
 * Qwen2-shaped KV driver: the store-then-attend sequence of Qwen2::forward /
 * forward_batch / prefill_run / verify_draft / reset_cache (qwen2.hpp:249-
 * 297) over paged device KV. Weights are outside this path: callers pass the
 * post-RoPE q/k/v of each layer (device pointers, rows as in the batch).
 * A step is begun once (pages allocated, plan uploaded) and then run layer
 * by layer.
 * ------------------------------------------------------------------------ */
typedef struct tge_qwen2_kv tge_qwen2_kv;

typedef struct {
  int layers;
  int q_heads;
  int kv_heads;
  int head_dim;
  int context;      /* max positions per sequence (qwen2.cpp:25-26) */
  int sequences;    /* KV slots */
  int pages;        /* physical pages in the shared pool */
  int format;       /* enum tge_kv_format */
  int scale_format; /* enum tge_scale_format */
} tge_qwen2_kv_config;

int tge_qwen2_kv_create(const tge_qwen2_kv_config* config, tge_qwen2_kv** out);
void tge_qwen2_kv_destroy(tge_qwen2_kv* model);

/* forward(sequence, token, position): one token of one sequence. */
int tge_qwen2_kv_begin_forward(tge_qwen2_kv* model, int sequence, int position,
                               void* stream);
/* forward_batch: row i is (sequences[i], positions[i]); each sequence's rows
 * must be consecutive positions in ascending row order. */
int tge_qwen2_kv_begin_forward_batch(tge_qwen2_kv* model, const int* positions,
                                     int count, const int* sequences,
                                     void* stream);
/* prefill_run: `count` tokens of one sequence from start_position. */
int tge_qwen2_kv_begin_prefill(tge_qwen2_kv* model, int sequence,
                               int start_position, int count, void* stream);
/* verify_draft: count <= 6 (kSpeculativeBatch, qwen2.hpp:140) draft tokens. */
int tge_qwen2_kv_begin_verify(tge_qwen2_kv* model, int sequence,
                              int start_position, int count, void* stream);
/* Append the step's K/V rows for `layer`, then attend. */
int tge_qwen2_kv_layer(tge_qwen2_kv* model, int layer, const float* q,
                       const float* k, const float* v, float* out,
                       void* stream);
/* layer() with the step before the store fused: args->k/v/q are the rows
 * before bias and RoPE (tge_kv_append_rope); attention then reads
 * args->q_out. */
int tge_qwen2_kv_layer_rope(tge_qwen2_kv* model, int layer,
                            const tge_rope_append_args* args, float* out,
                            void* stream);
/* Store the step's K/V rows for `layer` without attending: cache priming
 * (prime_cache_from_table, qwen2.hpp:283-288). */
int tge_qwen2_kv_store(tge_qwen2_kv* model, int layer, const float* k,
                       const float* v, void* stream);
/* reset_cache(sequence): release the sequence's pages in logical order. */
int tge_qwen2_kv_reset(tge_qwen2_kv* model, int sequence);
/* Positions currently cached for a sequence; its page ids (logical order). */
int tge_qwen2_kv_length(const tge_qwen2_kv* model, int sequence);
int tge_qwen2_kv_pages(const tge_qwen2_kv* model, int sequence, int* ids,
                       int cap);
const tge_kv_pool* tge_qwen2_kv_pool(const tge_qwen2_kv* model);
const tge_batch* tge_qwen2_kv_batch(const tge_qwen2_kv* model);
int tge_qwen2_kv_free_pages(const tge_qwen2_kv* model);
/* set_sparse_config (qwen2.cpp:182-189): static sparse attention for every
 * later step, applied to F16 caches only as in the reference (i8 stays
 * dense, uses_sparse qwen2.cpp:1313-1317). See tge_batch_set_sparse. */
int tge_qwen2_kv_set_sparse(tge_qwen2_kv* model, int enabled, int sink,
                            int window, int stride);

/* Shared prefixes over pages (the BlockTable recipe of prefix sharing,
 * replacing the reference's four-slot snapshot table, qwen2.cpp:40-72),
 * matched token by token.
 *
 * remember_prefix: record, for each cached page among the sequence's first
 * `count` tokens, the tokens it holds (the last page may be partial) and
 * the page before it (the populate step, qwen2.cpp:2388-2465, without its
 * four-slot and 256-token caps); full pages are also keyed in the block
 * table under hash_tokens of tokens[0, 16(k+1)). Returns the tokens
 * recorded.
 * shared_prefix_len: the longest run of tokens, from the first, that a
 * recorded chain of pages holds (qwen2.cpp:1948-1971). Every token is
 * compared; a hash alone never decides a match.
 * attach_prefix: an empty sequence takes that run by reference count (no
 * copy; qwen2.cpp:1973-2026 copies rows), its last page possibly in part,
 * and is cached up to the returned length; the caller prefills from there.
 * A later step that writes into a page another sequence still holds copies
 * it first (copy-on-write), so sharers never see each other's writes; a
 * step that rewrites recorded rows of a page in place drops the record of
 * that page and of the pages recorded after it, and a page's record goes
 * when its last holder releases it. */
int tge_qwen2_kv_remember_prefix(tge_qwen2_kv* model, int sequence,
                                 const int* tokens, int count);
int tge_qwen2_kv_shared_prefix_len(const tge_qwen2_kv* model, const int* tokens,
                                   int count);
int tge_qwen2_kv_attach_prefix(tge_qwen2_kv* model, int sequence,
                               const int* tokens, int count);

/* The driver's own block table (a view, owned by the driver; do not destroy).
 * Lets a caller pre-shape the free list before the first step; pages held by
 * sequences must not be released through it. */
tge_block_table* tge_qwen2_kv_table(tge_qwen2_kv* model);

/*
 * Health check, with no counterpart in the reference: the number of bounded
 * in-kernel waits that ran out since the process started (the block-prefill
 * kernel's tile barrier between its two halves of waves, bounded at about
 * 0.2 s so that a launch can never hang). Non-zero means some launch
 * finished with wrong rows. Synchronous (waits for the device counter).
 */
int tge_wait_expiries(unsigned int* count);

/* ---------------------------------------------------------------------------
 * Measurement helper, with no counterpart in the reference: the HBM read
 * ceiling of this GPU, beside the 8 TB/s specification. One launch reads
 * every byte of the device buffer `buf` once and writes nothing:
 *   TGE_READ_STREAM  4 KiB chunks dealt round-robin to the workgroups
 *                    (256 threads, `workgroups_per_cu` per compute unit,
 *                    1..64), 16 B per lane, eight chunks in flight per
 *                    workgroup (bytes: a multiple of 4096);
 *   TGE_READ_BLOCKS  bytes / block_bytes blocks of `block_bytes` (16..17408,
 *                    a multiple of 16; a pool's page-block size), one wave
 *                    per block, in a scattered order, two blocks in flight
 *                    per wave (the decode kernel's access shape).
 * The caller times the launch (e.g. events on `stream`).
 */
enum tge_read_pattern { TGE_READ_STREAM = 0, TGE_READ_BLOCKS = 1 };
int tge_read_ceiling(const void* buf, size_t bytes, int pattern, int workgroups_per_cu,
                     int block_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TGE_KV_H */
