/*
 * CPU oracle for the paged-KV hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference engine's scalar semantics
 * (AegeanWorks/Aegean-TGE). It exists so that tests/, the smoke check and the
 * CPU-baseline leg of bench.py can check the HIP path against it. Nothing in
 * the product links, loads or calls this library; the product fails loudly
 * when its HIP extension is missing instead of falling back to code here.
 *
 * Every function cites the reference file:line it follows. Build flags are
 * fixed by oracle/Makefile: -O2 -ffp-contract=off, baseline x86-64 (SSE2
 * scalar float), which is what the reference's ISO-C++20 scalar TUs compile
 * to (reference CMakeLists.txt:12-14,36-43: no ISA flags on qwen2.cpp or
 * attention_scalar.cpp, CMAKE_CXX_EXTENSIONS OFF so GCC does not contract).
 *
 * Pinning status of each function (how it is checked, see tests/):
 *   orc_half_to_float        exhaustive 2^16 vs hardware F16C, vs oracle/_ref
 *   orc_float_to_half        exhaustive 2^32 vs an independent bit model, KATs
 *                            from test_attention.cpp:107-115, vs oracle/_ref
 *   orc_quantize_kv_block    closed forms: exact-ratio blocks, the all-zero
 *                            sign rule, +-0.49999997 rounding, blocks whose
 *                            codes change if x*inv +- 0.5 is fused into one
 *                            multiply-add, blocks whose codes change if they
 *                            come from the f16-rounded scale (expected codes
 *                            from exact float64 arithmetic); property checks
 *                            on random blocks (nearest code within fp32
 *                            slack, the maximum maps to +-127)
 *   orc_attention_head       vs oracle/_ref attention_head_scalar (bit-exact),
 *                            closed forms (span 1, equal keys, dominant key),
 *                            float64 truth
 *   orc_attention_group      vs oracle/_ref attention_group_scalar (bit-exact)
 *   orc_merge_chunks         split-count invariance vs orc_attention_head,
 *                            closed forms
 *   orc_attention_block_head vs orc_attention_head per query (1e-5), vs
 *                            oracle/_ref attention_block_head_avx2 (1e-4)
 *   orc_rope_neox            vs oracle/_ref apply_rope_avx2 (fma = 1) and
 *                            apply_rope_scalar (fma = 0), bit-exact; closed
 *                            forms (position 0 is the identity, the two
 *                            roundings differ only through the fused step)
 *   orc_bias_rope_row        composition of the above with fp32 bias adds
 *                            (the reference's loop order, checked through
 *                            orc_rope_neox and a float64 model)
 *   orc_rope_tables          same C library calls as the reference loader;
 *                            within 2 ulp of float64 truth
 *   orc_sparse_index         closed forms (dense below sink + window, sink /
 *                            strided middle / window parts), and the kept set
 *                            the reference kernels walk (through them)
 *   orc_attention_head_sparse vs oracle/_ref attention_head_static_sparse_avx2
 *                            and _fp16_avx2 (1e-5: their exp is a vectorised
 *                            approximation); equals orc_attention_head when
 *                            the span fits sink + window, and on a cache
 *                            whose dropped rows were removed
 */
#ifndef TGE_ORACLE_H
#define TGE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KV storage formats of the oracle's flat cache. */
enum { ORC_KV_F32 = 0, ORC_KV_F16 = 1, ORC_KV_I8 = 2 };

/* kernels.hpp:325-354 — exact IEEE half -> float. */
float orc_half_to_float(uint16_t value);

/* kernels.hpp:358-386 — float -> half with the reference's guard-bit rounding
 * (ties away from zero in magnitude, |x| < 2^-24 flushes to signed zero,
 * NaN -> sign|0x7E00, overflow -> sign|0x7C00). */
uint16_t orc_float_to_half(float value);

/* Bulk forms over n elements. */
void orc_float_to_half_n(const float* src, uint16_t* dst, size_t n);
void orc_half_to_float_n(const uint16_t* src, float* dst, size_t n);

/* qwen2.cpp:88-104 — one 32-value block to int8 codes; returns the fp32
 * scale (absmax / 127). */
float orc_quantize_kv_block(const float* source, int8_t* destination);

/* qwen2.cpp:109-120 (store_kv_q8) generalised to n rows of kv_dim: codes at
 * row*kv_dim, fp32 scales at row*kv_dim/32. */
void orc_quantize_rows(const float* src, int rows, int kv_dim, int8_t* codes,
                       float* scales);

/* Flat element offset of one (sequence, layer) slot, qwen2.hpp:112-119. */
size_t orc_kv_layer_offset(int sequence, int layer, int block_count,
                           int context, int kv_dim);

/*
 * Store of one token's K and V rows into the flat cache at element offset
 * `slot` — the store sites qwen2.cpp:2073-2093 / 1681-1702 / 2308-2329.
 * format F16: k16/v16 receive orc_float_to_half bits.
 * format I8:  k8/v8 codes, ks/vs fp32 scales at slot/32 (store_kv_q8).
 * format F32: k32/v32 plain copy.
 */
void orc_store_token(int format, const float* k, const float* v, int kv_dim,
                     size_t slot, void* k_cache, void* v_cache,
                     float* k_scales, float* v_scales);

/*
 * One query head against `span` rows — attention_scalar.cpp:48-115
 * (attention_head_scalar). `keys`/`values` point at the head's first element
 * (row 0, column kv_head*head_dim) and rows are kv_stride apart. For I8 the
 * scale arrays are indexed exactly as the reference does:
 * scales[token*(kv_stride/32) + index/32], pointing at (offset/32).
 * `scores` (span floats) is overwritten with the unnormalised exponentials.
 * Returns 0, or -1 on the argument errors attention_scalar.cpp:11-44 throws.
 */
int orc_attention_head(int format, const float* query, const void* keys,
                       const void* values, const float* k_scales,
                       const float* v_scales, int kv_stride, int span,
                       int head_dim, float scale, float* scores, float* out);

/* Same computation in float64 from the same dequantised inputs (the "truth"
 * the fp32 paths are priced against). */
int orc_attention_head_f64(int format, const float* query, const void* keys,
                           const void* values, const float* k_scales,
                           const float* v_scales, int kv_stride, int span,
                           int head_dim, double scale, double* out);

/*
 * One KV group over `count` rows with online softmax — attention_scalar.cpp:
 * 117-199 (attention_group_scalar). Writes maxima[group_heads],
 * sums[group_heads], accumulators[group_heads*head_dim].
 */
void orc_attention_group(int format, const float* queries, const void* keys,
                         const void* values, const float* k_scales,
                         const float* v_scales, int kv_stride, int count,
                         int head_dim, int group_heads, float scale,
                         float* maxima, float* sums, float* accumulators);

/*
 * Split-K reduction of one query head — qwen2.cpp:1469-1522
 * (merge_gqa_chunks). State index of chunk c is base + c*group + group_head.
 */
void orc_merge_chunks(const float* maxima, const float* sums,
                      const float* accumulators, size_t base, int chunks,
                      int group, int group_head, int head_dim, float* out);

/*
 * Split-K schedule for one decode step of one sequence — qwen2.cpp:1382-1467
 * (attention_gqa): chunk count from `threads`, group kernel per
 * (kv_head, chunk), then merge per query head. `queries` holds heads*head_dim,
 * `cache_k`/`cache_v`/scales point at the (sequence, layer) slot base.
 */
void orc_attention_gqa(int format, const float* queries, const void* cache_k,
                       const void* cache_v, const float* k_scales,
                       const float* v_scales, int heads, int kv_heads,
                       int head_dim, int span, int threads, float* out);

/* Chunk arithmetic of qwen2.cpp:1394-1402. Writes chunk_size, returns the
 * actual chunk count. */
int orc_gqa_chunks(int span, int kv_heads, int threads, int* chunk_size);

/*
 * Query-block prefill of one head — scalar restatement of
 * attention_avx2.cpp:660-864 (attention_block_head_avx2): pass 1 scores for
 * every visible key, softmax per query over span = start+token+1 with
 * normalisation, pass 2 P*V skipping zero weights. F32 and F16 only.
 * queries/out are tokens x query_stride; K/V are flat rows of kv_stride
 * starting at the slot base; kv_head_offset selects the head's columns.
 * `scores` must hold tokens*(start+tokens) floats.
 */
int orc_attention_block_head(int format, const float* queries,
                             const void* keys, const void* values, int tokens,
                             int start_position, int head_dim, int kv_stride,
                             int kv_head_offset, int query_stride, int head,
                             float scale, float* scores, float* out);

/* apply_rope over `heads` vectors of head_dim (NeoX halves: element i pairs
 * with i + head_dim/2), tables of one position (head_dim/2 entries).
 * fma = 1: norm_rope_avx2.cpp:97-131 (l*c - (h*s), l*s + (h*c), one rounding
 * each); fma = 0: norm_rope_scalar.cpp:23-40 (every product and sum rounded). */
void orc_rope_neox(float* values, int heads, int head_dim, const float* cos_t,
                   const float* sin_t, int fma);

/* One token's q/k/v before the store (qwen2.cpp:2062-2071, 1671-1680):
 * q += q_bias, k += k_bias, v += v_bias (each may be NULL), then apply_rope
 * on q (q_heads heads) and k (kv_heads heads). In place. */
void orc_bias_rope_row(float* q, float* k, float* v, const float* q_bias,
                       const float* k_bias, const float* v_bias, int q_heads,
                       int kv_heads, int head_dim, const float* cos_t,
                       const float* sin_t, int fma);

/* build_sparse_index (qwen2.cpp:192-220); `kept` holds >= span entries. */
int orc_sparse_index(int span, int sink, int window, int stride, int* kept);

/* attention_head over the static sparse subset (attention_avx2.cpp:263-490)
 * with the scalar kernel's arithmetic; f32 and f16 (the reference has no i8
 * sparse kernel; the oracle also accepts i8 for the GPU path's extension). */
int orc_attention_head_sparse(int format, const float* query, const void* keys,
                              const void* values, const float* k_scales,
                              const float* v_scales, int kv_stride, int span,
                              int head_dim, float scale, int sink, int window,
                              int stride, float* scores, float* out);

/* qwen2.cpp:608-681 rotary tables ([positions][head_dim/2]); factors NULL
 * means all ones. */
void orc_rope_tables(int head_dim, int positions, float theta, float attn_factor,
                     const float* factors, float* cos_out, float* sin_out);

#ifdef __cplusplus
}
#endif

#endif
