// C entry points over the reference engine's own hot-path code, compiled from
// /root/reference where it lies (oracle/Makefile, target `ref`) into
// oracle/_ref/libtge_ref.so — TEST INFRASTRUCTURE ONLY (checker and CPU
// baseline; never part of the product).
//
// Reference sources linked in: src/cpu/scalar/attention_scalar.cpp,
// src/cpu/avx2/attention_avx2.cpp, src/cpu/scalar/norm_rope_scalar.cpp,
// src/cpu/avx2/norm_rope_avx2.cpp. Header-only reference code used here:
// include/tge/cpu/kernels.hpp (float_to_half/half_to_float, arg structs),
// include/tge/models/block_table.hpp, include/tge/models/kv_block_layout.hpp.
// Exceptions never cross this boundary: they become negative return codes.
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "tge/cpu/kernels.hpp"
#include "tge/models/block_table.hpp"
#include "tge/models/kv_block_layout.hpp"

namespace {

enum { kF32 = 0, kF16 = 1, kI8 = 2 };

// Fills the reference's AttentionArgs from one flat description.
tge::cpu::AttentionArgs head_args(int format, const float* query,
                                  const void* keys, const void* values,
                                  const float* k_scales, const float* v_scales,
                                  int kv_stride, int span, int head_dim,
                                  float scale, float* scores, float* out) {
  tge::cpu::AttentionArgs a;
  a.query = query;
  if (format == kF16) {
    a.half = true;
    a.keys_half = static_cast<const std::uint16_t*>(keys);
    a.values_half = static_cast<const std::uint16_t*>(values);
  } else if (format == kI8) {
    a.q8 = true;
    a.keys_q8 = static_cast<const std::int8_t*>(keys);
    a.values_q8 = static_cast<const std::int8_t*>(values);
    a.keys_q8_scales = k_scales;
    a.values_q8_scales = v_scales;
  } else {
    a.keys = static_cast<const float*>(keys);
    a.values = static_cast<const float*>(values);
  }
  a.kv_stride = kv_stride;
  a.span = span;
  a.head_dim = head_dim;
  a.scale = scale;
  a.scores = scores;
  a.out = out;
  return a;
}

tge::cpu::AttentionGroupArgs group_args(int format, const float* queries,
                                        const void* keys, const void* values,
                                        const float* k_scales,
                                        const float* v_scales, int kv_stride,
                                        int count, int head_dim,
                                        int group_heads, float scale,
                                        float* maxima, float* sums,
                                        float* accumulators) {
  tge::cpu::AttentionGroupArgs a;
  a.queries = queries;
  if (format == kF16) {
    a.half = true;
    a.keys_half = static_cast<const std::uint16_t*>(keys);
    a.values_half = static_cast<const std::uint16_t*>(values);
  } else if (format == kI8) {
    a.q8 = true;
    a.keys_q8 = static_cast<const std::int8_t*>(keys);
    a.values_q8 = static_cast<const std::int8_t*>(values);
    a.keys_q8_scales = k_scales;
    a.values_q8_scales = v_scales;
  } else {
    a.keys = static_cast<const float*>(keys);
    a.values = static_cast<const float*>(values);
  }
  a.kv_stride = kv_stride;
  a.count = count;
  a.head_dim = head_dim;
  a.group_heads = group_heads;
  a.scale = scale;
  a.maxima = maxima;
  a.sums = sums;
  a.accumulators = accumulators;
  return a;
}

}  // namespace

extern "C" {

std::uint16_t ref_float_to_half(float x) { return tge::cpu::float_to_half(x); }
float ref_half_to_float(std::uint16_t h) { return tge::cpu::half_to_float(h); }

void ref_float_to_half_n(const float* src, std::uint16_t* dst, std::size_t n) {
  for (std::size_t i = 0; i < n; ++i) dst[i] = tge::cpu::float_to_half(src[i]);
}

int ref_attention_head(int avx2, int format, const float* query,
                       const void* keys, const void* values,
                       const float* k_scales, const float* v_scales,
                       int kv_stride, int span, int head_dim, float scale,
                       float* scores, float* out) {
  const auto a = head_args(format, query, keys, values, k_scales, v_scales,
                           kv_stride, span, head_dim, scale, scores, out);
  try {
    if (avx2) {
      tge::cpu::attention_head_avx2(a);
    } else {
      tge::cpu::attention_head_scalar(a);
    }
  } catch (const std::invalid_argument&) {
    return -1;
  }
  return 0;
}

void ref_attention_group(int avx2, int format, const float* queries,
                         const void* keys, const void* values,
                         const float* k_scales, const float* v_scales,
                         int kv_stride, int count, int head_dim,
                         int group_heads, float scale, float* maxima,
                         float* sums, float* accumulators) {
  const auto a = group_args(format, queries, keys, values, k_scales, v_scales,
                            kv_stride, count, head_dim, group_heads, scale,
                            maxima, sums, accumulators);
  if (avx2) {
    tge::cpu::attention_group_avx2(a);
  } else {
    tge::cpu::attention_group_scalar(a);
  }
}

// attention_block_head_avx2 for one head. `scores` is this head's slice,
// tokens x score_stride.
void ref_attention_block_head(int format, const float* queries,
                              const void* keys, const void* values, int tokens,
                              int start_position, int head_dim, int kv_stride,
                              int kv_head_offset, int query_stride,
                              int score_stride, int context, float scale,
                              int head, float* scores, float* out) {
  tge::cpu::AttentionBlockArgs a;
  a.queries = queries;
  if (format == kF16) {
    a.half = true;
    a.keys_half = static_cast<const std::uint16_t*>(keys);
    a.values_half = static_cast<const std::uint16_t*>(values);
  } else {
    a.keys = static_cast<const float*>(keys);
    a.values = static_cast<const float*>(values);
  }
  a.tokens = tokens;
  a.start_position = start_position;
  a.head_dim = head_dim;
  a.kv_stride = kv_stride;
  a.kv_head_offset = kv_head_offset;
  a.query_stride = query_stride;
  a.score_stride = score_stride;
  a.context = context;
  a.scale = scale;
  a.scores = scores;
  a.out = out;
  tge::cpu::attention_block_head_avx2(a, head);
}

// ---- BlockTable (block_table.hpp) behind an opaque handle. ----------------

void* ref_bt_create(int blocks, int block_tokens) {
  try {
    return new tge::models::BlockTable(blocks, block_tokens);
  } catch (const std::runtime_error&) {
    return nullptr;
  }
}

void ref_bt_destroy(void* t) { delete static_cast<tge::models::BlockTable*>(t); }

// Each returns >= 0 on success, -1 where the reference throws.
int ref_bt_allocate(void* t) {
  try {
    return static_cast<tge::models::BlockTable*>(t)->allocate();
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_release(void* t, int block) {
  try {
    static_cast<tge::models::BlockTable*>(t)->release(block);
    return 0;
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_share(void* t, int block) {
  try {
    static_cast<tge::models::BlockTable*>(t)->share(block);
    return 0;
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_refcount(void* t, int block) {
  try {
    return static_cast<tge::models::BlockTable*>(t)->refcount(block);
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_free_count(void* t) {
  return static_cast<tge::models::BlockTable*>(t)->free_count();
}

int ref_bt_slot_for(int pos, int block_tokens, int* block, int* offset) {
  try {
    const auto s = tge::models::BlockTable::slot_for(pos, block_tokens);
    *block = s.first;
    *offset = s.second;
    return 0;
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_hash_tokens(const int* tokens, int count, std::uint64_t* out) {
  try {
    *out = tge::models::BlockTable::hash_tokens(tokens, count);
    return 0;
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_remember_prefix(void* t, std::uint64_t hash, int block) {
  try {
    static_cast<tge::models::BlockTable*>(t)->remember_prefix(hash, block);
    return 0;
  } catch (const std::runtime_error&) {
    return -1;
  }
}

int ref_bt_find_prefix(void* t, std::uint64_t hash) {
  return static_cast<tge::models::BlockTable*>(t)->find_prefix(hash);
}

// gather_blocks_row_major over `nblocks` equal-size float blocks stored back
// to back in `pool` (block_elems each). Returns -1 where the reference throws.
int ref_gather_blocks(const float* pool, int nblocks, int block_elems,
                      const int* table, int count, int dim, float* out) {
  std::vector<std::vector<float>> blocks(static_cast<std::size_t>(nblocks));
  for (int b = 0; b < nblocks; ++b) {
    blocks[static_cast<std::size_t>(b)].assign(
        pool + static_cast<std::size_t>(b) * block_elems,
        pool + static_cast<std::size_t>(b + 1) * block_elems);
  }
  try {
    const auto g =
        tge::models::gather_blocks_row_major(blocks, table, count, dim);
    std::memcpy(out, g.data(), g.size() * sizeof(float));
    return static_cast<int>(g.size());
  } catch (const std::runtime_error&) {
    return -1;
  }
}

}  // extern "C"

// apply_rope_avx2 / apply_rope_scalar (norm_rope_*.cpp), in place.
extern "C" void ref_apply_rope(int avx2, float* values, int heads, int head_dim, int position,
                               const float* cos_t, const float* sin_t) {
  if (avx2) {
    tge::cpu::apply_rope_avx2(values, heads, head_dim, position, cos_t, sin_t);
  } else {
    tge::cpu::apply_rope_scalar(values, heads, head_dim, position, cos_t, sin_t);
  }
}

// attention_head_static_sparse_avx2 (f32) / _fp16_avx2 (f16), with the
// stride rule of Qwen2::attention_head (stride < 2 -> 2, qwen2.cpp:1293).
extern "C" int ref_attention_head_sparse(int format, const float* query, const void* keys,
                                         const void* values, int kv_stride, int span,
                                         int head_dim, float scale, int sink, int window,
                                         int stride, float* scores, float* out) {
  try {
    tge::cpu::AttentionArgs a = head_args(format, query, keys, values, nullptr, nullptr,
                                          kv_stride, span, head_dim, scale, scores, out);
    if (format == kF16) {
      tge::cpu::attention_head_static_sparse_fp16_avx2(a, sink, window, stride < 2 ? 2 : stride);
    } else {
      tge::cpu::attention_head_static_sparse_avx2(a, sink, window, stride < 2 ? 2 : stride);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}
