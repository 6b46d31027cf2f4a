/*
 * CPU oracle for the paged-KV hot path — TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract, the pinning status of each function and the
 * build flags. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library.
 */
#include "oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof u);
  return u;
}

static float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, sizeof x);
  return x;
}

/* kernels.hpp:325-354. Exact: every half value is a float value. Subnormal
 * halves are m * 2^-24, which ldexpf represents exactly. */
float orc_half_to_float(uint16_t value) {
  const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
  const uint32_t e = (value >> 10) & 0x1Fu;
  const uint32_t m = value & 0x3FFu;
  if (e == 0x1Fu) return bits_f32(sign | 0x7F800000u | (m << 13));
  if (e != 0) return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
  const float mag = ldexpf((float)m, -24);
  return sign ? -mag : mag;
}

/* kernels.hpp:358-386. The rounding adds the first dropped bit (the guard
 * bit) to the truncated result, so an exact tie rounds away from zero and
 * the sticky bits are ignored; a carry out of the mantissa lands in the
 * exponent field, which is also how 65520 becomes infinity. */
uint16_t orc_float_to_half(float value) {
  const uint32_t u = f32_bits(value);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t biased = (u >> 23) & 0xFFu;
  const uint32_t frac = u & 0x7FFFFFu;
  if (biased == 0xFFu) {
    /* inf keeps 0x7C00; any NaN payload collapses to the quiet bit. */
    return (uint16_t)(sign | 0x7C00u | (frac ? 0x200u : 0u));
  }
  const int exp2 = (int)biased - 127;
  if (exp2 < -24) return (uint16_t)sign; /* includes float subnormals/zero */
  if (exp2 > 15) return (uint16_t)(sign | 0x7C00u);
  if (exp2 < -14) {
    /* half subnormal: significand 1.frac shifted right by 13 + (-14 - e). */
    const uint32_t sig = 0x800000u | frac;
    const uint32_t drop = (uint32_t)(-14 - exp2) + 13u;
    const uint32_t kept = sig >> drop;
    const uint32_t guard = (sig >> (drop - 1u)) & 1u;
    return (uint16_t)(sign | (kept + guard));
  }
  const uint32_t kept = ((uint32_t)(exp2 + 15) << 10) | (frac >> 13);
  const uint32_t guard = (frac >> 12) & 1u;
  return (uint16_t)(sign | (kept + guard));
}

void orc_float_to_half_n(const float* src, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_float_to_half(src[i]);
}

void orc_half_to_float_n(const uint16_t* src, float* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_half_to_float(src[i]);
}

/* static_cast<int>(float) as x86-64 executes it (cvttss2si): truncation,
 * and the "integer indefinite" INT_MIN for NaN and out-of-range values. The
 * reference never feeds such values for finite KV, but the GPU kernel follows
 * the same rule so the two agree on every input. */
static int trunc_to_int_x86(float r) {
  if (!(r > -2147483904.0f && r < 2147483648.0f)) return INT_MIN;
  return (int)r;
}

/* qwen2.cpp:88-104. Sequential ternary fold for the absmax: a later equal
 * value replaces the running maximum, so an all-(+-0) block keeps the sign
 * of element 31. fp32 division for scale and inverse, then a separate fp32
 * multiply and add (never fused) before truncation. */
float orc_quantize_kv_block(const float* source, int8_t* destination) {
  float maximum = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float a = source[i] >= 0.0f ? source[i] : -source[i];
    if (!(maximum > a)) maximum = a;
  }
  const float scale = maximum / 127.0f;
  const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float scaled = source[i] * inverse;
    const float rounded = scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f;
    int code = trunc_to_int_x86(rounded);
    if (code > 127) code = 127;
    if (code < -127) code = -127;
    destination[i] = (int8_t)code;
  }
  return scale;
}

void orc_quantize_rows(const float* src, int rows, int kv_dim, int8_t* codes,
                       float* scales) {
  const int blocks = kv_dim / 32;
  for (int r = 0; r < rows; ++r) {
    for (int b = 0; b < blocks; ++b) {
      const size_t off = (size_t)r * kv_dim + (size_t)b * 32;
      scales[(size_t)r * blocks + b] =
          orc_quantize_kv_block(src + off, codes + off);
    }
  }
}

/* qwen2.hpp:112-119 */
size_t orc_kv_layer_offset(int sequence, int layer, int block_count,
                           int context, int kv_dim) {
  return ((size_t)sequence * (size_t)block_count + (size_t)layer) *
         (size_t)context * (size_t)kv_dim;
}

/* qwen2.cpp:2073-2093 and its twins; i8 is store_kv_q8, qwen2.cpp:109-120. */
void orc_store_token(int format, const float* k, const float* v, int kv_dim,
                     size_t slot, void* k_cache, void* v_cache,
                     float* k_scales, float* v_scales) {
  if (format == ORC_KV_F16) {
    uint16_t* ko = (uint16_t*)k_cache + slot;
    uint16_t* vo = (uint16_t*)v_cache + slot;
    for (int i = 0; i < kv_dim; ++i) {
      ko[i] = orc_float_to_half(k[i]);
      vo[i] = orc_float_to_half(v[i]);
    }
  } else if (format == ORC_KV_I8) {
    int8_t* ko = (int8_t*)k_cache;
    int8_t* vo = (int8_t*)v_cache;
    const size_t scale_slot = slot / 32;
    for (int b = 0; b < kv_dim / 32; ++b) {
      k_scales[scale_slot + b] = orc_quantize_kv_block(k + b * 32, ko + slot + b * 32);
      v_scales[scale_slot + b] = orc_quantize_kv_block(v + b * 32, vo + slot + b * 32);
    }
  } else {
    memcpy((float*)k_cache + slot, k, sizeof(float) * (size_t)kv_dim);
    memcpy((float*)v_cache + slot, v, sizeof(float) * (size_t)kv_dim);
  }
}

/* Dequantised element (row, index) of a head slice, as the reference reads
 * it inside its loops (attention_scalar.cpp:66-78). */
static float load_elem(int format, const void* base, const float* scales,
                       int kv_stride, int token, int index) {
  const size_t row = (size_t)token * (size_t)kv_stride;
  if (format == ORC_KV_I8) {
    const size_t block = (size_t)token * (size_t)(kv_stride / 32) + (size_t)(index / 32);
    return (float)((const int8_t*)base)[row + index] * scales[block];
  }
  if (format == ORC_KV_F16)
    return orc_half_to_float(((const uint16_t*)base)[row + index]);
  return ((const float*)base)[row + index];
}

static int check_head_args(int format, const float* query, const void* keys,
                           const void* values, const float* k_scales,
                           const float* v_scales, int kv_stride, int span,
                           int head_dim, const void* scores, const float* out) {
  /* attention_scalar.cpp:11-44 */
  if (head_dim <= 0 || span <= 0) return -1;
  if (kv_stride < head_dim) return -1;
  if (!query || !scores || !out || !keys || !values) return -1;
  if (format == ORC_KV_I8) {
    if (head_dim % 32 || kv_stride % 32) return -1;
    if (!k_scales || !v_scales) return -1;
  }
  return 0;
}

/* attention_scalar.cpp:48-115 */
int orc_attention_head(int format, const float* query, const void* keys,
                       const void* values, const float* k_scales,
                       const float* v_scales, int kv_stride, int span,
                       int head_dim, float scale, float* scores, float* out) {
  if (check_head_args(format, query, keys, values, k_scales, v_scales,
                      kv_stride, span, head_dim, scores, out))
    return -1;
  float maximum = -INFINITY;
  for (int t = 0; t < span; ++t) {
    float product = 0.0f;
    for (int d = 0; d < head_dim; ++d) {
      const float term = query[d] * load_elem(format, keys, k_scales, kv_stride, t, d);
      product += term;
    }
    const float scaled = product * scale;
    scores[t] = scaled;
    maximum = (maximum < scaled) ? scaled : maximum; /* std::max */
  }
  float total = 0.0f;
  for (int t = 0; t < span; ++t) {
    const float e = expf(scores[t] - maximum);
    scores[t] = e;
    total += e;
  }
  const float inverse = 1.0f / total;
  for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
  for (int t = 0; t < span; ++t) {
    const float weight = scores[t] * inverse;
    for (int d = 0; d < head_dim; ++d) {
      const float term = weight * load_elem(format, values, v_scales, kv_stride, t, d);
      out[d] += term;
    }
  }
  return 0;
}

int orc_attention_head_f64(int format, const float* query, const void* keys,
                           const void* values, const float* k_scales,
                           const float* v_scales, int kv_stride, int span,
                           int head_dim, double scale, double* out) {
  if (check_head_args(format, query, keys, values, k_scales, v_scales,
                      kv_stride, span, head_dim, out, (const float*)out))
    return -1;
  double* s = (double*)malloc(sizeof(double) * (size_t)span);
  if (!s) return -1;
  double maximum = -INFINITY;
  for (int t = 0; t < span; ++t) {
    double p = 0.0;
    for (int d = 0; d < head_dim; ++d)
      p += (double)query[d] *
           (double)load_elem(format, keys, k_scales, kv_stride, t, d);
    s[t] = p * scale;
    if (s[t] > maximum) maximum = s[t];
  }
  double total = 0.0;
  for (int t = 0; t < span; ++t) {
    s[t] = exp(s[t] - maximum);
    total += s[t];
  }
  for (int d = 0; d < head_dim; ++d) out[d] = 0.0;
  for (int t = 0; t < span; ++t) {
    const double w = s[t] / total;
    for (int d = 0; d < head_dim; ++d)
      out[d] += w * (double)load_elem(format, values, v_scales, kv_stride, t, d);
  }
  free(s);
  return 0;
}

/* attention_scalar.cpp:117-199 */
void orc_attention_group(int format, const float* queries, const void* keys,
                         const void* values, const float* k_scales,
                         const float* v_scales, int kv_stride, int count,
                         int head_dim, int group_heads, float scale,
                         float* maxima, float* sums, float* accumulators) {
  for (int h = 0; h < group_heads; ++h) {
    const float* q = queries + (size_t)h * head_dim;
    float* acc = accumulators + (size_t)h * head_dim;
    float maximum = -INFINITY;
    float sum = 0.0f;
    for (int d = 0; d < head_dim; ++d) acc[d] = 0.0f;
    for (int t = 0; t < count; ++t) {
      float product = 0.0f;
      for (int d = 0; d < head_dim; ++d) {
        const float term = q[d] * load_elem(format, keys, k_scales, kv_stride, t, d);
        product += term;
      }
      const float score = product * scale;
      if (score > maximum) {
        const float alpha = expf(maximum - score);
        sum = sum * alpha + 1.0f;
        for (int d = 0; d < head_dim; ++d) {
          const float scaled_acc = acc[d] * alpha;
          acc[d] = scaled_acc +
                   load_elem(format, values, v_scales, kv_stride, t, d);
        }
        maximum = score;
      } else {
        const float beta = expf(score - maximum);
        sum += beta;
        for (int d = 0; d < head_dim; ++d) {
          const float term = beta * load_elem(format, values, v_scales, kv_stride, t, d);
          acc[d] += term;
        }
      }
    }
    maxima[h] = maximum;
    sums[h] = sum;
  }
}

/* qwen2.cpp:1469-1522 */
void orc_merge_chunks(const float* maxima, const float* sums,
                      const float* accumulators, size_t base, int chunks,
                      int group, int group_head, int head_dim, float* out) {
  float* red = (float*)calloc((size_t)head_dim, sizeof(float));
  int have = 0;
  float maximum = -INFINITY, sum = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    const size_t st = base + (size_t)c * (size_t)group + (size_t)group_head;
    const float cm = maxima[st];
    const float cs = sums[st];
    if (!(cs > 0.0f)) continue;
    const float* ca = accumulators + st * (size_t)head_dim;
    if (!have) {
      maximum = cm;
      sum = cs;
      memcpy(red, ca, sizeof(float) * (size_t)head_dim);
      have = 1;
      continue;
    }
    const float mm = maximum > cm ? maximum : cm;
    const float alpha = expf(maximum - mm);
    const float beta = expf(cm - mm);
    const float s0 = sum * alpha;
    const float s1 = cs * beta;
    sum = s0 + s1;
    for (int d = 0; d < head_dim; ++d) {
      const float a0 = red[d] * alpha;
      const float a1 = ca[d] * beta;
      red[d] = a0 + a1;
    }
    maximum = mm;
  }
  if (have && sum > 0.0f) {
    const float inv = 1.0f / sum;
    for (int d = 0; d < head_dim; ++d) out[d] = red[d] * inv;
  } else {
    for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
  }
  free(red);
}

/* qwen2.cpp:1394-1402 */
int orc_gqa_chunks(int span, int kv_heads, int threads, int* chunk_size) {
  const int max_chunks = 16; /* kMaxGqaChunks, qwen2.cpp:76 */
  int base = (threads * 2 + kv_heads - 1) / kv_heads;
  if (base < 1) base = 1;
  if (base > max_chunks) base = max_chunks;
  int chunks = base;
  if (span >= 1024) {
    chunks = base < 4 ? 4 : base;
    if (chunks > max_chunks) chunks = max_chunks;
  }
  const int size = (span + chunks - 1) / chunks;
  *chunk_size = size;
  return (span + size - 1) / size;
}

static const void* advance(int format, const void* p, size_t elems) {
  if (format == ORC_KV_I8) return (const int8_t*)p + elems;
  if (format == ORC_KV_F16) return (const uint16_t*)p + elems;
  return (const float*)p + elems;
}

/* qwen2.cpp:1382-1467 run sequentially. */
void orc_attention_gqa(int format, const float* queries, const void* cache_k,
                       const void* cache_v, const float* k_scales,
                       const float* v_scales, int heads, int kv_heads,
                       int head_dim, int span, int threads, float* out) {
  const int group = heads / kv_heads;
  const int kv_dim = kv_heads * head_dim;
  int chunk_size = 0;
  const int chunks = orc_gqa_chunks(span, kv_heads, threads, &chunk_size);
  const size_t states = (size_t)kv_heads * (size_t)chunks * (size_t)group;
  float* mx = (float*)malloc(sizeof(float) * states);
  float* sm = (float*)malloc(sizeof(float) * states);
  float* ac = (float*)malloc(sizeof(float) * states * (size_t)head_dim);
  const float scale = 1.0f / sqrtf((float)head_dim);
  for (int task = 0; task < kv_heads * chunks; ++task) {
    const int h = task / chunks, c = task % chunks;
    const int start = c * chunk_size;
    const int count = (span - start) < chunk_size ? (span - start) : chunk_size;
    const size_t st = ((size_t)h * chunks + c) * group;
    const size_t off = (size_t)h * head_dim + (size_t)start * kv_dim;
    orc_attention_group(format, queries + (size_t)h * group * head_dim,
                        advance(format, cache_k, off),
                        advance(format, cache_v, off),
                        k_scales ? k_scales + off / 32 : NULL,
                        v_scales ? v_scales + off / 32 : NULL, kv_dim, count,
                        head_dim, group, scale, mx + st, sm + st,
                        ac + st * head_dim);
  }
  for (int head = 0; head < heads; ++head) {
    const int h = head / group, g = head % group;
    orc_merge_chunks(mx, sm, ac, (size_t)h * chunks * group, chunks, group, g,
                     head_dim, out + (size_t)head * head_dim);
  }
  free(mx);
  free(sm);
  free(ac);
}

/* attention_avx2.cpp:660-864, scalar, with expf in place of the vector exp. */
int orc_attention_block_head(int format, const float* queries,
                             const void* keys, const void* values, int tokens,
                             int start_position, int head_dim, int kv_stride,
                             int kv_head_offset, int query_stride, int head,
                             float scale, float* scores, float* out) {
  if (!queries || !scores || !out || tokens <= 0 || head_dim <= 0 || head < 0 ||
      format == ORC_KV_I8)
    return -1;
  const int last_key = start_position + tokens - 1;
  const int width = last_key + 1;
  const size_t head_off = (size_t)head * (size_t)head_dim;
  const void* kb = advance(format, keys, (size_t)kv_head_offset);
  const void* vb = advance(format, values, (size_t)kv_head_offset);
  for (int key = 0; key <= last_key; ++key) {
    int first = key - start_position;
    if (first < 0) first = 0;
    for (int t = first; t < tokens; ++t) {
      const float* q = queries + (size_t)t * query_stride + head_off;
      float s = 0.0f;
      for (int d = 0; d < head_dim; ++d) {
        const float term = q[d] * load_elem(format, kb, NULL, kv_stride, key, d);
        s += term;
      }
      scores[(size_t)t * width + key] = s * scale;
    }
  }
  for (int t = 0; t < tokens; ++t) {
    float* row = scores + (size_t)t * width;
    const int span = start_position + t + 1;
    float maximum = -INFINITY;
    for (int i = 0; i < span; ++i) maximum = maximum < row[i] ? row[i] : maximum;
    float total = 0.0f;
    for (int i = 0; i < span; ++i) {
      row[i] = expf(row[i] - maximum);
      total += row[i];
    }
    const float inv = 1.0f / total;
    for (int i = 0; i < span; ++i) row[i] *= inv;
  }
  for (int t = 0; t < tokens; ++t) {
    float* o = out + (size_t)t * query_stride + head_off;
    for (int d = 0; d < head_dim; ++d) o[d] = 0.0f;
    const int span = start_position + t + 1;
    for (int key = 0; key < span; ++key) {
      const float w = scores[(size_t)t * width + key];
      if (w == 0.0f) continue;
      for (int d = 0; d < head_dim; ++d) {
        const float term = w * load_elem(format, vb, NULL, kv_stride, key, d);
        o[d] += term;
      }
    }
  }
  return 0;
}

/* norm_rope_avx2.cpp:97-131 / norm_rope_scalar.cpp:23-40 */
void orc_rope_neox(float* values, int heads, int head_dim, const float* cos_t,
                   const float* sin_t, int fma) {
  const int half = head_dim / 2;
  for (int h = 0; h < heads; ++h) {
    float* v = values + (size_t)h * head_dim;
    for (int i = 0; i < half; ++i) {
      const float l = v[i], hi = v[i + half], c = cos_t[i], s = sin_t[i];
      if (fma) {
        const float hs = hi * s, hc = hi * c;
        v[i] = fmaf(l, c, -hs);
        v[i + half] = fmaf(l, s, hc);
      } else {
        const float lc = l * c, hs = hi * s, ls = l * s, hc = hi * c;
        v[i] = lc - hs;
        v[i + half] = ls + hc;
      }
    }
  }
}

/* qwen2.cpp:2062-2071 (forward), 1671-1680 (forward_batch),
 * 2290-2300 (prefill_run) */
void orc_bias_rope_row(float* q, float* k, float* v, const float* q_bias,
                       const float* k_bias, const float* v_bias, int q_heads,
                       int kv_heads, int head_dim, const float* cos_t,
                       const float* sin_t, int fma) {
  const int dim = q_heads * head_dim, kv_dim = kv_heads * head_dim;
  if (q && q_bias)
    for (int i = 0; i < dim; ++i) q[i] += q_bias[i];
  for (int i = 0; i < kv_dim; ++i) {
    if (k_bias) k[i] += k_bias[i];
    if (v_bias) v[i] += v_bias[i];
  }
  if (q) orc_rope_neox(q, q_heads, head_dim, cos_t, sin_t, fma);
  orc_rope_neox(k, kv_heads, head_dim, cos_t, sin_t, fma);
}

/* qwen2.cpp:608-681 (the YaRN factor set, when given, divides the
 * frequencies; attn_factor scales every entry) */
void orc_rope_tables(int head_dim, int positions, float theta, float attn_factor,
                     const float* factors, float* cos_out, float* sin_out) {
  const int half = head_dim / 2;
  for (int pos = 0; pos < positions; ++pos) {
    for (int i = 0; i < half; ++i) {
      float f = powf(theta, -2.0f * (float)i / (float)head_dim);
      if (factors) f /= factors[i];
      const float angle = (float)pos * f;
      cos_out[(size_t)pos * half + i] = cosf(angle) * attn_factor;
      sin_out[(size_t)pos * half + i] = sinf(angle) * attn_factor;
    }
  }
}

/* build_sparse_index (qwen2.cpp:192-220): ascending kept positions of a
 * span; dense (0..span-1) when the span fits sink + window. Returns the
 * count; `kept` holds at least span entries. */
int orc_sparse_index(int span, int sink, int window, int stride, int* kept) {
  int n = 0;
  if (span <= 0) return 0;
  if (span <= sink + window) {
    for (int p = 0; p < span; ++p) kept[n++] = p;
    return n;
  }
  if (stride < 2) stride = 2;
  const int sink_end = sink < span ? sink : span;
  for (int p = 0; p < sink_end; ++p) kept[n++] = p;
  const int window_start = span - window;
  for (int p = sink_end; p < window_start; p += stride) kept[n++] = p;
  for (int p = window_start > sink_end ? window_start : sink_end; p < span; ++p) kept[n++] = p;
  return n;
}

/* attention_head over the kept positions only: the static sparse kernels
 * (attention_head_static_sparse_avx2 / _fp16_avx2, attention_avx2.cpp:263-490)
 * restated with attention_head_scalar's arithmetic (std::exp, in-order
 * sums); the kept set as above. */
int orc_attention_head_sparse(int format, const float* query, const void* keys,
                              const void* values, const float* k_scales,
                              const float* v_scales, int kv_stride, int span,
                              int head_dim, float scale, int sink, int window,
                              int stride, float* scores, float* out) {
  if (check_head_args(format, query, keys, values, k_scales, v_scales,
                      kv_stride, span, head_dim, scores, out))
    return -1;
  int* kept = (int*)malloc(sizeof(int) * (size_t)span);
  if (!kept) return -1;
  const int n = orc_sparse_index(span, sink, window, stride, kept);
  float maximum = -INFINITY;
  for (int i = 0; i < n; ++i) {
    float product = 0.0f;
    for (int d = 0; d < head_dim; ++d) {
      const float term = query[d] * load_elem(format, keys, k_scales, kv_stride, kept[i], d);
      product += term;
    }
    const float scaled = product * scale;
    scores[i] = scaled;
    maximum = (maximum < scaled) ? scaled : maximum;
  }
  float total = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float e = expf(scores[i] - maximum);
    scores[i] = e;
    total += e;
  }
  const float inverse = 1.0f / total;
  for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float weight = scores[i] * inverse;
    for (int d = 0; d < head_dim; ++d) {
      const float term = weight * load_elem(format, values, v_scales, kv_stride, kept[i], d);
      out[d] += term;
    }
  }
  free(kept);
  return 0;
}
