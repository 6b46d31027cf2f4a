// Shared host/device definitions of the gfx950 paged-KV path: page layout,
// plan records, the reference's f32->f16 bit recipe and int8 block quantizer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tge_records.h"

namespace tge {

enum Format { kF16 = 1, kI8 = 2 };

// ---------------------------------------------------------------------------
// Page blocks. One layer's pool is one array of pages*kv_heads page blocks;
// block (page, kv_head) is number page*kv_heads + kv_head, and holds its 16
// tokens' K codes, V codes and (I8) K and V scales back to back, so one
// block is one contiguous run of HBM (I8, D=128, f16 scales: 4352 B):
//   [ K: 16*D elements | V: 16*D elements | K scales: 16*D/32 | V scales ]
// ---------------------------------------------------------------------------
struct BlockGeom {
  int kv_bytes;     // bytes of the K (= V) part
  int scale_bytes;  // bytes of one scale part (0 for F16)
  int block_bytes;  // bytes of a whole block (the block stride)
  __host__ __device__ int v_off() const { return kv_bytes; }
  __host__ __device__ int ks_off() const { return 2 * kv_bytes; }
  __host__ __device__ int vs_off() const { return 2 * kv_bytes + scale_bytes; }
};

// Width of the page blocks for a head size: heads of up to 64 dims are
// stored in 64-dim blocks, up to 128 in 128-dim blocks, up to 256 in
// 256-dim blocks, the dims from head_dim on holding zeros (so scores and
// values are those of the head's own dims). A head size must be a positive
// multiple of 4 (int8: of 32, the quantizer's block) of at most 256; 0 for
// any other. Every kernel reads and writes the head's own dims of q, k, v
// and out in 16-byte runs of 4 that lie wholly inside or outside them (the
// rows stay 16-byte aligned).
__host__ __device__ inline int block_dims_for(int head_dim, int format) {
  if (head_dim <= 0 || head_dim > 256 || head_dim % (format == kI8 ? 32 : 4) != 0) return 0;
  return head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
}

__host__ __device__ inline BlockGeom block_geom(int format, int head_dim, int scale_f32) {
  BlockGeom g;
  g.kv_bytes = 16 * head_dim * (format == kF16 ? 2 : 1);
  g.scale_bytes = format == kF16 ? 0 : 16 * (head_dim / 32) * (scale_f32 ? 4 : 2);
  g.block_bytes = 2 * g.kv_bytes + 2 * g.scale_bytes;
  return g;
}

// ---------------------------------------------------------------------------
// Page layout. One page block = 16 tokens x head_dim (D) of one KV head; NP =
// D/32; E = element bytes (2 f16, 1 int8). The in-block order is the register
// order of the CDNA4 matrix-core operands: each lane of a wave owns NP*8
// elements of each part (D=128: 64 B f16, 32 B int8), cut into 16-byte
// pieces, and piece i of lane l sits at byte i*1024 + l*16 of the part. So
// the wave's 16-byte load i (one per piece) reads one contiguous KiB, whole
// cache lines, and the direct-to-LDS copy of a block is the identity.
//
// A lane's elements, in its own order j = p*8 + h*4 + e (PE = 16/E elements
// per piece; element j lies in piece j/PE at position j%PE):
//  K (A operand of S^T = K.Q^T, row = token t):
//    d -> pair p = d/32, half h = (d/16)&1, group g = (d/4)&3, e = d&3
//    lane (g, t) = g*16 + t holds, per pair p, dims 32p+4g+e and 32p+16+4g+e:
//    the v_mfma_f32_16x16x32_f16 A operand of the 32-dim block p (k = 8g + j).
//  V (A operand of O^T = V^T.P^T, row = dim):
//    tile j = d/16, pair p = j/2, h = j&1, dl = d&15, g = t/4, e = t&3
//    lane (g, dl) = g*16 + dl holds tokens 4g..4g+3 of dims 32p+dl (h=0),
//    32p+16+dl (h=1): the v_mfma_f32_16x16x16_f16 A operand of tile j.
//    index = ((j/PE)*64 + lane)*PE + j%PE for both parts.
//  Scales (I8), one per (token t, 32-dim block b):
//    index = ((t/4)*NP + b)*4 + (t&3)
//    lanes of group g read the 4*NP scales of their four tokens at once.
// ---------------------------------------------------------------------------
__host__ __device__ inline int piece_index(int lane, int j, int esz) {
  const int pe = 16 / esz;  // elements per 16-byte piece
  return ((j / pe) * 64 + lane) * pe + (j % pe);
}
__host__ __device__ inline int k_index(int t, int d, int esz) {
  return piece_index(((d >> 2) & 3) * 16 + t, (d >> 5) * 8 + (((d >> 4) & 1) << 2) + (d & 3), esz);
}
__host__ __device__ inline int v_index(int t, int d, int esz) {
  return piece_index((t >> 2) * 16 + (d & 15), (d >> 5) * 8 + (((d >> 4) & 1) << 2) + (t & 3), esz);
}
__host__ __device__ inline int scale_index_np(int t, int b, int np) {
  return ((t >> 2) * np + b) * 4 + (t & 3);
}

// ---------------------------------------------------------------------------
// Reference conversions, restated (bit-for-bit) for host and device.
// ---------------------------------------------------------------------------
__host__ __device__ inline uint32_t f32_as_u32(float x) {
#ifdef __HIP_DEVICE_COMPILE__
  return __float_as_uint(x);
#else
  uint32_t u;
  __builtin_memcpy(&u, &x, 4);
  return u;
#endif
}

// kernels.hpp:358-386: truncate the mantissa and add the guard bit (first
// dropped bit), so exact ties go away from zero and sticky bits are ignored;
// |x| < 2^-24 flushes to signed zero, overflow gives infinity, NaN gives the
// quiet pattern sign|0x7E00. Pure integer work, identical on every target.
__host__ __device__ inline uint16_t float_to_half_ref(float value) {
  const uint32_t u = f32_as_u32(value);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t biased = (u >> 23) & 0xFFu;
  const uint32_t frac = u & 0x7FFFFFu;
  if (biased == 0xFFu) return (uint16_t)(sign | 0x7C00u | (frac ? 0x200u : 0u));
  const int e = (int)biased - 127;
  if (e < -24) return (uint16_t)sign;
  if (e > 15) return (uint16_t)(sign | 0x7C00u);
  if (e < -14) {
    const uint32_t sig = 0x800000u | frac;
    const uint32_t drop = (uint32_t)(-14 - e) + 13u;
    return (uint16_t)(sign | ((sig >> drop) + ((sig >> (drop - 1u)) & 1u)));
  }
  const uint32_t kept = ((uint32_t)(e + 15) << 10) | (frac >> 13);
  return (uint16_t)(sign | (kept + ((frac >> 12) & 1u)));
}

// static_cast<int>(float) as the reference's x86-64 build executes it
// (cvttss2si): truncation toward zero, INT_MIN for NaN and out-of-range.
__host__ __device__ inline int trunc_to_int_x86(float r) {
  if (!(r > -2147483904.0f && r < 2147483648.0f)) return (int)0x80000000u;
  return (int)r;
}

// qwen2.cpp:88-104 (quantize_kv_block) for 32 values: sequential absmax fold
// in which a later equal value wins (an all-zero block keeps the sign of
// element 31), correctly rounded fp32 division, then a separate multiply and
// add per code (never contracted into an FMA), truncation and clamp.
__host__ __device__ inline float quantize_block_ref(const float* x, int8_t* codes) {
  float maximum = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float a = x[i] >= 0.0f ? x[i] : -x[i];
    if (!(maximum > a)) maximum = a;
  }
#ifdef __HIP_DEVICE_COMPILE__
  const float scale = __fdiv_rn(maximum, 127.0f);
  const float inverse = scale != 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
#else
  const float scale = maximum / 127.0f;
  const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
#endif
  for (int i = 0; i < 32; ++i) {
#ifdef __HIP_DEVICE_COMPILE__
    const float scaled = __fmul_rn(x[i], inverse);
    const float rounded =
        scaled >= 0.0f ? __fadd_rn(scaled, 0.5f) : __fadd_rn(scaled, -0.5f);
#else
    const float scaled = x[i] * inverse;
    const float rounded = scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f;
#endif
    int c = trunc_to_int_x86(rounded);
    c = c > 127 ? 127 : (c < -127 ? -127 : c);
    codes[i] = (int8_t)c;
  }
  return scale;
}

// The reference's absmax fold over a block, `if (!(m > a)) m = a` for
// a = |x| as `x >= 0 ? x : -x` (qwen2.cpp:90-93), split over the 4 lanes that
// hold 8 values each. A lane summarises its run as (nan, v): without a NaN,
// v is the run's fold from -inf (its maximum; the later of equal values, so
// an all-zero run keeps the sign of its last element); with a NaN, the fold
// restarts after the last NaN whatever came before, and v is that restarted
// fold (NaN itself when the run ends with a NaN). Runs combine in order:
// a run with a NaN overrides what precedes it, otherwise the later run wins
// unless the earlier value is strictly greater. Starting the block's fold
// from +0 changes nothing (every a is >= -0 or NaN), so the block's maximum
// is the combined v.
struct FoldRun {
  bool nan;
  float v;
};

__host__ __device__ inline float fold_step(float m, float a) { return (m > a) ? m : a; }

__host__ __device__ inline FoldRun fold_run(const float* x) {
  FoldRun r{false, -__builtin_huge_valf()};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = x[i] >= 0.0f ? x[i] : -x[i];
    if (a != a) {
      r.nan = true;
      r.v = a;  // the state after a NaN is the NaN; the next value replaces it
    } else {
      r.v = fold_step(r.v, a);
    }
  }
  return r;
}

__host__ __device__ inline FoldRun fold_join(FoldRun first, FoldRun then) {
  if (then.nan) return then;
  return FoldRun{first.nan, fold_step(first.v, then.v)};
}

}  // namespace tge
