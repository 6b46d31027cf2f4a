// The append's per-lane store, shared by the append kernels and the fused
// small-step kernel so every path writes the same bits: four adjacent lanes
// own one 32-value block of one K or V row of one KV head. Every arithmetic
// step is an explicit round-to-nearest intrinsic, so the result does not
// depend on the translation unit's contraction setting.
#pragma once

#include "tge_common.h"
#include "tge_kernels.h"

namespace tge {
namespace {

// One lane's 8 values of a 32-value block (dims 32b + 8*quarter ..) of a K
// or V row in stored form: f16, 8 halves (w[0..3], pairs low first); int8,
// 8 codes (w[0..1], bytes in dim order) and the block's scale.
struct LaneCodes {
  uint32_t w[4];
  float scale;
};

// Encode one lane's 8 values. f16: each value with the reference's
// float_to_half recipe. int8: the four lanes of the block (adjacent,
// aligned to 4 in the wave) combine their absmax runs in order (see
// FoldRun), then each computes the block's scale and inverse exactly as
// quantize_kv_block does (correctly rounded fp32 division) and quantizes
// its 8 values. Every lane of the wave takes part (the shuffles); lanes
// whose values are not stored still compute.
template <int FMT>
__device__ __forceinline__ LaneCodes encode_lane(const float (&x)[8]) {
  LaneCodes c{{0, 0, 0, 0}, 0.0f};
  if (FMT == kF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      c.w[i] = float_to_half_ref(x[2 * i]) | ((uint32_t)float_to_half_ref(x[2 * i + 1]) << 16);
  } else {
    // the block's absmax: lane runs joined in lane order
    const FoldRun mine = fold_run(x);
    const int base = (threadIdx.x & 63) & ~3;
    FoldRun all{false, -INFINITY};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const FoldRun o{__shfl(mine.nan ? 1 : 0, base + j) != 0, __shfl(mine.v, base + j)};
      all = j == 0 ? o : fold_join(all, o);
    }
    const float maximum = all.v;
    const float scale = __fdiv_rn(maximum, 127.0f);
    const float inverse = scale != 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float scaled = __fmul_rn(x[i], inverse);
      const float rounded = scaled >= 0.0f ? __fadd_rn(scaled, 0.5f) : __fadd_rn(scaled, -0.5f);
      int q = trunc_to_int_x86(rounded);
      q = q > 127 ? 127 : (q < -127 ? -127 : q);
      c.w[i >> 2] |= (uint32_t)(uint8_t)(int8_t)q << (8 * (i & 3));
    }
    c.scale = scale;
  }
  return c;
}

// Write one lane's encoded values of token slot t into a page block through
// `put` (byte offset in the block, value, bytes: 1, 2, 4 or 8; a write never
// crosses a 16-byte boundary): K, two runs of 4 dims (k_index is
// contiguous in d&3); V, 8 single elements; int8, the block's scale from
// the quarter-0 lane.
template <int FMT, typename Put>
__device__ __forceinline__ void write_lane(Put&& put, const BlockGeom& g, int nb, bool scale_f32,
                                           const LaneCodes& c, int t, int which, int b, int quarter) {
  const int d0 = 32 * b + 8 * quarter;  // first dim of this lane
  constexpr int E = FMT == kF16 ? 2 : 1;  // element bytes
  if (which == 0) {
    const int k0 = k_index(t, d0, E) * E;
    const int k1 = k_index(t, d0 + 4, E) * E;
    if (FMT == kF16) {
      put(k0, (uint64_t)c.w[0] | ((uint64_t)c.w[1] << 32), 8);
      put(k1, (uint64_t)c.w[2] | ((uint64_t)c.w[3] << 32), 8);
    } else {
      put(k0, c.w[0], 4);
      put(k1, c.w[1], 4);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int off = g.v_off() + v_index(t, d0 + i, E) * E;
      if (FMT == kF16)
        put(off, (c.w[i >> 1] >> (16 * (i & 1))) & 0xffffu, 2);
      else
        put(off, (c.w[i >> 2] >> (8 * (i & 3))) & 0xffu, 1);
    }
  }
  if (FMT != kF16 && quarter == 0) {
    const int sp = which ? g.vs_off() : g.ks_off();
    if (scale_f32)
      put(sp + scale_index_np(t, b, nb) * 4, __float_as_uint(c.scale), 4);
    else
      put(sp + scale_index_np(t, b, nb) * 2, float_to_half_ref(c.scale), 2);
  }
}

// Stores to global memory at `blk`.
struct GlobalPut {
  char* blk;
  __device__ __forceinline__ void operator()(int off, uint64_t v, int bytes) const {
    char* d = blk + off;
    if (bytes == 8)
      *reinterpret_cast<uint2*>(d) = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
    else if (bytes == 4)
      *reinterpret_cast<uint32_t*>(d) = (uint32_t)v;
    else if (bytes == 2)
      *reinterpret_cast<uint16_t*>(d) = (uint16_t)v;
    else
      *reinterpret_cast<uint8_t*>(d) = (uint8_t)v;
  }
};

// Store one lane's 8 values of a 32-value block (dims 32b + 8*quarter ..)
// of K (which = 0) or V row `rr` of KV head h (encode_lane, then
// write_lane to the pool). Dead lanes (`live` false) take part in the
// shuffles and store nothing.
template <int FMT>
__device__ __forceinline__ void store_lane(const AppendParams& p, const float (&x)[8], const RowRec rr,
                                           int which, int h, int b, int quarter, bool live) {
  const LaneCodes c = encode_lane<FMT>(x);
  if (!live) return;
  char* const blk = static_cast<char*>(p.pool) + ((size_t)rr.page * p.kv_heads + h) * p.geom.block_bytes;
  write_lane<FMT>(GlobalPut{blk}, p.geom, p.head_dim >> 5, p.scale_f32 != 0, c, rr.slot, which, b, quarter);
}

__device__ __forceinline__ void load8(float (&x)[8], const float* src) {
  const float4 f0 = reinterpret_cast<const float4*>(src)[0];
  const float4 f1 = reinterpret_cast<const float4*>(src)[1];
  x[0] = f0.x; x[1] = f0.y; x[2] = f0.z; x[3] = f0.w;
  x[4] = f1.x; x[5] = f1.y; x[6] = f1.z; x[7] = f1.w;
}

// Dims d0 .. d0 + 7 of one head's row (d0 a multiple of 8): the dims from
// `dims` on read as zeros and are never loaded. Head sizes are multiples
// of 4, so each run of 4 lies wholly inside or outside the head. (Callers
// keep a single 8-value load for heads that are multiples of 8.)
__device__ __forceinline__ void load8_head(float (&x)[8], const float* head_row, int d0, int dims) {
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  const float4 f0 = d0 < dims ? *reinterpret_cast<const float4*>(head_row + d0) : z;
  const float4 f1 = d0 + 4 < dims ? *reinterpret_cast<const float4*>(head_row + d0 + 4) : z;
  x[0] = f0.x; x[1] = f0.y; x[2] = f0.z; x[3] = f0.w;
  x[4] = f1.x; x[5] = f1.y; x[6] = f1.z; x[7] = f1.w;
}

}  // namespace
}  // namespace tge
