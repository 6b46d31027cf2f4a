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

// Store one lane's 8 values of a 32-value block (dims 32b + 8*quarter ..)
// of K (which = 0) or V row `rr` of KV head h. f16: each lane converts its 8
// values with the reference's float_to_half recipe. int8: the four lanes of
// the block (adjacent, aligned to 4 in the wave) combine their absmax runs
// in order (see FoldRun), then each computes the block's scale and inverse
// exactly as quantize_kv_block does (correctly rounded fp32 division) and
// quantizes its 8 values. Dead lanes (`live` false) take part in the
// shuffles and store nothing.
template <int FMT>
__device__ __forceinline__ void store_lane(const AppendParams& p, const float (&x)[8], const RowRec rr,
                                           int which, int h, int b, int quarter, bool live) {
  const int nb = p.head_dim >> 5;
  char* const blk = static_cast<char*>(p.pool) + ((size_t)rr.page * p.kv_heads + h) * p.geom.block_bytes;
  const int t = rr.slot;
  const int d0 = 32 * b + 8 * quarter;  // first dim of this lane
  // K chunk of (token t, dims d0..d0+3) and (d0+4..d0+7): 4 contiguous
  // elements each (k_index_np is contiguous in d&3).
  const int k0 = k_index_np(t, d0, nb);
  const int k1 = k_index_np(t, d0 + 4, nb);

  if (FMT == kF16) {
    uint16_t hx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) hx[i] = float_to_half_ref(x[i]);
    if (!live) return;
    if (which == 0) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(blk);
      *reinterpret_cast<uint2*>(dst + k0) = make_uint2(hx[0] | ((uint32_t)hx[1] << 16), hx[2] | ((uint32_t)hx[3] << 16));
      *reinterpret_cast<uint2*>(dst + k1) = make_uint2(hx[4] | ((uint32_t)hx[5] << 16), hx[6] | ((uint32_t)hx[7] << 16));
    } else {
      uint16_t* dst = reinterpret_cast<uint16_t*>(blk + p.geom.v_off());
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[v_index_np(t, d0 + i, nb)] = hx[i];
    }
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
    uint32_t packed[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float scaled = __fmul_rn(x[i], inverse);
      const float rounded = scaled >= 0.0f ? __fadd_rn(scaled, 0.5f) : __fadd_rn(scaled, -0.5f);
      int c = trunc_to_int_x86(rounded);
      c = c > 127 ? 127 : (c < -127 ? -127 : c);
      packed[i >> 2] |= (uint32_t)(uint8_t)(int8_t)c << (8 * (i & 3));
    }
    if (!live) return;
    if (which == 0) {
      int8_t* dst = reinterpret_cast<int8_t*>(blk);
      *reinterpret_cast<uint32_t*>(dst + k0) = packed[0];
      *reinterpret_cast<uint32_t*>(dst + k1) = packed[1];
    } else {
      int8_t* dst = reinterpret_cast<int8_t*>(blk + p.geom.v_off());
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[v_index_np(t, d0 + i, nb)] = (int8_t)(packed[i >> 2] >> (8 * (i & 3)));
    }
    if (quarter == 0) {
      char* sp = blk + (which ? p.geom.vs_off() : p.geom.ks_off());
      if (p.scale_f32) {
        reinterpret_cast<float*>(sp)[scale_index_np(t, b, nb)] = scale;
      } else {
        reinterpret_cast<uint16_t*>(sp)[scale_index_np(t, b, nb)] = float_to_half_ref(scale);
      }
    }
  }
}

__device__ __forceinline__ void load8(float (&x)[8], const float* src) {
  const float4 f0 = reinterpret_cast<const float4*>(src)[0];
  const float4 f1 = reinterpret_cast<const float4*>(src)[1];
  x[0] = f0.x; x[1] = f0.y; x[2] = f0.z; x[3] = f0.w;
  x[4] = f1.x; x[5] = f1.y; x[6] = f1.z; x[7] = f1.w;
}

}  // namespace
}  // namespace tge
