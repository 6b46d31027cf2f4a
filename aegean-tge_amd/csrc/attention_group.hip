// Kernel-level GQA group attention over pages (the reference's
// KernelSet::attention_group slot, include/tge/core/dispatch.hpp:31-33, with
// AttentionGroupArgs, include/tge/cpu/kernels.hpp:262-283): the query heads
// of one KV head attend to positions [first, first + count) of one session,
// read through its block table, and each head's running online-softmax
// state (maximum, sum, accumulators) is written out for the caller's chunk
// merge (merge_gqa_chunks, src/models/qwen2.cpp:1469-1522).
//
// Per position the math is attention_group_scalar's
// (src/cpu/scalar/attention_scalar.cpp:117-199): score = (q . k) * scale in
// fp32; if score > max: alpha = exp(max - score), sum = sum*alpha + 1,
// acc = acc*alpha + v, max = score; else beta = exp(score - max),
// sum += beta, acc += beta*v. K and V are dequantised in fp32 (f16 bits
// exactly; int8 code times its block's scale).
//
// One workgroup per query head, four waves: wave w takes the chunk's pages
// w, w+4, ... (a fixed split), its lanes hold the head's dims (one or two
// each) and the dot product of a position is summed across the wave with
// DPP row operations and row broadcasts. The four waves' states are then
// combined in wave order (the merge rule above), so results are
// reproducible; they differ from the sequential CPU loop by fp32 rounding
// of the sums only.
#include <math.h>

#include "tge_common.h"
#include "tge_kernels.h"

namespace tge {
namespace {

constexpr int kGroupWaves = 4;

// Sum over the 64 lanes of a wave, returned to every lane: quad swaps, the
// half-row and row mirrors (each lane then holds its 16-lane row's sum),
// row broadcasts 15 and 31 (lane 63 holds the total), then lane 63 is read.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xF>(v);  // row_mirror
  v = dpp_add<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
  v = dpp_add<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// f16 bits -> fp32, exact (every half is a float).
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Element (t, d) of a page block's K or V part, dequantised in fp32 (int8:
// code times the scale of its 32-dim block; the block's parts are K, V,
// K scales, V scales back to back).
template <int FMT, bool SF32, int D, bool V>
__device__ __forceinline__ float load_kv(const char* blk, int t, int d) {
  constexpr int NP = D / 32;
  constexpr int ESZ = FMT == kF16 ? 2 : 1;
  const int i = V ? v_index(t, d, ESZ) : k_index(t, d, ESZ);
  const char* part = blk + (V ? 16 * D * ESZ : 0);
  if constexpr (FMT == kF16) {
    return half_bits_to_float(reinterpret_cast<const uint16_t*>(part)[i]);
  } else {
    constexpr int SB = 16 * NP * (SF32 ? 4 : 2);  // bytes of one scale part
    const char* sc = blk + 2 * 16 * D + (V ? SB : 0);
    const int si = scale_index_np(t, d >> 5, NP);
    const float s = SF32 ? reinterpret_cast<const float*>(sc)[si]
                         : half_bits_to_float(reinterpret_cast<const uint16_t*>(sc)[si]);
    return (float)reinterpret_cast<const int8_t*>(part)[i] * s;
  }
}

template <int FMT, bool SF32, int D>
__global__ __launch_bounds__(64 * kGroupWaves) void attention_group_kernel(GroupParams p) {
  constexpr int PER = D / 64;  // dims per lane: d = lane + 64 * e
  __shared__ float sh_m[kGroupWaves], sh_s[kGroupWaves];
  __shared__ float sh_acc[kGroupWaves][D];
  __shared__ int sh_bad;

  const int head = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (threadIdx.x == 0) sh_bad = 0;
  float q[PER], acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int d = lane + 64 * e;  // (dims past the head's own are zeros)
    q[e] = d < p.dims ? p.queries[(size_t)head * p.dims + d] : 0.0f;
    acc[e] = 0.0f;
  }
  float maximum = -INFINITY, sum = 0.0f;
  bool bad = false;
  const int end = p.first + p.count;
  // this wave's pages of the chunk, in order
  for (int pg = (p.first >> 4) + wave; pg * 16 < end; pg += kGroupWaves) {
    const int id = p.page_ids[pg];
    if (id < 0 || id >= p.pages) {  // outside the pool: no read, the outputs become NaN
      bad = true;
      break;
    }
    const char* blk = static_cast<const char*>(p.pool) +
                      ((size_t)id * p.kv_heads + p.kv_head) * p.block_bytes;
    const int t0 = max(p.first - pg * 16, 0), t1 = min(end - pg * 16, 16);
    // every load of the page's positions first, then the math
    float kx[16][PER], vx[16][PER];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        kx[t][e] = load_kv<FMT, SF32, D, false>(blk, t, lane + 64 * e);
        vx[t][e] = load_kv<FMT, SF32, D, true>(blk, t, lane + 64 * e);
      }
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      if (t < t0 || t >= t1) continue;  // wave-uniform
      float prod = 0.0f;
#pragma unroll
      for (int e = 0; e < PER; ++e) prod = fmaf(q[e], kx[t][e], prod);
      const float score = wave_sum(prod) * p.scale;
      if (score > maximum) {
        const float alpha = expf(maximum - score);
        sum = sum * alpha + 1.0f;
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[e] = acc[e] * alpha + vx[t][e];
        maximum = score;
      } else {
        const float beta = expf(score - maximum);
        sum += beta;
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[e] = fmaf(beta, vx[t][e], acc[e]);
      }
    }
  }
  __syncthreads();  // sh_bad is initialised
  if (bad && lane == 0) sh_bad = 1;
  if (lane == 0) {
    sh_m[wave] = maximum;
    sh_s[wave] = sum;
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) sh_acc[wave][lane + 64 * e] = acc[e];
  __syncthreads();
  if (wave != 0) return;
  // combine the waves' states in wave order (merge_gqa_chunks' rule)
  float m = -INFINITY;
#pragma unroll
  for (int w = 0; w < kGroupWaves; ++w)
    if (sh_s[w] > 0.0f) m = fmaxf(m, sh_m[w]);
  float s = 0.0f, a[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) a[e] = 0.0f;
#pragma unroll
  for (int w = 0; w < kGroupWaves; ++w) {
    if (!(sh_s[w] > 0.0f)) continue;
    const float f = expf(sh_m[w] - m);
    s = fmaf(sh_s[w], f, s);
#pragma unroll
    for (int e = 0; e < PER; ++e) a[e] = fmaf(sh_acc[w][lane + 64 * e], f, a[e]);
  }
  const bool fail = sh_bad != 0;
  if (lane == 0) {
    p.maxima[head] = fail ? NAN : m;
    p.sums[head] = fail ? NAN : s;
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int d = lane + 64 * e;
    if (d < p.dims) p.accumulators[(size_t)head * p.dims + d] = fail ? NAN : a[e];
  }
}

}  // namespace

hipError_t launch_attention_group(int format, int scale_f32, int head_dim, const GroupParams& p,
                                  hipStream_t stream) {
  const dim3 grid((unsigned)p.group_heads), block(64 * kGroupWaves);
#define TGE_GRP(F, S, DD) \
  hipLaunchKernelGGL((attention_group_kernel<F, S, DD>), grid, block, 0, stream, p)
  if (format == kF16) {
    if (head_dim == 64) TGE_GRP(kF16, false, 64);
    else if (head_dim == 128) TGE_GRP(kF16, false, 128);
    else if (head_dim == 256) TGE_GRP(kF16, false, 256);
    else return hipErrorInvalidValue;
  } else if (format == kI8) {
    if (head_dim == 64) {
      if (scale_f32) TGE_GRP(kI8, true, 64); else TGE_GRP(kI8, false, 64);
    } else if (head_dim == 128) {
      if (scale_f32) TGE_GRP(kI8, true, 128); else TGE_GRP(kI8, false, 128);
    } else if (head_dim == 256) {
      if (scale_f32) TGE_GRP(kI8, true, 256); else TGE_GRP(kI8, false, 256);
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
#undef TGE_GRP
  return hipGetLastError();
}

}  // namespace tge
