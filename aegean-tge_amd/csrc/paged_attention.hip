// Paged GQA attention on CDNA4 matrix cores: decode (one or a few new tokens
// per session, split-K over long contexts) and chunked prefill (a query tile
// against every prior page) share one workgroup kernel.
//
// Reference semantics (AegeanWorks/Aegean-TGE):
//   per-head oracle      attention_scalar.cpp:48-115
//   GQA group + split-K  attention_scalar.cpp:117-199, qwen2.cpp:1382-1467
//   split merge          qwen2.cpp:1469-1522 (merge_gqa_chunks)
//   block prefill        attention_avx2.cpp:660-864, qwen2.cpp:1524-1571
//   verify (multi-query) qwen2.cpp:2502-2532
// out = softmax(q.K^T / sqrt(D)) V with fp32 accumulation; query i of a
// session sees positions 0 .. ctx+i.
//
// Work unit (one 256-thread workgroup = 4 waves): one session, one KV head,
// up to 16*NRG query rows, a range of logical pages. Rows are (query, head)
// pairs: decode packs the whole GQA group of every new token into the rows
// (so each K/V page is fetched once for the group), prefill packs 16*NRG
// consecutive queries of one head. Wave w takes pages w, w+4, ... of the
// range; each page costs one scalar table load and one contiguous 1 KiB
// (f16) / 512 B (int8) load per operand.
//
// Per page and 16-row group, per wave (lane = group g (0..3), col c (0..15)):
//   S^T[token][row] = K_page (16 x D) . Q^T     v_mfma_f32_16x16x16_f16
//     lane (g, c) ends up holding row c, tokens 4g..4g+3
//   online softmax per row in the log2 domain; the row maximum needs two
//   cross-lane steps (lanes c, c+16, c+32, c+48 share a row)
//   O^T[dim][row] += V^T_page (D x 16) . P^T     v_mfma_f32_16x16x16_f16
//     lane (g, c) holds row c, dims 16j+4g..16j+4g+3: the same row as its
//     softmax state, so rescaling needs no data movement.
// Q is split into f16 hi + lo parts for decode (two MFMAs, ~fp32 accurate);
// int8 K codes are exact in f16, the per-(token, 32-dim) K scale multiplies
// the fp32 partial score of each 32-dim block; int8 V is dequantised to f16
// in registers (code * scale). The 4 waves merge through LDS in a fixed
// order (deterministic output); units of a split context write partial
// (max, sum, acc) for the reduction kernel.
#include <math.h>

#include "tge_common.h"
#include "tge_kernels.h"

namespace tge {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half4_t u2_as_half4(uint32_t a, uint32_t b) {
  union {
    uint32_t u[2];
    half4_t h;
  } x;
  x.u[0] = a;
  x.u[1] = b;
  return x.h;
}

// Four int8 codes (one dword) -> four exact f16 values.
__device__ __forceinline__ half4_t i8x4_to_half4(uint32_t w) {
  half4_t r;
  r[0] = (_Float16)(float)(int)(int8_t)(w & 0xFFu);
  r[1] = (_Float16)(float)(int)(int8_t)((w >> 8) & 0xFFu);
  r[2] = (_Float16)(float)(int)(int8_t)((w >> 16) & 0xFFu);
  r[3] = (_Float16)(float)(int)(int8_t)(w >> 24);
  return r;
}

// Four int8 codes times four per-token scales -> f16.
__device__ __forceinline__ half4_t i8x4_scaled(uint32_t w, const float (&s)[4]) {
  half4_t r;
  r[0] = (_Float16)((float)(int)(int8_t)(w & 0xFFu) * s[0]);
  r[1] = (_Float16)((float)(int)(int8_t)((w >> 8) & 0xFFu) * s[1]);
  r[2] = (_Float16)((float)(int)(int8_t)((w >> 16) & 0xFFu) * s[2]);
  r[3] = (_Float16)((float)(int)(int8_t)(w >> 24) * s[3]);
  return r;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  union {
    uint16_t u;
    _Float16 f;
  } x;
  x.u = (uint16_t)h;
  return (float)x.f;
}

template <bool SF32>
__device__ __forceinline__ void load_scales4(const void* base, size_t off, float (&s)[4]) {
  if (SF32) {
    const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    s[0] = f.x;
    s[1] = f.y;
    s[2] = f.z;
    s[3] = f.w;
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
    s[0] = half_bits_to_float(u.x & 0xFFFFu);
    s[1] = half_bits_to_float(u.x >> 16);
    s[2] = half_bits_to_float(u.y & 0xFFFFu);
    s[3] = half_bits_to_float(u.y >> 16);
  }
}

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x16f16((a), (b), (c), 0, 0, 0)

template <int FMT, bool SF32, int D, int NRG, bool QSPLIT>
__global__ __launch_bounds__(256) void paged_attention_kernel(AttnParams p) {
  constexpr int NP = D / 32;  // 32-dim pairs (= int8 scale blocks)
  constexpr int NT = D / 16;  // 16-dim tiles
  constexpr int ELEMS = 16 * D;
  constexpr int ROWS = 16 * NRG;
  constexpr int OPAD = D + 4;

  __shared__ float lds_m[kWaves][ROWS];
  __shared__ float lds_l[kWaves][ROWS];
  __shared__ float lds_o[ROWS * OPAD];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;

  const WorkRec w = p.work[blockIdx.x];
  const SessionRec s = p.sessions[w.session];
  const int q_stride = p.q_heads * D;
  const int geff = w.rows_per_query;

  // Per-lane row bookkeeping: query index, visible limit, Q operands.
  int lim[NRG];
  half4_t qhi[NRG][NT];
  half4_t qlo[NRG][NT];
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    if (r < w.rows) {
      const int qi = w.row_begin + r / geff;
      const int head = w.head_base + r % geff;
      lim[rg] = s.ctx + qi;
      const float* qp = p.q + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * grp;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float4 x = *reinterpret_cast<const float4*>(qp + 16 * t);
        half4_t hi;
        hi[0] = (_Float16)x.x;
        hi[1] = (_Float16)x.y;
        hi[2] = (_Float16)x.z;
        hi[3] = (_Float16)x.w;
        qhi[rg][t] = hi;
        if (QSPLIT) {
          half4_t lo;
          lo[0] = (_Float16)(x.x - (float)hi[0]);
          lo[1] = (_Float16)(x.y - (float)hi[1]);
          lo[2] = (_Float16)(x.z - (float)hi[2]);
          lo[3] = (_Float16)(x.w - (float)hi[3]);
          qlo[rg][t] = lo;
        }
      }
    } else {
      lim[rg] = -1;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        qhi[rg][t] = half4_t{0, 0, 0, 0};
        qlo[rg][t] = half4_t{0, 0, 0, 0};
      }
    }
  }

  float m[NRG], l[NRG];
  float4_t o[NRG][NT];
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    m[rg] = -INFINITY;
    l[rg] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) o[rg][t] = float4_t{0, 0, 0, 0};
  }

  const int* table = p.tables + s.table_off;
  const int first_limit = s.ctx + w.row_begin;  // smallest limit of the unit
  const size_t head_block = (size_t)w.kv_head;

  for (int pi = w.page_begin + wave; pi < w.page_end; pi += kWaves) {
    const int page = __builtin_amdgcn_readfirstlane(table[pi]);
    const size_t blk = (size_t)page * p.kv_heads + head_block;
    const int lane_off = ((grp)*16 + col) * 8;  // + pair*512 elements

    // ---- fetch the page's operands ------------------------------------
    uint32_t kw[NP][4], vw[NP][4];
    float ks[NP][4], vs[NP][4];
    if (FMT == kF16) {
      const uint16_t* kb = static_cast<const uint16_t*>(p.kpool) + blk * ELEMS + lane_off;
      const uint16_t* vb = static_cast<const uint16_t*>(p.vpool) + blk * ELEMS + lane_off;
#pragma unroll
      for (int pp = 0; pp < NP; ++pp) {
        const uint4 a = *reinterpret_cast<const uint4*>(kb + pp * 512);
        const uint4 b = *reinterpret_cast<const uint4*>(vb + pp * 512);
        kw[pp][0] = a.x; kw[pp][1] = a.y; kw[pp][2] = a.z; kw[pp][3] = a.w;
        vw[pp][0] = b.x; vw[pp][1] = b.y; vw[pp][2] = b.z; vw[pp][3] = b.w;
      }
    } else {
      const int8_t* kb = static_cast<const int8_t*>(p.kpool) + blk * ELEMS + lane_off;
      const int8_t* vb = static_cast<const int8_t*>(p.vpool) + blk * ELEMS + lane_off;
      const size_t sb = blk * (size_t)(16 * NP) + 4 * grp;
#pragma unroll
      for (int pp = 0; pp < NP; ++pp) {
        const uint2 a = *reinterpret_cast<const uint2*>(kb + pp * 512);
        const uint2 b = *reinterpret_cast<const uint2*>(vb + pp * 512);
        kw[pp][0] = a.x; kw[pp][1] = a.y;
        vw[pp][0] = b.x; vw[pp][1] = b.y;
        load_scales4<SF32>(p.kscale, sb + pp * 16, ks[pp]);
        load_scales4<SF32>(p.vscale, sb + pp * 16, vs[pp]);
      }
    }

    // ---- operands as f16 ----------------------------------------------
    half4_t ka[NT], va[NT];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      if (FMT == kF16) {
        ka[2 * pp] = u2_as_half4(kw[pp][0], kw[pp][1]);
        ka[2 * pp + 1] = u2_as_half4(kw[pp][2], kw[pp][3]);
        va[2 * pp] = u2_as_half4(vw[pp][0], vw[pp][1]);
        va[2 * pp + 1] = u2_as_half4(vw[pp][2], vw[pp][3]);
      } else {
        ka[2 * pp] = i8x4_to_half4(kw[pp][0]);
        ka[2 * pp + 1] = i8x4_to_half4(kw[pp][1]);
        va[2 * pp] = i8x4_scaled(vw[pp][0], vs[pp]);
        va[2 * pp + 1] = i8x4_scaled(vw[pp][1], vs[pp]);
      }
    }

    const int pos0 = pi * 16 + 4 * grp;
    const bool need_mask = pi * 16 + 15 > first_limit;

#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      // ---- scores S^T = K Q^T ------------------------------------------
      float4_t sacc = float4_t{0, 0, 0, 0};
      if (FMT == kF16) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          sacc = MFMA16(ka[t], qhi[rg][t], sacc);
          if (QSPLIT) sacc = MFMA16(ka[t], qlo[rg][t], sacc);
        }
      } else {
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) {
          float4_t bacc = float4_t{0, 0, 0, 0};
          bacc = MFMA16(ka[2 * pp], qhi[rg][2 * pp], bacc);
          if (QSPLIT) bacc = MFMA16(ka[2 * pp], qlo[rg][2 * pp], bacc);
          bacc = MFMA16(ka[2 * pp + 1], qhi[rg][2 * pp + 1], bacc);
          if (QSPLIT) bacc = MFMA16(ka[2 * pp + 1], qlo[rg][2 * pp + 1], bacc);
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[e] += bacc[e] * ks[pp][e];
        }
      }

      // ---- online softmax (log2 domain) ---------------------------------
      float sv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = !need_mask || (pos0 + e <= lim[rg]);
        sv[e] = ok ? sacc[e] * p.scale_log2 : -INFINITY;
      }
      float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(m[rg], mx);
      const bool live = mn != -INFINITY;
      const float alpha = live ? exp2f(m[rg] - mn) : 1.0f;
      float pe[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) pe[e] = live ? exp2f(sv[e] - mn) : 0.0f;
      l[rg] = l[rg] * alpha + ((pe[0] + pe[1]) + (pe[2] + pe[3]));
      m[rg] = mn;
      half4_t pv;
      pv[0] = (_Float16)pe[0];
      pv[1] = (_Float16)pe[1];
      pv[2] = (_Float16)pe[2];
      pv[3] = (_Float16)pe[3];

      // ---- O^T += V^T P^T ------------------------------------------------
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        o[rg][t] *= alpha;
        o[rg][t] = MFMA16(va[t], pv, o[rg][t]);
      }
    }
  }

  // ---- merge the four waves (fixed order) and write --------------------
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    l[rg] += __shfl_xor(l[rg], 16);
    l[rg] += __shfl_xor(l[rg], 32);
    if (grp == 0) {
      lds_m[wave][rg * 16 + col] = m[rg];
      lds_l[wave][rg * 16 + col] = l[rg];
    }
  }
  __syncthreads();
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    float mm = lds_m[0][r];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) mm = fmaxf(mm, lds_m[k][r]);
    const float f = (m[rg] == -INFINITY) ? 0.0f : exp2f(m[rg] - mm);
#pragma unroll
    for (int t = 0; t < NT; ++t) o[rg][t] *= f;
  }
  for (int k = 0; k < kWaves; ++k) {
    if (wave == k) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          float4_t* dst = reinterpret_cast<float4_t*>(&lds_o[(rg * 16 + col) * OPAD + 16 * t + 4 * grp]);
          if (k == 0) {
            *dst = o[rg][t];
          } else {
            *dst += o[rg][t];
          }
        }
      }
    }
    __syncthreads();
  }

  for (int idx = threadIdx.x; idx < w.rows * (D / 4); idx += 256) {
    const int r = idx / (D / 4);
    const int d4 = idx % (D / 4);
    float mm = lds_m[0][r];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) mm = fmaxf(mm, lds_m[k][r]);
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      const float mk = lds_m[k][r];
      if (mk != -INFINITY) sum += lds_l[k][r] * exp2f(mk - mm);
    }
    const float4_t acc = *reinterpret_cast<const float4_t*>(&lds_o[r * OPAD + 4 * d4]);
    if (w.part < 0) {
      const int qi = w.row_begin + r / geff;
      const int head = w.head_base + r % geff;
      float4_t res = float4_t{0, 0, 0, 0};
      if (sum > 0.0f) res = acc * (1.0f / sum);
      *reinterpret_cast<float4_t*>(p.out + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * d4) = res;
    } else {
      *reinterpret_cast<float4_t*>(p.part_o + ((size_t)w.part * p.rows_cap + r) * D + 4 * d4) = acc;
      if (d4 == 0) {
        p.part_ml[((size_t)w.part * p.rows_cap + r) * 2] = mm;
        p.part_ml[((size_t)w.part * p.rows_cap + r) * 2 + 1] = sum;
      }
    }
  }
}

// Merge the partial states of the splits of one unit (merge_gqa_chunks:
// splits with no visible position are skipped, none at all gives zeros).
template <int D>
__global__ __launch_bounds__(256) void split_reduce_kernel(ReduceParams p) {
  const ReduceRec it = p.items[blockIdx.x];
  const SessionRec s = p.sessions[it.session];
  const int q_stride = p.q_heads * D;
  for (int idx = threadIdx.x; idx < it.rows * (D / 4); idx += 256) {
    const int r = idx / (D / 4);
    const int d4 = idx % (D / 4);
    float mm = -INFINITY;
    for (int k = 0; k < it.n_parts; ++k) {
      const float* ml = p.part_ml + ((size_t)(it.first_part + k) * p.rows_cap + r) * 2;
      if (ml[1] > 0.0f) mm = fmaxf(mm, ml[0]);
    }
    float sum = 0.0f;
    float4_t acc = float4_t{0, 0, 0, 0};
    for (int k = 0; k < it.n_parts; ++k) {
      const size_t pr = (size_t)(it.first_part + k) * p.rows_cap + r;
      const float* ml = p.part_ml + pr * 2;
      if (!(ml[1] > 0.0f)) continue;
      const float f = exp2f(ml[0] - mm);
      sum += ml[1] * f;
      acc += *reinterpret_cast<const float4_t*>(p.part_o + pr * D + 4 * d4) * f;
    }
    const int qi = it.row_begin + r / it.rows_per_query;
    const int head = it.head_base + r % it.rows_per_query;
    float4_t res = float4_t{0, 0, 0, 0};
    if (sum > 0.0f) res = acc * (1.0f / sum);
    *reinterpret_cast<float4_t*>(p.out + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * d4) = res;
  }
}

template <int FMT, bool SF32, int D, bool QSPLIT>
hipError_t launch_rg(int row_groups, int n_work, const AttnParams& p, hipStream_t stream) {
  const dim3 grid((unsigned)n_work), block(256);
  switch (row_groups) {
    case 1: hipLaunchKernelGGL((paged_attention_kernel<FMT, SF32, D, 1, QSPLIT>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((paged_attention_kernel<FMT, SF32, D, 2, QSPLIT>), grid, block, 0, stream, p); break;
    case 3: hipLaunchKernelGGL((paged_attention_kernel<FMT, SF32, D, 3, QSPLIT>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((paged_attention_kernel<FMT, SF32, D, 4, QSPLIT>), grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int FMT, bool SF32, bool QSPLIT>
hipError_t launch_d(int head_dim, int row_groups, int n_work, const AttnParams& p, hipStream_t stream) {
  if (head_dim == 64) return launch_rg<FMT, SF32, 64, QSPLIT>(row_groups, n_work, p, stream);
  if (head_dim == 128) return launch_rg<FMT, SF32, 128, QSPLIT>(row_groups, n_work, p, stream);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attention(int format, int scale_f32, int head_dim, int row_groups, bool qsplit,
                            int n_work, const AttnParams& p, hipStream_t stream) {
  if (n_work == 0) return hipSuccess;
  if (format == kF16) {
    return qsplit ? launch_d<kF16, false, true>(head_dim, row_groups, n_work, p, stream)
                  : launch_d<kF16, false, false>(head_dim, row_groups, n_work, p, stream);
  }
  if (!qsplit) return hipErrorInvalidValue;
  return scale_f32 ? launch_d<kI8, true, true>(head_dim, row_groups, n_work, p, stream)
                   : launch_d<kI8, false, true>(head_dim, row_groups, n_work, p, stream);
}

hipError_t launch_reduce(int head_dim, int n_items, const ReduceParams& p, hipStream_t stream) {
  if (n_items == 0) return hipSuccess;
  const dim3 grid((unsigned)n_items), block(256);
  if (head_dim == 64) {
    hipLaunchKernelGGL(split_reduce_kernel<64>, grid, block, 0, stream, p);
  } else if (head_dim == 128) {
    hipLaunchKernelGGL(split_reduce_kernel<128>, grid, block, 0, stream, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tge
