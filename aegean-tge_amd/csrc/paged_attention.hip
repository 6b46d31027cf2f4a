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
// (each K/V page is fetched once for the group), prefill packs 16*NRG
// consecutive queries of one head. Wave w takes pages w, w+4, ... of the
// range. Each lane owns one contiguous chunk of every page block (see the
// layout in tge_common.h) and fetches it with 16-byte loads; the next page
// is fetched while the current one is consumed, and page ids come in
// batches of 64 (one per lane, then readlane). The Q^T operands (f16 hi +
// lo) sit in LDS, so the accumulators, the two page register sets and the
// softmax state fit the architectural VGPRs at two waves per SIMD.
//
// Per page, per 16-row group, per wave (lane = group g 0..3, column c 0..15):
//   S^T[token][row] = K (16 x D) . Q^T: one v_mfma_f32_16x16x32_f16 per 32-dim
//     block (two with Q split into f16 hi + lo for fp32-grade scores);
//     int8 codes are exact in f16 and the block's per-token scale multiplies
//     the block's fp32 partial score. Lane (g, c) then holds row c,
//     tokens 4g..4g+3.
//   online softmax per row in the log2 domain; the reference maximum only
//     moves when a score exceeds it by more than 2^8, so the accumulators
//     are rescaled rarely (weights stay <= 256, exact enough in f16).
//   O^T[dim][row] += V^T (D x 16) . P^T: v_mfma_f32_16x16x16_f16 per 16-dim
//     tile; lane (g, c) holds row c, dims 16j+4g..+3, the same row as its
//     softmax state. int8 V is dequantised in f16 (exact code times the f16
//     scale, one rounding).
// The 4 waves merge through LDS in a fixed order (deterministic output);
// units of a split context write partial (max, sum, acc) for the reduction
// kernel.
#include <math.h>

#include "tge_common.h"
#include "tge_kernels.h"

namespace tge {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLazyMax = 8.0f;  // log2 of the largest tolerated weight

template <typename T, typename F>
__device__ __forceinline__ T bitcast(F x) {
  static_assert(sizeof(T) == sizeof(F), "size");
  T y;
  __builtin_memcpy(&y, &x, sizeof(T));
  return y;
}

__device__ __forceinline__ half4_t as_half4(uint32_t a, uint32_t b) {
  return bitcast<half4_t>(make_uint2(a, b));
}

// Four signed int8 codes (one dword) -> four exact f16 values: bias the
// bytes to unsigned, splice them under the f16 exponent of 1024 (0x64xx =
// 1024 + byte), and subtract 1152 with packed f16 arithmetic.
__device__ __forceinline__ half4_t i8x4_to_half4(uint32_t w) {
  const uint32_t x = w ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(x, 0x64646464u, 0x00050004u);
  const uint32_t hi = __builtin_amdgcn_perm(x, 0x64646464u, 0x00070006u);
  const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const half2_t a = bitcast<half2_t>(lo) - bias;
  const half2_t b = bitcast<half2_t>(hi) - bias;
  return half4_t{a[0], a[1], b[0], b[1]};
}

// Registers of one page block as fetched by one lane.
template <int FMT, bool SF32, int D>
struct PageRegs {
  static constexpr int NP = D / 32;
  static constexpr int KW = FMT == kF16 ? 4 * NP : 2 * NP;             // dwords of K (=V)
  static constexpr int SW = FMT == kF16 ? 0 : (SF32 ? 4 * NP : 2 * NP);  // dwords of scales
  uint32_t k[KW];
  uint32_t v[KW];
  uint32_t ks[SW > 0 ? SW : 1];
  uint32_t vs[SW > 0 ? SW : 1];
};

// Buffer resources of one layer's K, V and scale arrays. Loads address a
// page block with a wave-uniform byte offset (SGPR) plus the lane's fixed
// chunk offset (VGPR), so fetching a page costs no per-lane address math;
// offsets past the end of an array read zeros instead of faulting.
struct LayerRsrc {
  __amdgpu_buffer_rsrc_t k, v, ks, vs;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int N>
__device__ __forceinline__ void buffer_dwords(uint32_t (&dst)[N], __amdgpu_buffer_rsrc_t r,
                                              int voff, int soff) {
  static_assert(N % 4 == 0, "16-byte loads");
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * i, soff, 0);
    dst[4 * i] = x.x;
    dst[4 * i + 1] = x.y;
    dst[4 * i + 2] = x.z;
    dst[4 * i + 3] = x.w;
  }
}

// Fetch page block `blk` (page * kv_heads + kv_head) into registers.
template <int FMT, bool SF32, int D>
__device__ __forceinline__ void load_page(PageRegs<FMT, SF32, D>& r, const LayerRsrc& rs, int blk,
                                          int chunk, int grp) {
  using R = PageRegs<FMT, SF32, D>;
  const int kv_bytes = R::KW * 4 * 64;
  buffer_dwords(r.k, rs.k, chunk * R::KW * 4, blk * kv_bytes);
  buffer_dwords(r.v, rs.v, chunk * R::KW * 4, blk * kv_bytes);
  if constexpr (FMT == kI8) {
    const int sc_bytes = R::SW * 4 * 4;
    buffer_dwords(r.ks, rs.ks, grp * R::SW * 4, blk * sc_bytes);
    buffer_dwords(r.vs, rs.vs, grp * R::SW * 4, blk * sc_bytes);
  }
}

// K operand (16x16x32 A) of 32-dim block pp.
template <int FMT, bool SF32, int D>
__device__ __forceinline__ half8_t k_operand(const PageRegs<FMT, SF32, D>& r, int pp) {
  if (FMT == kF16) {
    return bitcast<half8_t>(make_uint4(r.k[4 * pp], r.k[4 * pp + 1], r.k[4 * pp + 2], r.k[4 * pp + 3]));
  } else {
    const half4_t a = i8x4_to_half4(r.k[2 * pp]);
    const half4_t b = i8x4_to_half4(r.k[2 * pp + 1]);
    return half8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
}

// Per-token scales (4 tokens of the lane's group) of 32-dim block b.
template <bool SF32>
__device__ __forceinline__ float4_t scales4(const uint32_t* s, int b) {
  if (SF32) {
    return float4_t{__uint_as_float(s[4 * b]), __uint_as_float(s[4 * b + 1]),
                    __uint_as_float(s[4 * b + 2]), __uint_as_float(s[4 * b + 3])};
  } else {
    const half4_t h = as_half4(s[2 * b], s[2 * b + 1]);
    return float4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
}

#define MFMA16x16x16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x16f16((a), (b), (c), 0, 0, 0)
#define MFMA16x16x32(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

template <int FMT, bool SF32, int D, int NRG, bool QSPLIT>
struct Unit {
  static constexpr int NP = D / 32;
  static constexpr int NT = D / 16;
  using Regs = PageRegs<FMT, SF32, D>;

  // Q^T operands in LDS: [rg][pp][hi/lo][lane] half8, one ds_read_b128 each
  const half8_t* qs;
  int lane;
  int lim[NRG];
  // Online softmax state per row, log2 domain. Scores are kept relative to
  // `base`; the weights exp2(s - base) never exceed 2^kLazyMax because base
  // moves (rarely) whenever a score passes base + kLazyMax. `thr` is that
  // threshold, -inf while the row has seen no visible position.
  float base[NRG], thr[NRG];
  float4_t l4[NRG];  // row sums (all four entries equal), via the ones MFMA
  float4_t o[NRG][NT];

  __device__ __forceinline__ half8_t qop(int rg, int pp, int part) const {
    return qs[((rg * NP + pp) * 2 + part) * 64 + lane];
  }

  // One page: scores relative to base, online softmax, value accumulation.
  // `masked` pages hold positions beyond the unit's smallest visible limit.
  __device__ __forceinline__ void consume(const Regs& r, int pi, int grp, bool masked) {
    float4_t sacc[NRG];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) sacc[rg] = float4_t{-base[rg], -base[rg], -base[rg], -base[rg]};
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      const half8_t ka = k_operand<FMT, SF32, D>(r, pp);
      if (FMT == kF16) {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
          sacc[rg] = MFMA16x16x32(ka, qop(rg, pp, 0), sacc[rg]);
          if (QSPLIT) sacc[rg] = MFMA16x16x32(ka, qop(rg, pp, 1), sacc[rg]);
        }
      } else {
        const float4_t ks = scales4<SF32>(r.ks, pp);
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
          float4_t b = MFMA16x16x32(ka, qop(rg, pp, 0), (float4_t{0, 0, 0, 0}));
          if (QSPLIT) b = MFMA16x16x32(ka, qop(rg, pp, 1), b);
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[rg][e] = fmaf(b[e], ks[e], sacc[rg][e]);
        }
      }
    }

    half4_t pw[NRG];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      if (masked) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (pi * 16 + 4 * grp + e > lim[rg]) sacc[rg][e] = -INFINITY;
        }
      }
      const float lmax = fmaxf(fmaxf(sacc[rg][0], sacc[rg][1]), fmaxf(sacc[rg][2], sacc[rg][3]));
      if (__builtin_expect(__any(lmax > thr[rg]), 0)) {
        // rare: some row passed its threshold; move that row's base
        float rmax = fmaxf(lmax, __shfl_xor(lmax, 16));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 32));
        const bool grow = rmax > thr[rg];
        const float delta = grow ? rmax : 0.0f;
        const float alpha = (grow && thr[rg] != -INFINITY) ? __builtin_amdgcn_exp2f(-rmax) : 1.0f;
        base[rg] += delta;
        thr[rg] = grow ? kLazyMax : thr[rg];
#pragma unroll
        for (int e = 0; e < 4; ++e) sacc[rg][e] -= delta;
        l4[rg] *= alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t) o[rg][t] *= alpha;
      }
      pw[rg] = half4_t{(_Float16)__builtin_amdgcn_exp2f(sacc[rg][0]),
                       (_Float16)__builtin_amdgcn_exp2f(sacc[rg][1]),
                       (_Float16)__builtin_amdgcn_exp2f(sacc[rg][2]),
                       (_Float16)__builtin_amdgcn_exp2f(sacc[rg][3])};
      const half4_t ones = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
      l4[rg] = MFMA16x16x16(ones, pw[rg], l4[rg]);
    }

#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      half4_t va[2];
      if (FMT == kF16) {
        va[0] = as_half4(r.v[4 * pp], r.v[4 * pp + 1]);
        va[1] = as_half4(r.v[4 * pp + 2], r.v[4 * pp + 3]);
      } else if (SF32) {
        const float4_t s = scales4<SF32>(r.vs, pp);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const half4_t c = i8x4_to_half4(r.v[2 * pp + h]);
          va[h] = half4_t{(_Float16)((float)c[0] * s[0]), (_Float16)((float)c[1] * s[1]),
                          (_Float16)((float)c[2] * s[2]), (_Float16)((float)c[3] * s[3])};
        }
      } else {
        // exact codes times the f16 scales: one packed multiply, one rounding
        const half4_t s = as_half4(r.vs[2 * pp], r.vs[2 * pp + 1]);
        va[0] = i8x4_to_half4(r.v[2 * pp]) * s;
        va[1] = i8x4_to_half4(r.v[2 * pp + 1]) * s;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) o[rg][2 * pp + h] = MFMA16x16x16(va[h], pw[rg], o[rg][2 * pp + h]);
      }
    }
  }
};

template <int FMT, bool SF32, int D, int NRG, bool QSPLIT, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void paged_attention_kernel(AttnParams p) {
  using U = Unit<FMT, SF32, D, NRG, QSPLIT>;
  using Regs = typename U::Regs;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;
  constexpr int ROWS = 16 * NRG;
  constexpr int OPAD = D + 4;

  __shared__ float lds_m[kWaves][ROWS];
  __shared__ float lds_l[kWaves][ROWS];
  __shared__ float lds_o[ROWS * OPAD];
  __shared__ half8_t lds_q[NRG * NP * 2 * 64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int chunk = grp * 16 + col;

  const WorkRec w = p.work[blockIdx.x];
  const SessionRec s = p.sessions[w.session];
  const int q_stride = p.q_heads * D;
  const int geff = w.rows_per_query;

  U u;
  u.lane = lane;
  u.qs = lds_q;
  // Q^T operands: lane (g, c) of row group rg holds row c, dims
  // {32pp+4g+e, 32pp+16+4g+e} (the K operand's dim order), pre-multiplied by
  // log2(e)/sqrt(D) and split into f16 hi + lo.
  for (int slot = threadIdx.x; slot < NRG * NP * 64; slot += 256) {
    const int ln = slot & 63, pp = (slot >> 6) % NP, rg = (slot >> 6) / NP;
    const int r = rg * 16 + (ln & 15), g = ln >> 4;
    const bool valid = r < w.rows;
    const int qi = w.row_begin + (valid ? r / geff : 0);
    const int head = w.head_base + (valid ? r % geff : 0);
    const float* qp = p.q + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * g + 32 * pp;
    float4 a = make_float4(0, 0, 0, 0), b = make_float4(0, 0, 0, 0);
    if (valid) {
      a = *reinterpret_cast<const float4*>(qp);
      b = *reinterpret_cast<const float4*>(qp + 16);
    }
    const float c = p.scale_log2;
    const float x[8] = {a.x * c, a.y * c, a.z * c, a.w * c, b.x * c, b.y * c, b.z * c, b.w * c};
    half8_t hi, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      hi[j] = (_Float16)x[j];
      lo[j] = QSPLIT ? (_Float16)(x[j] - (float)hi[j]) : (_Float16)0.0f;
    }
    lds_q[((rg * NP + pp) * 2 + 0) * 64 + ln] = hi;
    lds_q[((rg * NP + pp) * 2 + 1) * 64 + ln] = lo;
  }
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    u.lim[rg] = r < w.rows ? s.ctx + w.row_begin + r / geff : -1;
    u.base[rg] = 0.0f;
    u.thr[rg] = -INFINITY;
    u.l4[rg] = float4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] = float4_t{0, 0, 0, 0};
  }
  __syncthreads();

  LayerRsrc rs;
  rs.k = make_rsrc(p.kpool, p.kv_array_bytes);
  rs.v = make_rsrc(p.vpool, p.kv_array_bytes);
  if constexpr (FMT == kI8) {
    rs.ks = make_rsrc(p.kscale, p.scale_array_bytes);
    rs.vs = make_rsrc(p.vscale, p.scale_array_bytes);
  } else {
    rs.ks = rs.k;
    rs.vs = rs.v;
  }

  // This wave's pages j = 0 .. mine-1 are pages page_begin + wave + 4j; the
  // first `clean` of them hold no position any row of the unit may not see.
  const int* table = p.tables + s.table_off;
  const int first_limit = s.ctx + w.row_begin;  // smallest visible limit of the unit
  const int mine = w.page_begin + wave < w.page_end
                       ? (w.page_end - w.page_begin - wave + kWaves - 1) / kWaves
                       : 0;
  const int unmasked_pages = (first_limit + 1) / 16;  // pi*16+15 <= first_limit
  int clean = 0;
  if (unmasked_pages > w.page_begin + wave) {
    clean = (unmasked_pages - w.page_begin - wave + kWaves - 1) / kWaves;
    clean = clean < mine ? clean : mine;
  }
  if (mine > 0) {
    // Page id of this wave's j-th page lives in lane j % 64 of `ids`.
    auto fetch_ids = [&](int j0) {
      const int j = j0 + lane;
      return j < mine ? table[w.page_begin + wave + kWaves * j] : 0;
    };
    auto block_of = [&](int ids_reg, int j) {
      return __builtin_amdgcn_readlane(ids_reg, j & 63) * p.kv_heads + w.kv_head;
    };
    int ids = fetch_ids(0);
    // Two register sets in turn: page j+1 is in flight while page j is used.
    Regs ra, rb;
    load_page<FMT, SF32, D>(ra, rs, block_of(ids, 0), chunk, grp);
    for (int j = 0; j < mine; j += 2) {
      if (j + 1 < mine) {
        if (((j + 1) & 63) == 0) ids = fetch_ids(j + 1);
        load_page<FMT, SF32, D>(rb, rs, block_of(ids, j + 1), chunk, grp);
      }
      u.consume(ra, w.page_begin + wave + kWaves * j, grp, j >= clean);
      if (j + 1 < mine) {
        if (j + 2 < mine) {
          if (((j + 2) & 63) == 0) ids = fetch_ids(j + 2);
          load_page<FMT, SF32, D>(ra, rs, block_of(ids, j + 2), chunk, grp);
        }
        u.consume(rb, w.page_begin + wave + kWaves * (j + 1), grp, j + 1 >= clean);
      }
    }
  }

  // ---- merge the four waves (fixed order) and write --------------------
  // Each wave's state for a row is (base, l, o): o and l are sums of
  // exp2(s - base). Rows that saw no visible position have thr = -inf.
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    if (grp == 0) {
      lds_m[wave][rg * 16 + col] = u.thr[rg] == -INFINITY ? -INFINITY : u.base[rg];
      lds_l[wave][rg * 16 + col] = u.l4[rg][0];
    }
  }
  __syncthreads();
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    float mm = lds_m[0][r];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) mm = fmaxf(mm, lds_m[k][r]);
    const float mine_m = lds_m[wave][r];
    const float f = (mine_m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mine_m - mm);
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] *= f;
  }
  for (int k = 0; k < kWaves; ++k) {
    if (wave == k) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          float4_t* dst = reinterpret_cast<float4_t*>(&lds_o[(rg * 16 + col) * OPAD + 16 * t + 4 * grp]);
          if (k == 0) {
            *dst = u.o[rg][t];
          } else {
            *dst += u.o[rg][t];
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
      if (mk != -INFINITY) sum += lds_l[k][r] * __builtin_amdgcn_exp2f(mk - mm);
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
// One thread per (row, 4 dims), blockIdx.y selecting a 256-slot slice of
// the item's rows; the split states are read in batches of 8 independent
// loads.
template <int D>
__global__ __launch_bounds__(256) void split_reduce_kernel(ReduceParams p) {
  const ReduceRec it = p.items[blockIdx.x];
  const SessionRec s = p.sessions[it.session];
  const int q_stride = p.q_heads * D;
  {
    const int idx = blockIdx.y * 256 + threadIdx.x;
    if (idx >= it.rows * (D / 4)) return;
    const int r = idx / (D / 4);
    const int d4 = idx % (D / 4);
    const float2* ml = reinterpret_cast<const float2*>(p.part_ml) + (size_t)it.first_part * p.rows_cap + r;
    const float* po = p.part_o + ((size_t)it.first_part * p.rows_cap + r) * D + 4 * d4;
    const size_t stride_ml = p.rows_cap;
    const size_t stride_o = (size_t)p.rows_cap * D;
    float mm = -INFINITY;
    for (int k = 0; k < it.n_parts; ++k) {
      const float2 x = ml[k * stride_ml];
      if (x.y > 0.0f) mm = fmaxf(mm, x.x);
    }
    float sum = 0.0f;
    float4_t acc = float4_t{0, 0, 0, 0};
    for (int k0 = 0; k0 < it.n_parts; k0 += 8) {
      float4_t v[8];
      float f[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const bool ok = k0 + k < it.n_parts;
        const float2 x = ok ? ml[(k0 + k) * stride_ml] : make_float2(0.0f, 0.0f);
        f[k] = x.y > 0.0f ? __builtin_amdgcn_exp2f(x.x - mm) : 0.0f;
        sum += x.y * f[k];
        v[k] = ok ? *reinterpret_cast<const float4_t*>(po + (k0 + k) * stride_o) : float4_t{0, 0, 0, 0};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) acc += v[k] * f[k];
    }
    const int qi = it.row_begin + r / it.rows_per_query;
    const int head = it.head_base + r % it.rows_per_query;
    float4_t res = float4_t{0, 0, 0, 0};
    if (sum > 0.0f) res = acc * (1.0f / sum);
    *reinterpret_cast<float4_t*>(p.out + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * d4) = res;
  }
}

// Waves per SIMD each variant is compiled for: the register budget that keeps
// every live value in the 256 architectural VGPRs (no AGPR round trips on
// the accumulators) while leaving room for a second wave to hide latency.
template <int FMT, int D, int NRG, bool QSPLIT>
constexpr int waves_per_eu() {
  return D == 64 ? (NRG <= 2 ? 3 : 2) : (NRG <= 2 ? 2 : 1);
}

template <int FMT, bool SF32, int D, bool QSPLIT>
hipError_t launch_rg(int row_groups, int n_work, const AttnParams& p, hipStream_t stream) {
  const dim3 grid((unsigned)n_work), block(256);
  switch (row_groups) {
#define TGE_RG(n)                                                                          \
  case n:                                                                                  \
    hipLaunchKernelGGL((paged_attention_kernel<FMT, SF32, D, n, QSPLIT, waves_per_eu<FMT, D, n, QSPLIT>()>), \
                       grid, block, 0, stream, p);                                         \
    break;
    TGE_RG(1)
    TGE_RG(2)
    TGE_RG(3)
    TGE_RG(4)
#undef TGE_RG
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
  const dim3 grid((unsigned)n_items, (unsigned)((p.rows_cap * head_dim / 4 + 255) / 256)), block(256);
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
