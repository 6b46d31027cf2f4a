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

// acc / sum per component, correctly rounded: a row with one visible
// position (weight w) yields exactly (w*v)/w = v.
__device__ __forceinline__ float4_t div4(float4_t a, float b) {
  return float4_t{__fdiv_rn(a[0], b), __fdiv_rn(a[1], b), __fdiv_rn(a[2], b), __fdiv_rn(a[3], b)};
}

// 2^e for an integer-valued float e (exact; 0 for very negative e). Every
// row base is an integer, so rescaling a state by the difference of two
// bases is exact and the f16 weights exp2(s - base) round the same way
// whatever base a wave happened to pick: results do not depend on how the
// pages were split between waves beyond fp32 summation order.
__device__ __forceinline__ float pow2i(float e) {
  return __builtin_amdgcn_ldexpf(1.0f, (int)fmaxf(e, -300.0f));
}

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
// chunk offset (VGPR); offsets past the end of an array read zeros instead
// of faulting.
struct LayerRsrc {
  __amdgpu_buffer_rsrc_t k, v;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void global_void_t;
typedef const __attribute__((address_space(4))) int sconst_int;  // scalar (constant) loads

// Per-wave LDS ring of page slots filled by direct-to-LDS loads. A slot
// holds the K and V chunks of every lane (piece i of lane l at
// i*1024 + 16*l, the order the lane reads them back) and, for int8 pools,
// the page block's K and V scales as stored.
template <int FMT, bool SF32, int D>
struct Ring {
  using R = PageRegs<FMT, SF32, D>;
  static constexpr int PIECES = R::KW / 4;                   // 16-byte pieces per lane
  static constexpr int KV_BYTES = PIECES * 1024;             // one operand per slot
  static constexpr int SC_BYTES = FMT == kI8 ? 16 * (D / 32) * (SF32 ? 4 : 2) : 0;
  static constexpr int SC_LOADS = (2 * SC_BYTES + 255) / 256;  // dword loads: K then V scales
  static constexpr int SLOT = 2 * KV_BYTES + 256 * SC_LOADS;
  static constexpr int LOADS = 2 * PIECES + SC_LOADS;        // loads per page
};

// Waves per SIMD each variant is compiled for: the register budget that keeps
// every live value in the 256 architectural VGPRs (no AGPR round trips on
// the accumulators) while leaving room for a second wave to hide latency.
template <int FMT, int D, int NRG, bool QSPLIT>
constexpr int waves_per_eu() {
  return D == 64 ? (NRG <= 2 ? 3 : 2) : (NRG <= 2 ? 2 : 1);
}

// Ring slots per wave: as many as the workgroups resident on a CU (one per
// wave per SIMD) leave room for in the 160 KiB of LDS, between 2 and 4.
// NB slots keep NB-1 pages in flight while the wave consumes one.
template <int FMT, bool SF32, int D, int NRG, bool QSPLIT>
constexpr int ring_slots() {
  constexpr int budget = 160 * 1024 / waves_per_eu<FMT, D, NRG, QSPLIT>();
  constexpr int n = budget / (kWaves * Ring<FMT, SF32, D>::SLOT);
  return n < 2 ? 2 : (n > 4 ? 4 : n);
}

// Issue the direct-to-LDS loads of page block `blk` into `slot`.
template <int FMT, bool SF32, int D>
__device__ __forceinline__ void fetch_page(char* slot, const LayerRsrc& rs, const AttnParams& p,
                                           int blk, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS-load builtins exist for the device pass only
  using RG = Ring<FMT, SF32, D>;
  const int kv_block = RG::KV_BYTES;  // bytes of one K (or V) page block
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.k, (lds_void_t*)(slot + i * 1024), 16,
                                             lane * RG::PIECES * 16 + i * 16, blk * kv_block, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.v, (lds_void_t*)(slot + RG::KV_BYTES + i * 1024), 16,
                                             lane * RG::PIECES * 16 + i * 16, blk * kv_block, 0, 0);
  }
  if constexpr (FMT == kI8) {
    // dword d of the slot's scale area (K scales then V scales)
    char* sdst = slot + 2 * RG::KV_BYTES;
#pragma unroll
    for (int i = 0; i < RG::SC_LOADS; ++i) {
      // dword d of [K scales | V scales]; lanes past the end re-read the
      // first K scale dword into the slot's padding.
      const int d = i * 64 + lane;
      const int per = RG::SC_BYTES / 4;
      const char* kb = static_cast<const char*>(p.kscale) + (size_t)blk * RG::SC_BYTES;
      const char* vb = static_cast<const char*>(p.vscale) + (size_t)blk * RG::SC_BYTES;
      const char* src = d < per ? kb + 4 * d : (d < 2 * per ? vb + 4 * (d - per) : kb);
      __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)(sdst + i * 256), 4, 0, 0);
    }
  }
#endif
}

// Read a landed page back into registers (the lane's own chunk and its
// group's scales).
template <int FMT, bool SF32, int D>
__device__ __forceinline__ void read_page(PageRegs<FMT, SF32, D>& r, const char* slot, int lane,
                                          int grp) {
  using RG = Ring<FMT, SF32, D>;
  using R = PageRegs<FMT, SF32, D>;
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    const u32x4_t k = *reinterpret_cast<const u32x4_t*>(slot + i * 1024 + 16 * lane);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(slot + RG::KV_BYTES + i * 1024 + 16 * lane);
    r.k[4 * i] = k.x; r.k[4 * i + 1] = k.y; r.k[4 * i + 2] = k.z; r.k[4 * i + 3] = k.w;
    r.v[4 * i] = v.x; r.v[4 * i + 1] = v.y; r.v[4 * i + 2] = v.z; r.v[4 * i + 3] = v.w;
  }
  if constexpr (FMT == kI8) {
    const char* sk = slot + 2 * RG::KV_BYTES + grp * R::SW * 4;
    const char* sv = sk + RG::SC_BYTES;
#pragma unroll
    for (int i = 0; i < R::SW / 4; ++i) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(sk + 16 * i);
      const u32x4_t b = *reinterpret_cast<const u32x4_t*>(sv + 16 * i);
      r.ks[4 * i] = a.x; r.ks[4 * i + 1] = a.y; r.ks[4 * i + 2] = a.z; r.ks[4 * i + 3] = a.w;
      r.vs[4 * i] = b.x; r.vs[4 * i + 1] = b.y; r.vs[4 * i + 2] = b.z; r.vs[4 * i + 3] = b.w;
    }
  }
}

// s_waitcnt vmcnt(n) (other counters untouched), n <= 63.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// wait_vmcnt<n * LOADS> for a wave-uniform n in [0, MAXN]: all but this
// wave's n most recently issued pages have landed.
template <int MAXN, int LOADS>
__device__ __forceinline__ void wait_vmcnt_pages(int n) {
  static_assert(MAXN <= 3, "up to three pages in flight");
  if (MAXN >= 3 && n >= 3) {
    wait_vmcnt<(MAXN >= 3 ? 3 : 0) * LOADS>();
  } else if (MAXN >= 2 && n == 2) {
    wait_vmcnt<(MAXN >= 2 ? 2 : 0) * LOADS>();
  } else if (MAXN >= 1 && n == 1) {
    wait_vmcnt<(MAXN >= 1 ? 1 : 0) * LOADS>();
  } else {
    wait_vmcnt<0>();
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

  half8_t qhi[NRG][NP];
  half8_t qlo[NRG][NP];
  int lim[NRG];
  // Online softmax state per row, log2 domain. Scores are kept relative to
  // `base`; the weights exp2(s - base) never exceed 2^kLazyMax because base
  // moves (rarely) whenever a score passes base + kLazyMax. `thr` is that
  // threshold, -inf while the row has seen no visible position.
  float base[NRG], thr[NRG];
  float4_t l4[NRG];  // row sums (all four entries equal), via the ones MFMA
  float4_t o[NRG][NT];

  __device__ __forceinline__ half8_t qop(int rg, int pp, int part) const {
    return part ? qlo[rg][pp] : qhi[rg][pp];
  }

  // One page: scores relative to base, online softmax, value accumulation.
  // `masked` pages hold positions beyond the unit's smallest visible limit.
  __device__ __forceinline__ void consume(const Regs& r, int pi, int grp, bool masked) {
    float4_t sacc[NRG];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) sacc[rg] = float4_t{0, 0, 0, 0};
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
      sacc[rg] -= base[rg];  // exact: base is an integer
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
        const float delta = grow ? ceilf(rmax) : 0.0f;  // integer steps keep base integral
        const float alpha = (grow && thr[rg] != -INFINITY) ? pow2i(-delta) : 1.0f;
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

// Workgroup LDS: the four waves' page rings; after the page loop the same
// bytes hold the merge buffers.
template <int FMT, bool SF32, int D, int NRG, bool QSPLIT>
struct Shared {
  static constexpr int ROWS = 16 * NRG;
  static constexpr int OPAD = D + 4;
  static constexpr int MERGE_BYTES = (2 * kWaves * ROWS + ROWS * OPAD) * 4;
  static constexpr int RING_BYTES =
      kWaves * ring_slots<FMT, SF32, D, NRG, QSPLIT>() * Ring<FMT, SF32, D>::SLOT;
  static constexpr int BYTES = RING_BYTES > MERGE_BYTES ? RING_BYTES : MERGE_BYTES;
  alignas(16) char raw[BYTES];
};

// One work item (unit) by the whole workgroup.
template <int FMT, bool SF32, int D, int NRG, bool QSPLIT>
__device__ __forceinline__ void attend_unit(const AttnParams& p, const WorkRec& w,
                                            Shared<FMT, SF32, D, NRG, QSPLIT>& sh) {
  using U = Unit<FMT, SF32, D, NRG, QSPLIT>;
  using Regs = typename U::Regs;
  using RG = Ring<FMT, SF32, D>;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;
  constexpr int ROWS = 16 * NRG;
  constexpr int OPAD = D + 4;
  constexpr int NB = ring_slots<FMT, SF32, D, NRG, QSPLIT>();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;

  const SessionRec s = p.sessions[w.session];
  const int q_stride = p.q_heads * D;
  const int geff = w.rows_per_query;

  U u;
  // Q^T operands: lane (g, c) of row group rg holds row c, dims
  // {32pp+4g+e, 32pp+16+4g+e} (the K operand's dim order), pre-multiplied by
  // log2(e)/sqrt(D) and split into f16 hi + lo.
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    const bool valid = r < w.rows;
    const int qi = w.row_begin + (valid ? r / geff : 0);
    const int head = w.head_base + (valid ? r % geff : 0);
    const float* qp = p.q + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * grp;
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      float4 a = make_float4(0, 0, 0, 0), b = make_float4(0, 0, 0, 0);
      if (valid) {
        a = *reinterpret_cast<const float4*>(qp + 32 * pp);
        b = *reinterpret_cast<const float4*>(qp + 32 * pp + 16);
      }
      const float c = p.scale_log2;
      const float x[8] = {a.x * c, a.y * c, a.z * c, a.w * c, b.x * c, b.y * c, b.z * c, b.w * c};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const _Float16 hi = (_Float16)x[j];
        u.qhi[rg][pp][j] = hi;
        u.qlo[rg][pp][j] = QSPLIT ? (_Float16)(x[j] - (float)hi) : (_Float16)0.0f;
      }
    }
    u.lim[rg] = valid ? s.ctx + w.row_begin + r / geff : -1;
    u.base[rg] = 0.0f;
    u.thr[rg] = -INFINITY;
    u.l4[rg] = float4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] = float4_t{0, 0, 0, 0};
  }

  LayerRsrc rs;
  rs.k = make_rsrc(p.kpool, p.kv_array_bytes);
  rs.v = make_rsrc(p.vpool, p.kv_array_bytes);

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
  char* ring = sh.raw + wave * NB * RG::SLOT;
  if (mine > 0) {
    // Page ids come through the scalar cache (read-only constant loads), one
    // page ahead of their use, so no vector-memory wait is tied to them.
    const sconst_int* ids = (const sconst_int*)(table + w.page_begin + wave);
    auto block_of = [&](int id) -> int { return id * p.kv_heads + w.kv_head; };
#pragma unroll
    for (int b = 0; b < NB - 1; ++b) {
      if (b < mine) fetch_page<FMT, SF32, D>(ring + b * RG::SLOT, rs, p, block_of(ids[kWaves * b]), lane);
    }
    int id_next = NB - 1 < mine ? ids[kWaves * (NB - 1)] : 0;
    int slot = 0;
    for (int j = 0; j < mine; ++j) {
      const int jn = j + NB - 1;
      if (jn < mine) {
        const int id = id_next;
        id_next = jn + 1 < mine ? ids[kWaves * (jn + 1)] : 0;
        int sn = slot + NB - 1;
        sn = sn >= NB ? sn - NB : sn;
        fetch_page<FMT, SF32, D>(ring + sn * RG::SLOT, rs, p, block_of(id), lane);
        wait_vmcnt<(NB - 1) * RG::LOADS>();  // page j has landed
      } else {
        wait_vmcnt<0>();
      }
      Regs r;
      read_page<FMT, SF32, D>(r, ring + slot * RG::SLOT, lane, grp);
      u.consume(r, w.page_begin + wave + kWaves * j, grp, j >= clean);
      slot = slot + 1 == NB ? 0 : slot + 1;
    }
  }

  float* lds_base = reinterpret_cast<float*>(sh.raw);
  float (*lds_m)[ROWS] = reinterpret_cast<float (*)[ROWS]>(lds_base);
  float (*lds_l)[ROWS] = reinterpret_cast<float (*)[ROWS]>(lds_base + kWaves * ROWS);
  float* lds_o = lds_base + 2 * kWaves * ROWS;
  __syncthreads();  // every wave is done with its ring before it is reused

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
    const float f = (mine_m == -INFINITY) ? 0.0f : pow2i(mine_m - mm);
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
      if (mk != -INFINITY) sum += lds_l[k][r] * pow2i(mk - mm);
    }
    const float4_t acc = *reinterpret_cast<const float4_t*>(&lds_o[r * OPAD + 4 * d4]);
    if (w.part < 0) {
      const int qi = w.row_begin + r / geff;
      const int head = w.head_base + r % geff;
      float4_t res = float4_t{0, 0, 0, 0};
      if (sum > 0.0f) res = div4(acc, sum);
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

// The workgroup runs its work items in turn: items [first[g], first[g+1])
// for workgroup g under a balanced schedule (every workgroup of the launch
// gets the same number of pages), or item g alone when `first` is null.
template <int FMT, bool SF32, int D, int NRG, bool QSPLIT, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void paged_attention_kernel(AttnParams p) {
  __shared__ Shared<FMT, SF32, D, NRG, QSPLIT> sh;
  int it = blockIdx.x, end = blockIdx.x + 1;
  if (p.wg_first) {
    it = p.wg_first[blockIdx.x];
    end = p.wg_first[blockIdx.x + 1];
  }
  for (; it < end; ++it) {
    const WorkRec w = p.work[it];
    attend_unit<FMT, SF32, D, NRG, QSPLIT>(p, w, sh);
    __syncthreads();  // LDS is reused by the next item
  }
}

// ---------------------------------------------------------------------------
// Decode kernel: persistent workgroups of four waves (as many per CU as the
// registers allow), each covering a contiguous share of the plan's page
// sequence (its work items in order).
//
// Within a unit the waves take pages round-robin (wave w: pages w, w+4,
// ...). Each wave streams its pages through a private LDS ring and crosses
// unit boundaries without draining: the next unit's first pages are already
// in flight while the current unit is merged. A unit ends for a wave when
// its next page belongs to a later unit (or the share is exhausted); the
// four waves then merge their states for that unit in wave order, so every
// wave passes the same barriers. The page split is fixed by the plan, so
// results are bit-reproducible.
// ---------------------------------------------------------------------------
template <int FMT, bool SF32, int D, int NRG, int WPE>
struct DecodeShared {
  static constexpr int ROWS = 16 * NRG;
  static constexpr int OPAD = D + 4;
  static constexpr int MERGE_FLOATS = 2 * kWaves * ROWS + ROWS * OPAD;
  static constexpr int SLOT = Ring<FMT, SF32, D>::SLOT;
  // LDS of one of the WPE workgroups that share a CU.
  static constexpr int BUDGET = 160 * 1024 / WPE - 4 * MERGE_FLOATS - 64;
  static constexpr int NB_FIT = BUDGET / (kWaves * SLOT);
  static constexpr int NB = NB_FIT > 4 ? 4 : NB_FIT;
  static_assert(NB >= 2, "the decode ring needs two slots per wave");
  alignas(16) char ring[kWaves * NB * SLOT];
  alignas(16) float merge[MERGE_FLOATS];
};

typedef const __attribute__((address_space(4))) WorkRec sconst_work;

// Workgroup barrier ordering LDS only: this wave's LDS accesses complete,
// then all waves meet. Direct-to-LDS page loads stay in flight across it
// (they fill the wave's own ring, which no other wave reads); the
// __syncthreads fence would wait for them.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A work record read through the scalar cache.
__device__ __forceinline__ WorkRec load_work(const sconst_work* w) {
  const sconst_int* q = (const sconst_int*)w;
  WorkRec r;
  r.session = q[0];
  r.kv_head = q[1];
  r.page_begin = q[2];
  r.page_end = q[3];
  r.part = q[4];
  r.row_begin = q[5];
  r.rows = q[6];
  r.rows_per_query = q[7];
  r.head_base = q[8];
  r.ctx = q[9];
  r.q_row = q[10];
  r.table_off = q[11];
  return r;
}

// Share indices of the pages in a wave's ring, oldest first (a FIFO of at
// most four wave-uniform values kept in scalar registers).
struct PageFifo {
  int t0 = 0, t1 = 0, t2 = 0, t3 = 0;
  __device__ __forceinline__ void push(int n, int g) {  // n = entries before the push
    t0 = n == 0 ? g : t0;
    t1 = n == 1 ? g : t1;
    t2 = n == 2 ? g : t2;
    t3 = n == 3 ? g : t3;
  }
  __device__ __forceinline__ void pop() {
    t0 = t1;
    t1 = t2;
    t2 = t3;
  }
};

template <int FMT, bool SF32, int D, int NRG, bool QSPLIT, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void paged_decode_kernel(AttnParams p) {
  constexpr int W = kWaves;
  using SH = DecodeShared<FMT, SF32, D, NRG, WPE>;
  using U = Unit<FMT, SF32, D, NRG, QSPLIT>;
  using Regs = typename U::Regs;
  using RG = Ring<FMT, SF32, D>;
  constexpr int NB = SH::NB;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;
  constexpr int ROWS = 16 * NRG;
  constexpr int OPAD = D + 4;
  __shared__ SH sh;

  const int first = p.wg_first[blockIdx.x];
  const int last = p.wg_first[blockIdx.x + 1];
  if (first >= last) return;  // the whole workgroup leaves together

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  const sconst_work* work = (const sconst_work*)p.work;
  const int q_stride = p.q_heads * D;

  LayerRsrc rs;
  rs.k = make_rsrc(p.kpool, p.kv_array_bytes);
  rs.v = make_rsrc(p.vpool, p.kv_array_bytes);
  char* ring = sh.ring + wave * NB * RG::SLOT;

  // ---- issue side: this wave's next page, its block, its fetch -------------
  // Cursor over the share's units: unit `ik` covers share pages
  // [ibase, ibase + its page count); `jn` is this wave's next page in it.
  int ik = first, ibase = 0, jn = wave;
  WorkRec iw = load_work(work + first);
  WorkRec iw_next = load_work(work + (first + 1 < last ? first + 1 : first));
  int pend_g = -1, pend_block = 0;  // next page to fetch (share index, block)
  auto request = [&]() __attribute__((always_inline)) -> void {
    bool ok = true;
    while (ok && jn >= iw.page_end - iw.page_begin) {
      if (ik + 1 >= last) {
        ok = false;  // past the share: the cursor stays on its last unit
      } else {
        const int np = iw.page_end - iw.page_begin;
        ibase += np;
        ++ik;
        jn = wave;
        iw = iw_next;
        iw_next = load_work(work + (ik + 1 < last ? ik + 1 : ik));
      }
    }
    // (index 0 when past the share keeps the table read inside the unit)
    const sconst_int* t = (const sconst_int*)(p.tables + iw.table_off + iw.page_begin);
    const int id = t[ok ? jn : 0];
    pend_g = ok ? ibase + jn : -1;
    pend_block = id * p.kv_heads + iw.kv_head;
    jn += W;
  };
  // Fetch the pending page into `slot` and take the next; returns the
  // fetched page's share index, or -1 when the share is exhausted.
  auto issue = [&](int slot) __attribute__((always_inline)) -> int {
    const int g = pend_g;
    if (g >= 0) {
      fetch_page<FMT, SF32, D>(ring + slot * RG::SLOT, rs, p, pend_block, lane);
      request();
    }
    return g;
  };

  // ---- consume side: unit state --------------------------------------------
  int ck = first, cbase = 0;
  WorkRec cw = load_work(work + first);
  U u;
  int unmasked = 0;
  auto reset_unit = [&]() __attribute__((always_inline)) -> void {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const int r = rg * 16 + col;
      u.lim[rg] = r < cw.rows ? cw.ctx + cw.row_begin + r / cw.rows_per_query : -1;
      u.base[rg] = 0.0f;
      u.thr[rg] = -INFINITY;
      u.l4[rg] = float4_t{0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < NT; ++t) u.o[rg][t] = float4_t{0, 0, 0, 0};
    }
    unmasked = (cw.ctx + cw.row_begin + 1) / 16;  // pages with no masked position
  };
  // Q^T operands of the unit (see attend_unit), loaded before its first page.
  auto load_q = [&]() __attribute__((always_inline)) -> void {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const int r = rg * 16 + col;
      const bool valid = r < cw.rows;
      const int qi = cw.row_begin + (valid ? r / cw.rows_per_query : 0);
      const int head = cw.head_base + (valid ? r % cw.rows_per_query : 0);
      const float* qp = p.q + (size_t)(cw.q_row + qi) * q_stride + (size_t)head * D + 4 * grp;
#pragma unroll
      for (int pp = 0; pp < NP; ++pp) {
        float4 a = make_float4(0, 0, 0, 0), b = make_float4(0, 0, 0, 0);
        if (valid) {
          a = *reinterpret_cast<const float4*>(qp + 32 * pp);
          b = *reinterpret_cast<const float4*>(qp + 32 * pp + 16);
        }
        const float c = p.scale_log2;
        const float x[8] = {a.x * c, a.y * c, a.z * c, a.w * c, b.x * c, b.y * c, b.z * c, b.w * c};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const _Float16 hi = (_Float16)x[j];
          u.qhi[rg][pp][j] = hi;
          u.qlo[rg][pp][j] = QSPLIT ? (_Float16)(x[j] - (float)hi) : (_Float16)0.0f;
        }
      }
    }
  };
  // Merge the W waves' states of unit `cw` in wave order and write the
  // output rows (or the unit's partial). Every wave calls this once per unit.
  float* mbase = sh.merge;
  float (*lds_m)[ROWS] = reinterpret_cast<float (*)[ROWS]>(mbase);
  float (*lds_l)[ROWS] = reinterpret_cast<float (*)[ROWS]>(mbase + W * ROWS);
  float* lds_o = mbase + 2 * W * ROWS;
  auto finalize = [&]() __attribute__((always_inline)) -> void {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      if (grp == 0) {
        lds_m[wave][rg * 16 + col] = u.thr[rg] == -INFINITY ? -INFINITY : u.base[rg];
        lds_l[wave][rg * 16 + col] = u.l4[rg][0];
      }
    }
    lds_barrier();
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const int r = rg * 16 + col;
      float mm = lds_m[0][r];
#pragma unroll
      for (int k = 1; k < W; ++k) mm = fmaxf(mm, lds_m[k][r]);
      const float mine_m = lds_m[wave][r];
      const float f = (mine_m == -INFINITY) ? 0.0f : pow2i(mine_m - mm);
#pragma unroll
      for (int t = 0; t < NT; ++t) u.o[rg][t] *= f;
    }
    for (int k = 0; k < W; ++k) {
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
      lds_barrier();
    }
    for (int idx = threadIdx.x; idx < cw.rows * (D / 4); idx += 64 * W) {
      const int r = idx / (D / 4);
      const int d4 = idx % (D / 4);
      float mm = lds_m[0][r];
#pragma unroll
      for (int k = 1; k < W; ++k) mm = fmaxf(mm, lds_m[k][r]);
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const float mk = lds_m[k][r];
        if (mk != -INFINITY) sum += lds_l[k][r] * pow2i(mk - mm);
      }
      const float4_t acc = *reinterpret_cast<const float4_t*>(&lds_o[r * OPAD + 4 * d4]);
      if (cw.part < 0) {
        const int qi = cw.row_begin + r / cw.rows_per_query;
        const int head = cw.head_base + r % cw.rows_per_query;
        float4_t res = float4_t{0, 0, 0, 0};
        if (sum > 0.0f) res = div4(acc, sum);
        *reinterpret_cast<float4_t*>(p.out + (size_t)(cw.q_row + qi) * q_stride + (size_t)head * D + 4 * d4) = res;
      } else {
        *reinterpret_cast<float4_t*>(p.part_o + ((size_t)cw.part * p.rows_cap + r) * D + 4 * d4) = acc;
        if (d4 == 0) {
          p.part_ml[((size_t)cw.part * p.rows_cap + r) * 2] = mm;
          p.part_ml[((size_t)cw.part * p.rows_cap + r) * 2 + 1] = sum;
        }
      }
    }
    lds_barrier();  // the merge area is free for the next unit
  };
  auto next_unit = [&]() __attribute__((always_inline)) -> void {
    cbase += cw.page_end - cw.page_begin;
    ++ck;
    cw = load_work(work + (ck < last ? ck : last - 1));
    reset_unit();
  };
  // Q^T of the unit is loaded when the wave starts it, so the previous
  // unit's Q is dead while that unit is merged.

  // ---- the page loop -----------------------------------------------------------
  reset_unit();
  load_q();
  request();
  PageFifo fifo;
  int head = 0, count = 0;
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) {
    if (count == b) {
      const int g = issue(b);
      if (g >= 0) {
        fifo.push(count, g);
        ++count;
      }
    }
  }
  while (count > 0) {
    int nslot = head + count;
    nslot = nslot >= NB ? nslot - NB : nslot;
    const int gn = issue(nslot);
    if (gn >= 0) {
      fifo.push(count, gn);
      ++count;
      wait_vmcnt<(NB - 1) * RG::LOADS>();  // the ring is full: the oldest page has landed
    } else {
      wait_vmcnt<0>();
    }
    const int g = fifo.t0;
    if (g >= cbase + (cw.page_end - cw.page_begin)) {
      do {
        finalize();
        next_unit();
      } while (g >= cbase + (cw.page_end - cw.page_begin));
      load_q();
    }
    Regs r;
    read_page<FMT, SF32, D>(r, ring + head * RG::SLOT, lane, grp);
    const int pi = cw.page_begin + (g - cbase);
    u.consume(r, pi, grp, pi >= unmasked);
    head = head + 1 == NB ? 0 : head + 1;
    --count;
    fifo.pop();
  }
  // The share is exhausted: close this wave's remaining units.
  while (ck < last) {
    finalize();
    next_unit();
  }
}

// ---------------------------------------------------------------------------
// Block-prefill kernel: one workgroup per (session, KV head, query tile,
// page split). The tile holds up to 128 rows, (query, head) pairs of the KV
// head's query group in query-major order; wave w owns rows [32w, 32w+32).
// The waves share the pages instead of splitting them: each iteration every
// wave fetches one page of a four-page tile into a shared LDS ring, and after
// one barrier all four waves run their own rows against all four pages. Rows
// never meet across waves, so each wave writes its rows (or its split's
// partial) directly.
// ---------------------------------------------------------------------------
template <int FMT, bool SF32, int D, int WPE>
struct PrefillShared {
  static constexpr int SLOT = Ring<FMT, SF32, D>::SLOT;
  static constexpr int TILE = kWaves * SLOT;  // four pages
  static constexpr int NB_FIT = (160 * 1024 / WPE - 64) / TILE;
  static constexpr int NB = NB_FIT > 4 ? 4 : NB_FIT;
  static_assert(NB >= 2, "the prefill ring needs two tiles");
  alignas(16) char ring[NB * TILE];
};

template <int FMT, bool SF32, int D, bool QSPLIT, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void paged_prefill_kernel(AttnParams p) {
  constexpr int NRG = 2;  // 32 rows per wave
  using SH = PrefillShared<FMT, SF32, D, WPE>;
  using U = Unit<FMT, SF32, D, NRG, QSPLIT>;
  using Regs = typename U::Regs;
  using RG = Ring<FMT, SF32, D>;
  constexpr int NB = SH::NB;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;
  __shared__ SH sh;

  const WorkRec w = load_work((const sconst_work*)p.work + blockIdx.x);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int q_stride = p.q_heads * D;
  const int row0 = wave * 32;
  const bool has_rows = row0 < w.rows;

  LayerRsrc rs;
  rs.k = make_rsrc(p.kpool, p.kv_array_bytes);
  rs.v = make_rsrc(p.vpool, p.kv_array_bytes);

  // This wave's rows: Q^T operands (as in attend_unit) and visible limits.
  U u;
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = row0 + rg * 16 + col;
    const bool valid = r < w.rows;
    const int qi = w.row_begin + (valid ? r / w.rows_per_query : 0);
    const int head = w.head_base + (valid ? r % w.rows_per_query : 0);
    const float* qp = p.q + (size_t)(w.q_row + qi) * q_stride + (size_t)head * D + 4 * grp;
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      float4 a = make_float4(0, 0, 0, 0), b = make_float4(0, 0, 0, 0);
      if (valid) {
        a = *reinterpret_cast<const float4*>(qp + 32 * pp);
        b = *reinterpret_cast<const float4*>(qp + 32 * pp + 16);
      }
      const float c = p.scale_log2;
      const float x[8] = {a.x * c, a.y * c, a.z * c, a.w * c, b.x * c, b.y * c, b.z * c, b.w * c};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const _Float16 hi = (_Float16)x[j];
        u.qhi[rg][pp][j] = hi;
        u.qlo[rg][pp][j] = QSPLIT ? (_Float16)(x[j] - (float)hi) : (_Float16)0.0f;
      }
    }
    u.lim[rg] = valid ? w.ctx + w.row_begin + r / w.rows_per_query : -1;
    u.base[rg] = 0.0f;
    u.thr[rg] = -INFINITY;
    u.l4[rg] = float4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] = float4_t{0, 0, 0, 0};
  }
  // Pages at or past `unmasked` hold a position some row of the wave may not see.
  const int unmasked = (w.ctx + w.row_begin + row0 / w.rows_per_query + 1) / 16;

  const int npages = w.page_end - w.page_begin;
  const int ntiles = (npages + kWaves - 1) / kWaves;
  const sconst_int* table = (const sconst_int*)(p.tables + w.table_off + w.page_begin);
  // Tile k, page `wave` of it: fetched by this wave (nothing past the range).
  auto fetch_tile = [&](int k) __attribute__((always_inline)) -> void {
    const int j = k * kWaves + wave;
    if (j < npages) {
      fetch_page<FMT, SF32, D>(sh.ring + (k % NB) * SH::TILE + wave * RG::SLOT, rs, p,
                               table[j] * p.kv_heads + w.kv_head, lane);
    }
  };
#pragma unroll
  for (int k = 0; k < NB - 1; ++k) {
    if (k < ntiles) fetch_tile(k);
  }
  // Last tile holding a page of this wave.
  const int t_last = wave < npages ? (npages - 1 - wave) / kWaves : -1;
  for (int k = 0; k < ntiles; ++k) {
    // this wave's page of tile k has landed (its pages of up to NB - 2
    // younger tiles may still be in flight), then every wave's has, and
    // every wave is done with tile k - 1, whose slot the fetch below refills
    if (k <= t_last) {
      const int younger = (k + NB - 2 < t_last ? k + NB - 2 : t_last) - k;
      wait_vmcnt_pages<NB - 2, RG::LOADS>(younger);
    }
    lds_barrier();
    if (k + NB - 1 < ntiles) fetch_tile(k + NB - 1);
    if (has_rows) {
      const char* tile = sh.ring + (k % NB) * SH::TILE;
#pragma unroll
      for (int j = 0; j < kWaves; ++j) {
        const int pg = k * kWaves + j;
        if (pg < npages) {
          Regs r;
          read_page<FMT, SF32, D>(r, tile + j * RG::SLOT, lane, grp);
          const int pi = w.page_begin + pg;
          u.consume(r, pi, grp, pi >= unmasked);
        }
      }
    }
  }
  if (!has_rows) return;

  // Write this wave's rows: normalised output, or the split's partial state.
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = row0 + rg * 16 + col;
    if (r >= w.rows) continue;
    const float sum = u.l4[rg][0];
    if (w.part < 0) {
      const int qi = w.row_begin + r / w.rows_per_query;
      const int head = w.head_base + r % w.rows_per_query;
      float* op = p.out + (size_t)(w.q_row + qi) * q_stride + (size_t)head * D + 4 * grp;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float4_t res = float4_t{0, 0, 0, 0};
        if (sum > 0.0f) res = div4(u.o[rg][t], sum);
        *reinterpret_cast<float4_t*>(op + 16 * t) = res;
      }
    } else {
      float* po = p.part_o + ((size_t)w.part * p.rows_cap + r) * D + 4 * grp;
#pragma unroll
      for (int t = 0; t < NT; ++t) *reinterpret_cast<float4_t*>(po + 16 * t) = u.o[rg][t];
      if (grp == 0) {
        p.part_ml[((size_t)w.part * p.rows_cap + r) * 2] = u.thr[rg] == -INFINITY ? -INFINITY : u.base[rg];
        p.part_ml[((size_t)w.part * p.rows_cap + r) * 2 + 1] = sum;
      }
    }
  }
}

// Merge the partial states of the splits of one unit (merge_gqa_chunks:
// splits with no visible position are skipped, none at all gives zeros).
// A row's D/4 lanes (4 dims each) are replicated over S slots; slot j folds
// splits j, j+S, ... (loads issued in batches of 8) into a running
// (max, sum, acc) state, and slot 0 combines the S states in slot order, so
// the result does not depend on timing. Rows per block = 256 / (D/4 * S).
template <int D, int S>
__global__ __launch_bounds__(256) void split_reduce_kernel(ReduceParams p) {
  constexpr int L = D / 4;
  constexpr int RPB = 256 / (L * S);
  static_assert(RPB >= 1 && RPB * L * S == 256, "block shape");
  __shared__ float sh_m[RPB][S];
  __shared__ float sh_l[RPB][S];
  __shared__ float4_t sh_o[RPB][S][L];

  const ReduceRec it = p.items[blockIdx.x];
  const int t = threadIdx.x;
  const int d4 = t % L;
  const int slot = (t / L) % S;
  const int rr = t / (L * S);
  const int r = blockIdx.y * RPB + rr;
  const bool active = r < it.rows;

  float m = -INFINITY, sum = 0.0f;
  float4_t acc = float4_t{0, 0, 0, 0};
  if (active) {
    const float2* ml = reinterpret_cast<const float2*>(p.part_ml) + (size_t)it.first_part * p.rows_cap + r;
    const float* po = p.part_o + ((size_t)it.first_part * p.rows_cap + r) * D + 4 * d4;
    const size_t stride_ml = p.rows_cap;
    const size_t stride_o = (size_t)p.rows_cap * D;
    for (int k0 = slot; k0 < it.n_parts; k0 += 8 * S) {
      float2 x[8];
      float4_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = k0 + S * i;
        const bool ok = k < it.n_parts;
        x[i] = ok ? ml[k * stride_ml] : make_float2(-INFINITY, 0.0f);
        v[i] = ok ? *reinterpret_cast<const float4_t*>(po + k * stride_o) : float4_t{0, 0, 0, 0};
      }
      float bm = m;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (x[i].y > 0.0f) bm = fmaxf(bm, x[i].x);
      if (bm == -INFINITY) continue;  // nothing visible in this batch yet
      const float c = m == -INFINITY ? 0.0f : pow2i(m - bm);
      sum *= c;
      acc *= c;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float f = x[i].y > 0.0f ? pow2i(x[i].x - bm) : 0.0f;
        sum += x[i].y * f;
        acc += v[i] * f;
      }
      m = bm;
    }
  }
  if constexpr (S > 1) {
    sh_o[rr][slot][d4] = acc;
    if (d4 == 0) {
      sh_m[rr][slot] = m;
      sh_l[rr][slot] = sum;
    }
    __syncthreads();
    if (slot != 0 || !active) return;
    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < S; ++j) mm = fmaxf(mm, sh_m[rr][j]);
    sum = 0.0f;
    acc = float4_t{0, 0, 0, 0};
    if (mm != -INFINITY) {
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const float mj = sh_m[rr][j];
        const float f = mj == -INFINITY ? 0.0f : pow2i(mj - mm);
        sum += sh_l[rr][j] * f;
        acc += sh_o[rr][j][d4] * f;
      }
    }
  } else {
    if (!active) return;
  }
  const SessionRec s = p.sessions[it.session];
  const int q_stride = p.q_heads * D;
  const int qi = it.row_begin + r / it.rows_per_query;
  const int head = it.head_base + r % it.rows_per_query;
  float4_t res = float4_t{0, 0, 0, 0};
  if (sum > 0.0f) res = div4(acc, sum);
  *reinterpret_cast<float4_t*>(p.out + (size_t)(s.q_row + qi) * q_stride + (size_t)head * D + 4 * d4) = res;
}

}  // namespace

// Whether a variant's decode ring (two or more slots per wave) and merge
// area fit its share of LDS; the others run the unit-at-a-time kernel.
template <int FMT, bool SF32, int D, int NRG>
constexpr bool decode_fits() {
  constexpr int wpe = waves_per_eu<FMT, D, NRG, true>();
  constexpr int rows = 16 * NRG;
  constexpr int merge = 4 * (2 * kWaves * rows + rows * (D + 4));
  return (160 * 1024 / wpe - merge - 64) / (kWaves * Ring<FMT, SF32, D>::SLOT) >= 2;
}

template <int FMT, bool SF32, int D>
hipError_t launch_decode_d(int row_groups, int n_groups, const AttnParams& p, hipStream_t stream) {
  switch (row_groups) {
#define TGE_DEC(n)                                                                                 \
  case n: {                                                                                        \
    constexpr int wpe = waves_per_eu<FMT, D, n, true>();                                           \
    if constexpr (decode_fits<FMT, SF32, D, n>()) {                                                \
      hipLaunchKernelGGL((paged_decode_kernel<FMT, SF32, D, n, true, wpe>),                        \
                         dim3((unsigned)n_groups), dim3(256), 0, stream, p);                       \
    } else {                                                                                       \
      hipLaunchKernelGGL((paged_attention_kernel<FMT, SF32, D, n, true, wpe>),                     \
                         dim3((unsigned)n_groups), dim3(256), 0, stream, p);                       \
    }                                                                                              \
    break;                                                                                         \
  }
    TGE_DEC(1)
    TGE_DEC(2)
    TGE_DEC(3)
    TGE_DEC(4)
#undef TGE_DEC
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int FMT, bool SF32, int D>
int decode_blocks_d(int row_groups) {
  int n = 0;
  hipError_t e = hipErrorInvalidValue;
  switch (row_groups) {
#define TGE_DOCC(r)                                                                          \
  case r: {                                                                                  \
    constexpr int wpe = waves_per_eu<FMT, D, r, true>();                                     \
    if constexpr (decode_fits<FMT, SF32, D, r>()) {                                          \
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(                                      \
          &n, paged_decode_kernel<FMT, SF32, D, r, true, wpe>, 256, 0);                      \
    } else {                                                                                 \
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(                                      \
          &n, paged_attention_kernel<FMT, SF32, D, r, true, wpe>, 256, 0);                   \
    }                                                                                        \
    break;                                                                                   \
  }
    TGE_DOCC(1)
    TGE_DOCC(2)
    TGE_DOCC(3)
    TGE_DOCC(4)
#undef TGE_DOCC
    default:
      break;
  }
  return e == hipSuccess ? n : 0;
}

hipError_t launch_decode(int format, int scale_f32, int head_dim, int row_groups, int n_groups,
                         const AttnParams& p, hipStream_t stream) {
  if (n_groups <= 0) return hipSuccess;
  if (!p.wg_first) return hipErrorInvalidValue;
  if (format == kF16) {
    if (head_dim == 64) return launch_decode_d<kF16, false, 64>(row_groups, n_groups, p, stream);
    if (head_dim == 128) return launch_decode_d<kF16, false, 128>(row_groups, n_groups, p, stream);
  } else if (format == kI8) {
    if (head_dim == 64)
      return scale_f32 ? launch_decode_d<kI8, true, 64>(row_groups, n_groups, p, stream)
                       : launch_decode_d<kI8, false, 64>(row_groups, n_groups, p, stream);
    if (head_dim == 128)
      return scale_f32 ? launch_decode_d<kI8, true, 128>(row_groups, n_groups, p, stream)
                       : launch_decode_d<kI8, false, 128>(row_groups, n_groups, p, stream);
  }
  return hipErrorInvalidValue;
}

int decode_blocks_per_cu(int format, int scale_f32, int head_dim, int row_groups) {
  if (format == kF16) {
    return head_dim == 64 ? decode_blocks_d<kF16, false, 64>(row_groups)
                          : decode_blocks_d<kF16, false, 128>(row_groups);
  }
  if (head_dim == 64)
    return scale_f32 ? decode_blocks_d<kI8, true, 64>(row_groups) : decode_blocks_d<kI8, false, 64>(row_groups);
  return scale_f32 ? decode_blocks_d<kI8, true, 128>(row_groups) : decode_blocks_d<kI8, false, 128>(row_groups);
}

template <int FMT, bool SF32, int D, bool QSPLIT>
hipError_t launch_prefill_d(int n_units, const AttnParams& p, hipStream_t stream) {
  constexpr int wpe = waves_per_eu<FMT, D, 2, QSPLIT>();
  hipLaunchKernelGGL((paged_prefill_kernel<FMT, SF32, D, QSPLIT, wpe>), dim3((unsigned)n_units),
                     dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_prefill(int format, int scale_f32, int head_dim, bool qsplit, int n_units,
                          const AttnParams& p, hipStream_t stream) {
  if (n_units <= 0) return hipSuccess;
  if (format == kF16) {
    if (head_dim == 64)
      return qsplit ? launch_prefill_d<kF16, false, 64, true>(n_units, p, stream)
                    : launch_prefill_d<kF16, false, 64, false>(n_units, p, stream);
    if (head_dim == 128)
      return qsplit ? launch_prefill_d<kF16, false, 128, true>(n_units, p, stream)
                    : launch_prefill_d<kF16, false, 128, false>(n_units, p, stream);
  } else if (format == kI8 && qsplit) {
    if (head_dim == 64)
      return scale_f32 ? launch_prefill_d<kI8, true, 64, true>(n_units, p, stream)
                       : launch_prefill_d<kI8, false, 64, true>(n_units, p, stream);
    if (head_dim == 128)
      return scale_f32 ? launch_prefill_d<kI8, true, 128, true>(n_units, p, stream)
                       : launch_prefill_d<kI8, false, 128, true>(n_units, p, stream);
  }
  return hipErrorInvalidValue;
}

template <int D>
hipError_t launch_reduce_d(int n_items, int max_parts, const ReduceParams& p, hipStream_t stream) {
  // Slots per row: about one per 4 splits, at most 8.
  const int want = (max_parts + 3) / 4;
  const int slots = want <= 1 ? 1 : (want <= 2 ? 2 : (want <= 4 ? 4 : 8));
  const int rpb = 256 / (D / 4 * slots);
  const dim3 grid((unsigned)n_items, (unsigned)((p.rows_cap + rpb - 1) / rpb)), block(256);
  switch (slots) {
    case 1: hipLaunchKernelGGL((split_reduce_kernel<D, 1>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((split_reduce_kernel<D, 2>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((split_reduce_kernel<D, 4>), grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL((split_reduce_kernel<D, 8>), grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

hipError_t launch_reduce(int head_dim, int n_items, int max_parts, const ReduceParams& p,
                         hipStream_t stream) {
  if (n_items == 0) return hipSuccess;
  if (head_dim == 64) return launch_reduce_d<64>(n_items, max_parts, p, stream);
  if (head_dim == 128) return launch_reduce_d<128>(n_items, max_parts, p, stream);
  return hipErrorInvalidValue;
}

}  // namespace tge
