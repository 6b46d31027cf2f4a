// Shared device code of the paged attention kernels (decode, block prefill,
// small decode steps): vector types, the page-block register image, the
// LDS ring and its direct-to-LDS fetch, the int8 -> f16 conversion, and the
// per-page online-softmax unit on CDNA4 matrix cores. See paged_attention.hip
// for the math and the page layout in tge_common.h.
#pragma once

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

// max(a, b, c) in one instruction (scores are never signalling NaNs, so
// the operand quieting fmaxf would add is not needed).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
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

// Buffer resource of one page block (64-bit base, so a layer's array may
// exceed 4 GiB). Loads add the lane's piece offset (VGPR); offsets past the
// block read zeros instead of faulting.
[[maybe_unused]] __device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                                         uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void_t;
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

// Waves per SIMD the block-prefill kernel is compiled for: the register
// budget that keeps every live value in the 256 architectural VGPRs while
// leaving room for a second wave to hide latency.
template <int FMT, int D, int NRG>
constexpr int waves_per_eu() {
  return D == 64 ? (NRG <= 2 ? 3 : 2) : D == 128 ? (NRG <= 2 ? 2 : 1) : 1;
}

// Cache policy of the decode kernels' page-block loads: non-temporal (the
// gfx950 "nt" bit of the buffer instruction's cache-policy operand). A decode
// launch reads every page block once; with this hint, and each instruction
// covering a whole contiguous KiB, scattered 4352-byte blocks stream at
// 6.6-6.9 TB/s on an MI355X against 5.9-6.0 TB/s with the default policy or
// with 16-byte pieces 32 bytes apart. Block-prefill tiles of one KV head
// read the same pages, so the prefill kernel keeps the default policy
// (kPageReusePolicy), under which those re-reads hit the L2.
constexpr int kPageLoadPolicy = 2;
constexpr int kPageReusePolicy = 0;

// Issue the direct-to-LDS loads of the page block at `block` into `slot`:
// the block's K part, V part and (int8) the K and V scale parts, which follow
// each other in memory. Load i of a part copies its i-th KiB (piece i of
// every lane, page layout in tge_common.h), so the slot holds the block in
// its memory layout. The block gets its own buffer resource (wave-uniform,
// built from the 64-bit address in scalar registers); the instruction offset
// field stays 0 (it would move the LDS address too), so every offset goes
// into the lane's VGPR.
template <int FMT, bool SF32, int D, int POLICY = kPageLoadPolicy>
__device__ __forceinline__ void fetch_page(char* slot, const char* block, uint32_t block_bytes,
                                           int lane) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS-load builtins exist for the device pass only
  using RG = Ring<FMT, SF32, D>;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(block, block_bytes);
  constexpr uint32_t boff = 0;
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + i * 1024), 16,
                                             i * 1024 + lane * 16, boff, 0, POLICY);
  }
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + RG::KV_BYTES + i * 1024), 16,
                                             RG::KV_BYTES + i * 1024 + lane * 16, boff, 0,
                                             POLICY);
  }
  if constexpr (FMT == kI8) {
    // dword d of [K scales | V scales]; lanes past the end re-read dword 0
    // into the slot's padding (never the next block).
#pragma unroll
    for (int i = 0; i < RG::SC_LOADS; ++i) {
      const int d = i * 64 + lane;
      const int dd = d < RG::SC_BYTES / 2 ? d : 0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + 2 * RG::KV_BYTES + i * 256),
                                               4, 2 * RG::KV_BYTES + 4 * dd, boff, 0, POLICY);
    }
  }
#endif
}

// Read a landed page back into registers (the lane's own pieces and its
// group's scales): the K half (K codes and scales) and the V half, so a
// consumer can hold only the half it is using.
template <int FMT, bool SF32, int D, bool V>
__device__ __forceinline__ void read_half(PageRegs<FMT, SF32, D>& r, const char* slot, int lane,
                                          int grp) {
  using RG = Ring<FMT, SF32, D>;
  using R = PageRegs<FMT, SF32, D>;
  uint32_t* c = V ? r.v : r.k;
  uint32_t* sc = V ? r.vs : r.ks;
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(slot + (V ? RG::KV_BYTES : 0) + i * 1024 + 16 * lane);
    c[4 * i] = x.x; c[4 * i + 1] = x.y; c[4 * i + 2] = x.z; c[4 * i + 3] = x.w;
  }
  if constexpr (FMT == kI8) {
    const char* ss = slot + 2 * RG::KV_BYTES + grp * R::SW * 4 + (V ? RG::SC_BYTES : 0);
#pragma unroll
    for (int i = 0; i < R::SW / 4; ++i) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(ss + 16 * i);
      sc[4 * i] = a.x; sc[4 * i + 1] = a.y; sc[4 * i + 2] = a.z; sc[4 * i + 3] = a.w;
    }
  }
}

template <int FMT, bool SF32, int D>
__device__ __forceinline__ void read_page(PageRegs<FMT, SF32, D>& r, const char* slot, int lane,
                                          int grp) {
  read_half<FMT, SF32, D, false>(r, slot, lane, grp);
  read_half<FMT, SF32, D, true>(r, slot, lane, grp);
}

typedef const __attribute__((address_space(4))) WorkRec sconst_work;

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
  r.red = q[12];
  return r;
}

// Barrier of a group of a workgroup's waves through an LDS counter: this
// wave's LDS reads are complete, it counts in, and waits until `target`
// arrivals have been counted in total. The wait is bounded (about 0.2 s):
// past the bound the wave goes on (the launch completes with wrong rows
// instead of hanging) and the expiry is counted in *expired.
__device__ __forceinline__ void bounded_barrier(int* ctr, int target, unsigned int* expired) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  constexpr int kSpins = 1 << 21;
  int spin = 0;
  for (; spin < kSpins; ++spin) {
    const int seen = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (seen >= target) break;
    __builtin_amdgcn_s_sleep(1);
  }
  if (spin == kSpins && (threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
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

// ---- In-kernel split merge (the last piece of a split record merges) ------
// A piece of a split (session, KV head[, query tile]) writes its partial
// (max, sum, acc) with the device-coherent cache policy sc1 (written
// through, and read past, the XCD's non-coherent L2: the bits gfx950's
// agent-scope relaxed atomics carry), waits for those stores, and bumps the
// record's arrival counter; the piece that arrives last reads every partial
// of the record (again with sc1) and writes the output rows, then re-arms
// the counter for the next launch. No agent-scope fence is used: on gfx950
// it writes back the XCD's whole L2.
constexpr int kCohPolicy = 16;  // buffer cache-policy operand: sc1
__device__ __forceinline__ void coh_store4(__amdgpu_buffer_rsrc_t rs, uint32_t off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rs, off, 0, kCohPolicy);
}
__device__ __forceinline__ void coh_store2(__amdgpu_buffer_rsrc_t rs, uint32_t off, float a, float b) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{__float_as_uint(a), __float_as_uint(b)}, rs, off, 0,
                                        kCohPolicy);
}
__device__ __forceinline__ float4_t coh_load4(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kCohPolicy));
}
__device__ __forceinline__ float2 coh_load2(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kCohPolicy);
  return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

// Partial slot `part`, row r: its accumulators (4 dims at d4) and its
// (max, sum), written coherently.
template <int D>
__device__ __forceinline__ void store_partial_row(const AttnParams& p, int part, int r, int d4,
                                                  float4_t acc) {
  const auto rs = make_rsrc(p.part_o, 0x7fffffff);
  coh_store4(rs, (uint32_t)((((size_t)part * p.rows_cap + r) * D + 4 * d4) * 4), acc);
}
__device__ __forceinline__ void store_partial_ml(const AttnParams& p, int part, int r, float m,
                                                 float sum) {
  const auto rs = make_rsrc(p.part_ml, 0x7fffffff);
  coh_store2(rs, (uint32_t)(((size_t)part * p.rows_cap + r) * 8), m, sum);
}

// merge_gqa_chunks (qwen2.cpp:1469-1522) over the partial slots of record
// `rr` (at most RMAX rows) by the 256 threads of one workgroup; slots with
// no visible position are skipped, none at all gives zeros. `lds` is
// scratch of at least 10 * RMAX floats.
//   A. each row's common base M (the largest max of its visible slots) and
//      total sum S, one thread per row folding the slots in order;
//   B. the accumulators slot by slot: for a batch of slots the weights
//      2^(max - M) go to LDS, then every thread loads its (row, 4 dims)
//      pairs of those slots at once and adds them in slot order.
template <int D, int RMAX>
__device__ __forceinline__ void merge_record(const AttnParams& p, const ReduceRec& rr, float* lds) {
  constexpr int NT = 256;
  constexpr int L = D / 4;
  constexpr int PJ = (RMAX * L + NT - 1) / NT;       // pairs per thread
  constexpr int SB = PJ >= 32 ? 1 : 32 / PJ > 8 ? 8 : 32 / PJ;  // slots per batch of loads
  float* lM = lds;              // [RMAX]
  float* lS = lds + RMAX;       // [RMAX]
  float* lw = lds + 2 * RMAX;   // [8][RMAX] weights of a batch of slots
  const auto rs_o = make_rsrc(p.part_o, 0x7fffffff);
  const auto rs_ml = make_rsrc(p.part_ml, 0x7fffffff);
  const int n = rr.n_parts, rows = rr.rows;
  const int t = threadIdx.x;
  auto ml_off = [&](int k, int r) { return (uint32_t)((((size_t)(rr.first_part + k)) * p.rows_cap + r) * 8); };
  // A.
  if (t < rows) {
    float m = -INFINITY, sum = 0.0f;
    for (int k0 = 0; k0 < n; k0 += 8) {
      float2 x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = coh_load2(rs_ml, ml_off(min(k0 + i, n - 1), t));
      float bm = m;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < n && x[i].y > 0.0f) bm = fmaxf(bm, x[i].x);
      if (bm == -INFINITY) continue;
      sum *= m == -INFINITY ? 0.0f : pow2i(m - bm);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < n && x[i].y > 0.0f) sum += x[i].y * pow2i(x[i].x - bm);
      m = bm;
    }
    lM[t] = m;
    lS[t] = sum;
  }
  __syncthreads();
  // B.
  float4_t acc[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) acc[j] = float4_t{0, 0, 0, 0};
  for (int k0 = 0; k0 < n; k0 += 8) {
    const int kn = min(8, n - k0);
    for (int i = t; i < kn * rows; i += NT) {
      const int kk = i / rows, r = i - kk * rows;
      const float2 x = coh_load2(rs_ml, ml_off(k0 + kk, r));
      const float mm = lM[r];
      lw[kk * RMAX + r] = x.y > 0.0f && mm != -INFINITY ? pow2i(x.x - mm) : 0.0f;
    }
    __syncthreads();
    for (int kb = 0; kb < kn; kb += SB) {
      float4_t v[SB][PJ];
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        const int k = k0 + min(kb + b, kn - 1);
#pragma unroll
        for (int j = 0; j < PJ; ++j) {
          const int pair = min(t + NT * j, rows * L - 1);
          const int r = pair / L, d4 = pair - r * L;
          v[b][j] = coh_load4(rs_o, (uint32_t)(((((size_t)(rr.first_part + k)) * p.rows_cap + r) * D + 4 * d4) * 4));
        }
      }
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        if (kb + b >= kn) break;
#pragma unroll
        for (int j = 0; j < PJ; ++j) {
          const int pair = t + NT * j;
          if (pair < rows * L) acc[j] += v[b][j] * lw[(kb + b) * RMAX + pair / L];
        }
      }
    }
    __syncthreads();  // the weights of this batch are read
  }
  const int q_stride = p.q_heads * p.dims;
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int pair = t + NT * j;
    if (pair >= rows * L) continue;
    const int r = pair / L, d4 = pair - r * L;
    if (4 * d4 >= p.dims) continue;  // a dim past the head's own
    const float sum = lS[r];
    const int qi = rr.row_begin + r / rr.rows_per_query;
    const int head = rr.head_base + r % rr.rows_per_query;
    float4_t res = float4_t{0, 0, 0, 0};
    if (sum > 0.0f) res = div4(acc[j], sum);
    *reinterpret_cast<float4_t*>(p.out + (size_t)(rr.q_row + qi) * q_stride + (size_t)head * p.dims + 4 * d4) = res;
  }
}

// Called by every thread of a (256-thread) workgroup once its piece of
// split record `red` has written its partial rows (coherently): counts the
// arrival, and the last piece merges the record and re-arms its counter.
// `flag` is an LDS int of the workgroup, `scratch` 10 * RMAX LDS floats that
// nothing else uses meanwhile. Waits for all of this workgroup's memory
// operations (loads in flight included).
template <int D, int RMAX>
__device__ __forceinline__ void arrive_and_merge(const AttnParams& p, int red, int* flag, float* scratch) {
  const ReduceRec rr = p.reduce[red];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  wait_vmcnt<0>();  // this wave's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(p.counters + red, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = prev == rr.n_parts - 1;
  }
  __syncthreads();
  const bool last = *flag != 0;
  __syncthreads();  // every wave has read the flag before a later arrival rewrites it
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  merge_record<D, RMAX>(p, rr, scratch);
  if (threadIdx.x == 0) __hip_atomic_store(p.counters + red, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Byte address within the workgroup's LDS of a pointer into it.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
// 8 bytes of LDS at addr + OFF into an f16x4, as one ds_read_b64 that the
// compiler neither fuses with its neighbours nor waits for: the caller
// waits with lds_wait_operands before any use of the result.
template <int OFF>
__device__ __forceinline__ half4_t lds_read_b64(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  half4_t v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
// The PV operands of a page pair from its two LDS slots (lane chunk bases
// la, lb): operand (pp, h) = page A's then page B's 8 bytes at 1024*pp + 8*h.
template <int PP, int NP>
__device__ __forceinline__ void read_v_pairs(half8_t (&v8)[NP][2], uint32_t la, uint32_t lb) {
  if constexpr (PP < NP) {
    const half4_t a0 = lds_read_b64<1024 * PP>(la), b0 = lds_read_b64<1024 * PP>(lb);
    const half4_t a1 = lds_read_b64<1024 * PP + 8>(la), b1 = lds_read_b64<1024 * PP + 8>(lb);
    v8[PP][0] = half8_t{a0[0], a0[1], a0[2], a0[3], b0[0], b0[1], b0[2], b0[3]};
    v8[PP][1] = half8_t{a1[0], a1[1], a1[2], a1[3], b1[0], b1[1], b1[2], b1[3]};
    read_v_pairs<PP + 1, NP>(v8, la, lb);
  }
}
// Waits for this wave's LDS reads; the operands pass through the wait, so
// no use of them can be scheduled before it.
template <int NP>
__device__ __forceinline__ void lds_wait_operands(half8_t (&v)[NP][2]) {
  static_assert(NP == 2 || NP == 4 || NP == 8, "64, 128 or 256 dims");
  if constexpr (NP == 2) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[1][0]), "+v"(v[1][1]));
  } else if constexpr (NP == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[1][0]), "+v"(v[1][1]), "+v"(v[2][0]),
                   "+v"(v[2][1]), "+v"(v[3][0]), "+v"(v[3][1]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[1][0]), "+v"(v[1][1]), "+v"(v[2][0]),
                   "+v"(v[2][1]), "+v"(v[3][0]), "+v"(v[3][1]), "+v"(v[4][0]), "+v"(v[4][1]),
                   "+v"(v[5][0]), "+v"(v[5][1]), "+v"(v[6][0]), "+v"(v[6][1]), "+v"(v[7][0]),
                   "+v"(v[7][1]));
  }
}

#define MFMA16x16x16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x16f16((a), (b), (c), 0, 0, 0)
#define MFMA16x16x32(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

template <int FMT, bool SF32, int D, int NRG>
struct Unit {
  static constexpr int NP = D / 32;
  static constexpr int NT = D / 16;
  using Regs = PageRegs<FMT, SF32, D>;

  half8_t q[NRG][NP];  // Q^T operands (prefill; decode reads them from LDS)
  int lim[NRG];
  // Static sparse subset (attention_head_static_sparse_avx2 / _fp16_avx2,
  // attention_avx2.cpp:263-490; the kept set of build_sparse_index,
  // qwen2.cpp:192-220): a row whose span exceeds sink + window keeps the
  // positions below sink, every stride-th one from sink on, and the last
  // `window`; other rows are dense. mid[rg] is where the row's window
  // starts (sink for a dense row); sp_hi the largest mid of the unit's rows
  // (wave-uniform). sp_stride 0: off.
  int sp_sink, sp_stride, sp_hi;
  int mid[NRG];
  // the phase's modulo without a division per page (Lemire's fastmod:
  // sp_m = 2^64 / stride rounded up; (p0 + sp_off) mod stride equals
  // (p0 - sink) mod stride with a non-negative left side)
  uint64_t sp_m;
  int sp_off;
  // Strides up to 28: bit x of sp_on is set for x in {0, stride, 2*stride}
  // (a position's phase plus its index in the lane's run is below 32), and
  // sp_lo is the smallest window start over the wave's valid rows, so a
  // page in [sink, sp_lo) is wholly inside every row's strided middle.
  uint32_t sp_on;
  int sp_lo;

  __device__ __forceinline__ void set_sparse(int sink, int window, int stride, int span_max) {
    sp_sink = sink;
    if (stride > 0) {
      sp_m = ~0ull / (uint64_t)stride + 1;
      sp_off = stride - sink % stride;
    }
    sp_stride = stride;
    sp_hi = span_max > sink + window ? span_max - window : sink;
    int lo = 0x7fffffff;
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const int span = lim[rg] + 1;
      mid[rg] = span > sink + window ? span - window : sink;
      if (lim[rg] >= 0) lo = min(lo, mid[rg]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) lo = min(lo, __shfl_xor(lo, off));
    sp_lo = stride > 0 && stride <= 28 ? lo : sink;  // (sink: no page takes the fast path)
    sp_on = stride > 0 && stride <= 28 ? (1u | (1u << stride) | (stride <= 15 ? 1u << (2 * stride) : 0u)) : 0u;
  }
  // Whether page pi holds a position some row may drop (wave-uniform).
  __device__ __forceinline__ bool sparse_page(int pi) const {
    return sp_stride > 0 && pi * 16 + 15 >= sp_sink && pi * 16 < sp_hi;
  }
  // Phase of the lane's first position p0 on the stride: (p0 - sink) mod
  // stride in [0, stride), also when p0 < sink (a lane's 4 positions may
  // straddle sink).
  __device__ __forceinline__ int sparse_phase(int p0) const {
    const uint32_t a = (uint32_t)(p0 + sp_off);
    const uint64_t low = sp_m * a;
    const uint64_t s = (uint64_t)(uint32_t)(low >> 32) * (uint32_t)sp_stride +
                       __umulhi((uint32_t)low, (uint32_t)sp_stride);
    return (int)(s >> 32);
  }
  // Drop the lane's 4 positions p0..p0+3 of row group rg that fall between
  // sink and the row's window off the stride; `ph` = sparse_phase(p0).
  // ph + e < stride + 4 <= 3 * stride, so on-stride means ph + e is 0,
  // stride or 2 * stride.
  __device__ __forceinline__ void sparse_mask(float4_t& s, int p0, int ph, int rg) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p = p0 + e, x = ph + e;
      const bool on = x == 0 || x == sp_stride || x == 2 * sp_stride;
      if (p >= sp_sink && p < mid[rg] && !on) s[e] = -INFINITY;
    }
  }
  // Online softmax state per row, log2 domain. Scores are kept relative to
  // `base`; the weights exp2(s - base) never exceed 2^kLazyMax because base
  // moves (rarely) whenever a score passes base + kLazyMax. `thr` is that
  // threshold, -inf while the row has seen no visible position.
  float base[NRG], thr[NRG];
  float4_t l4[NRG];  // row sums (all four entries equal), via the ones MFMA
  float4_t o[NRG][NT];

  __device__ __forceinline__ half8_t qop(int rg, int pp) const {
    return q[rg][pp];
  }

  // S^T = K.Q^T of one page for every row group (fp32, K scales applied),
  // added onto the values already in sacc.
  template <class QF>
  __device__ __forceinline__ void scores_onto(const Regs& r, const QF& qf, float4_t (&sacc)[NRG]) const {
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      const half8_t ka = k_operand<FMT, SF32, D>(r, pp);
      if (FMT == kF16) {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
          sacc[rg] = MFMA16x16x32(ka, qf(rg, pp), sacc[rg]);
        }
      } else {
        const float4_t ks = scales4<SF32>(r.ks, pp);
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
          float4_t b = MFMA16x16x32(ka, qf(rg, pp), (float4_t{0, 0, 0, 0}));
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[rg][e] = fmaf(b[e], ks[e], sacc[rg][e]);
        }
      }
    }
  }

  // V^T operand (16 dims x 4 tokens per lane) of 16-dim tile 2pp+h.
  __device__ __forceinline__ half4_t v_operand(const Regs& r, int pp, int h) const {
    if (FMT == kF16) {
      return as_half4(r.v[4 * pp + 2 * h], r.v[4 * pp + 2 * h + 1]);
    } else if (SF32) {
      const float4_t sv = scales4<SF32>(r.vs, pp);
      const half4_t c = i8x4_to_half4(r.v[2 * pp + h]);
      return half4_t{(_Float16)((float)c[0] * sv[0]), (_Float16)((float)c[1] * sv[1]),
                     (_Float16)((float)c[2] * sv[2]), (_Float16)((float)c[3] * sv[3])};
    } else {
      return i8x4_to_half4(r.v[2 * pp + h]) * as_half4(r.vs[2 * pp], r.vs[2 * pp + 1]);
    }
  }

  // Two pages at once: the QK products of both, one softmax update over the
  // 32 positions, and the value and row-sum products on 16x16x32 MFMAs with
  // k = 8g + j = token 4g+j of page A (j < 4) or 4g+j-4 of page B: lane (g, c)
  // already holds exactly those tokens of both pages, for P as for V.
  // The score accumulators start at -base, so the scores come out relative
  // to the row bases; the causal mask runs only for pages on the diagonal
  // (masked_a / masked_b are wave-uniform), and one rarely taken branch
  // rebases every row group, so the exponentials, the row sums and the value
  // products of both row groups form one straight block.
  template <class QF>
  __device__ __forceinline__ void consume2(const Regs& ra, const Regs& rb, int pia, int pib, int grp,
                                           bool masked_a, bool masked_b, const QF& qf) {
    float4_t sa[NRG], sb[NRG];
    start_scores(sa, sb);
    scores_onto(ra, qf, sa);
    scores_onto(rb, qf, sb);
    half8_t pw[NRG];
    softmax2(sa, sb, pia, pib, grp, masked_a, masked_b, pw);
    values2(
        [&](int pp, int h) __attribute__((always_inline)) {
          const half4_t va = v_operand(ra, pp, h), vb = v_operand(rb, pp, h);
          return half8_t{va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
        },
        pw);
  }

  // The same for two f16 pages still in their LDS slots: the K halves are
  // read for the scores, and the V operands (four tokens of each page) are
  // read straight into their MFMA operand registers while the softmax runs.
  template <class QF>
  __device__ __forceinline__ void consume2_slots(const char* slot_a, const char* slot_b, int lane,
                                                 int pia, int pib, int grp, bool masked_a,
                                                 bool masked_b, const QF& qf) {
    static_assert(FMT == kF16, "f16 pages only");
    using RG = Ring<FMT, SF32, D>;
    Regs ra, rb;
    read_half<FMT, SF32, D, false>(ra, slot_a, lane, grp);
    read_half<FMT, SF32, D, false>(rb, slot_b, lane, grp);
    // V operands: page A's 8 bytes and page B's 8 bytes side by side in one
    // operand, each read by its own ds_read_b64 into its half of the
    // operand's registers (written as plain loads, the compiler fuses a
    // lane's two halves into one 16-byte read and splits it with moves).
    // The reads are not tracked by the compiler: lds_wait_operands below
    // waits for them before the first use.
    const uint32_t la = lds_addr(slot_a + RG::KV_BYTES + 16 * lane);
    const uint32_t lb = lds_addr(slot_b + RG::KV_BYTES + 16 * lane);
    half8_t v8[NP][2];
    read_v_pairs<0, NP>(v8, la, lb);
    float4_t sa[NRG], sb[NRG];
    start_scores(sa, sb);
    scores_onto(ra, qf, sa);
    scores_onto(rb, qf, sb);
    half8_t pw[NRG];
    softmax2(sa, sb, pia, pib, grp, masked_a, masked_b, pw);
    lds_wait_operands<NP>(v8);
    values2([&](int pp, int h) __attribute__((always_inline)) { return v8[pp][h]; }, pw);
  }

  __device__ __forceinline__ void start_scores(float4_t (&sa)[NRG], float4_t (&sb)[NRG]) const {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      sa[rg] = float4_t{-base[rg], -base[rg], -base[rg], -base[rg]};
      sb[rg] = sa[rg];
    }
  }

  // Online softmax over a page pair's scores (already relative to base):
  // the f16 weights go to pw, the row sums are updated.
  __device__ __forceinline__ void softmax2(float4_t (&sa)[NRG], float4_t (&sb)[NRG], int pia, int pib,
                                           int grp, bool masked_a, bool masked_b, half8_t (&pw)[NRG]) {
    if (masked_a || masked_b) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (masked_a && pia * 16 + 4 * grp + e > lim[rg]) sa[rg][e] = -INFINITY;
          if (masked_b && pib * 16 + 4 * grp + e > lim[rg]) sb[rg][e] = -INFINITY;
        }
      }
    }
    float lmax[NRG];
    bool over = false;
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const float x = max3f(sa[rg][0], sa[rg][1], sa[rg][2]);
      const float y = max3f(sa[rg][3], sb[rg][0], sb[rg][1]);
      lmax[rg] = max3f(max3f(sb[rg][2], sb[rg][3], x), y, y);
      over = over || lmax[rg] > thr[rg];
    }
    if (__builtin_expect(__any(over), 0)) {
      // (a row group none of whose rows passes its threshold keeps its base:
      // delta 0, alpha 1)
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        float rmax = fmaxf(lmax[rg], __shfl_xor(lmax[rg], 16));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 32));
        const bool grow = rmax > thr[rg];
        const float delta = grow ? ceilf(rmax) : 0.0f;
        const float alpha = (grow && thr[rg] != -INFINITY) ? pow2i(-delta) : 1.0f;
        base[rg] += delta;
        thr[rg] = grow ? kLazyMax : thr[rg];
        sa[rg] -= delta;
        sb[rg] -= delta;
        l4[rg] *= alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t) o[rg][t] *= alpha;
      }
    }
    const half8_t ones = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f,
                          (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      pw[rg] = half8_t{(_Float16)__builtin_amdgcn_exp2f(sa[rg][0]), (_Float16)__builtin_amdgcn_exp2f(sa[rg][1]),
                       (_Float16)__builtin_amdgcn_exp2f(sa[rg][2]), (_Float16)__builtin_amdgcn_exp2f(sa[rg][3]),
                       (_Float16)__builtin_amdgcn_exp2f(sb[rg][0]), (_Float16)__builtin_amdgcn_exp2f(sb[rg][1]),
                       (_Float16)__builtin_amdgcn_exp2f(sb[rg][2]), (_Float16)__builtin_amdgcn_exp2f(sb[rg][3])};
      l4[rg] = MFMA16x16x32(ones, pw[rg], l4[rg]);
    }
  }

  // o += V^T . P^T over a page pair; vf(pp, h) yields the V operand of
  // 16-dim tile 2pp+h (four tokens of each page).
  template <class VF>
  __device__ __forceinline__ void values2(const VF& vf, const half8_t (&pw)[NRG]) {
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const half8_t v8 = vf(pp, h);
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) o[rg][2 * pp + h] = MFMA16x16x32(v8, pw[rg], o[rg][2 * pp + h]);
      }
    }
  }

  // One page with the Q^T operands held in this unit's registers.
  template <bool SPARSE>
  __device__ __forceinline__ void consume(const Regs& r, int pi, int grp, bool masked) {
    consume_with<SPARSE>(r, pi, grp, masked,
                         [&](int rg, int pp) __attribute__((always_inline)) { return qop(rg, pp); });
  }

  // One page: scores relative to base, online softmax, value accumulation.
  // `masked` pages hold positions beyond the unit's smallest visible limit.
  // qf(rg, pp) yields the Q^T operand of row group rg, 32-dim block pp.
  // SPARSE: the static sparse subset may apply (see set_sparse).
  template <bool SPARSE, class QF>
  __device__ __forceinline__ void consume_with(const Regs& r, int pi, int grp, bool masked,
                                               const QF& qf) {
    half4_t pw[NRG];
    score_phase<SPARSE>(r, pi, grp, masked, qf, pw);
    value_phase(r, pw);
  }

  // The same for a page still in its LDS slot: the K half is read for the
  // scores and the V half only after the softmax, so the two halves are
  // never held at once (fewer live registers per wave).
  // `after_k` runs once the K half's reads are issued.
  template <bool SPARSE, class QF, class HOOK>
  __device__ __forceinline__ void consume_slot(const char* slot, int lane, int pi, int grp,
                                               bool masked, const QF& qf, const HOOK& after_k) {
    Regs r;
    read_half<FMT, SF32, D, false>(r, slot, lane, grp);
    after_k();
    half4_t pw[NRG];
    score_phase<SPARSE>(r, pi, grp, masked, qf, pw);
    read_half<FMT, SF32, D, true>(r, slot, lane, grp);
    value_phase(r, pw);
  }

  // Scores of one page (K half of r), online softmax; the f16 weights of
  // the page's 16 positions per row go to pw.
  template <bool SPARSE, class QF>
  __device__ __forceinline__ void score_phase(const Regs& r, int pi, int grp, bool masked,
                                              const QF& qf, half4_t (&pw)[NRG]) {
    // The scores start at -base (exact: base is an integer), so they come
    // out relative to the row bases with no subtraction pass.
    float4_t sacc[NRG];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) sacc[rg] = float4_t{-base[rg], -base[rg], -base[rg], -base[rg]};
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      const half8_t ka = k_operand<FMT, SF32, D>(r, pp);
      if (FMT == kF16) {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
          sacc[rg] = MFMA16x16x32(ka, qf(rg, pp), sacc[rg]);
        }
      } else {
        const float4_t ks = scales4<SF32>(r.ks, pp);
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
          float4_t b = MFMA16x16x32(ka, qf(rg, pp), (float4_t{0, 0, 0, 0}));
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[rg][e] = fmaf(b[e], ks[e], sacc[rg][e]);
        }
      }
    }

    const bool sp = SPARSE && sparse_page(pi);
    const int ph = sp ? sparse_phase(pi * 16 + 4 * grp) : 0;
    // (wave-uniform) the page lies inside every row's strided middle: the
    // lane's four positions are kept exactly where their phase is on the
    // stride, the same for every row group
    const bool inner = sp && pi * 16 >= sp_sink && pi * 16 + 16 <= sp_lo;
    const uint32_t on4 = (sp_on >> ph) & 15u;
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      if (masked) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (pi * 16 + 4 * grp + e > lim[rg]) sacc[rg][e] = -INFINITY;
        }
      }
      if (inner) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (!((on4 >> e) & 1u)) sacc[rg][e] = -INFINITY;
      } else if (sp) {
        sparse_mask(sacc[rg], pi * 16 + 4 * grp, ph, rg);
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
  }

  // Value accumulation of one page (V half of r) with the weights pw.
  __device__ __forceinline__ void value_phase(const Regs& r, const half4_t (&pw)[NRG]) {
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

}  // namespace
}  // namespace tge
