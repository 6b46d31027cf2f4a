// A small decode step in one launch: the step's K/V store, GQA decode
// attention and the split merge (the reference's store-then-attend sequence
// of forward / forward_batch, qwen2.cpp:2073-2095 and 1681-1747, with the
// group kernel and merge_gqa_chunks of qwen2.cpp:1382-1522).
//
// Small steps (one to a few sessions, a few thousand pages) are bound by
// launch and memory latency, not bandwidth: three launches (append, decode,
// merge) cost more than their work, and so does every memory round trip
// one workgroup makes in sequence. Here one workgroup of eight waves takes
// one piece of one (session, KV head) segment (StepRec), a piece being one
// batch of page loads per wave (or a few):
//   1. each wave issues the loads of its first batch of pages straight into
//      registers at once;
//   2. meanwhile the Q^T operands of the unit's rows go to an LDS table;
//      the piece holding the segment's new positions (when the context has
//      several pieces, a piece of just the pages those positions fall in)
//      first stores the new K/V rows of its KV head (the append's own
//      per-lane store, append_common.h, so the bits are those of
//      tge_kv_append), and loads its pages after a workgroup barrier;
//   3. each wave runs the decode unit's math on its pages (attn_common.h:
//      scores on 16x16x32 MFMAs, online softmax with integer row bases,
//      values on 16x16x16 MFMAs), loading further batches if the piece is
//      longer than one;
//   4. the eight waves merge through LDS in a fixed order;
//   5. a one-piece segment writes its output rows; otherwise the piece writes
//      its partial (max, sum, acc) and bumps the segment's arrival counter,
//      and the last piece to arrive merges the segment's partials in slot
//      order (slices of the slots on several threads, then the slices in
//      order), writes the rows and resets the counter for the next launch.
// Results do not depend on which piece arrives last.
//
// Visibility across workgroups (which may sit on different XCDs, each with
// its own L2) uses no agent-scope fence: on gfx950 that fence writes back
// the XCD's whole L2, about a microsecond each, serialised over the XCD's
// workgroups. Instead the partials are written and read with the
// device-coherent cache policy (sc1: written through, and read past, the
// non-coherent L2 copies; what agent-scope relaxed atomics compile to);
// each wave waits for its partial stores to complete before the barrier
// that precedes the counter update, and the last piece reads the partials
// only after the update returned. (AMD's rocPRIM decoupled look-back uses
// the same protocol on gfx942/gfx950.)
#include "append_common.h"
#include "attn_common.h"

namespace tge {
namespace {

template <int FMT, bool SF32, int D, int NRG>
struct StepCfg {
  using R = PageRegs<FMT, SF32, D>;
  // pages a wave loads at once (registers: PB page images beside the unit)
  static constexpr int PB = step_batch_pages(FMT == kI8, SF32, D, NRG);
  static constexpr int ROWS = 16 * NRG;
  static constexpr int SPAD = D + 4;  // staged row stride: rows on different banks
};

template <int FMT, bool SF32, int D, int NRG>
struct StepShared {
  using C = StepCfg<FMT, SF32, D, NRG>;
  alignas(16) half8_t q[NRG * (D / 32) * 64];  // [rg][pp][lane]
  alignas(16) float stage[kStepWaves][16][C::SPAD];
  float m[kStepWaves][C::ROWS];
  float l[kStepWaves][C::ROWS];
  float mm[C::ROWS];
  float sum[C::ROWS];
  int last;
};

// Partials are written and read with the device-coherent cache policy sc1
// (written through, and read past, the XCD's L2): the bits gfx950's
// agent-scope relaxed atomics carry, here on 16- and 8-byte buffer
// accesses (one instruction, one 32-bit offset register each).
constexpr int kCoherent = 16;  // buffer cache-policy operand: sc1
__device__ __forceinline__ void store_partial(__amdgpu_buffer_rsrc_t rs, uint32_t off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rs, off, 0, kCoherent);
}
__device__ __forceinline__ void store_partial(__amdgpu_buffer_rsrc_t rs, uint32_t off, float a, float b) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{__float_as_uint(a), __float_as_uint(b)}, rs, off, 0, kCoherent);
}
__device__ __forceinline__ float4_t load_partial4(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kCoherent));
}
__device__ __forceinline__ float2 load_partial2(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kCoherent);
  return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

// Order-preserving unsigned key of a float (larger float, larger key; every
// key of a non-NaN float is above 0) and its inverse.
__device__ __forceinline__ unsigned order_key(float f) {
  const unsigned b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(unsigned k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

typedef const __attribute__((address_space(4))) StepRec sconst_step;

__device__ __forceinline__ StepRec load_step(const sconst_step* s) {
  const sconst_int* q = (const sconst_int*)s;
  StepRec r;
  r.session = q[0];
  r.kv_head = q[1];
  r.page_begin = q[2];
  r.page_end = q[3];
  r.part = q[4];
  r.seg = q[5];
  r.seg_parts = q[6];
  r.seg_first = q[7];
  r.append = q[8];
  r.ctx = q[9];
  r.n_new = q[10];
  r.q_row = q[11];
  r.table_off = q[12];
  return r;
}

// A page block straight from memory into the lane's registers: the same
// image read_page takes from an LDS slot (piece i of lane l sits at
// i * 1024 + l * 16 in each part; scales as stored).
template <int FMT, bool SF32, int D>
__device__ __forceinline__ void load_page(PageRegs<FMT, SF32, D>& r, const char* block, int lane,
                                          int grp) {
  using RG = Ring<FMT, SF32, D>;
  using R = PageRegs<FMT, SF32, D>;
#pragma unroll
  for (int i = 0; i < RG::PIECES; ++i) {
    const u32x4_t k = *reinterpret_cast<const u32x4_t*>(block + i * 1024 + lane * 16);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(block + RG::KV_BYTES + i * 1024 + lane * 16);
    r.k[4 * i] = k.x; r.k[4 * i + 1] = k.y; r.k[4 * i + 2] = k.z; r.k[4 * i + 3] = k.w;
    r.v[4 * i] = v.x; r.v[4 * i + 1] = v.y; r.v[4 * i + 2] = v.z; r.v[4 * i + 3] = v.w;
  }
  if constexpr (FMT == kI8) {
    const char* sk = block + 2 * RG::KV_BYTES + grp * R::SW * 4;
#pragma unroll
    for (int i = 0; i < R::SW / 4; ++i) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(sk + 16 * i);
      const u32x4_t b = *reinterpret_cast<const u32x4_t*>(sk + RG::SC_BYTES + 16 * i);
      r.ks[4 * i] = a.x; r.ks[4 * i + 1] = a.y; r.ks[4 * i + 2] = a.z; r.ks[4 * i + 3] = a.w;
      r.vs[4 * i] = b.x; r.vs[4 * i + 1] = b.y; r.vs[4 * i + 2] = b.z; r.vs[4 * i + 3] = b.w;
    }
  }
}

// SP: the static sparse subset of p.sp_* applies (attention_head_static_sparse,
// attention_avx2.cpp:263-490: every page is read and the dropped positions
// are masked per row).
template <int FMT, bool SF32, int D, int NRG, bool SP = false>
__global__ __launch_bounds__(64 * kStepWaves) void paged_step_kernel(StepParams p) {
  using C = StepCfg<FMT, SF32, D, NRG>;
  using SH = StepShared<FMT, SF32, D, NRG>;
  static_assert(sizeof(SH::stage) >= sizeof(float) * 2 * kStepMaxParts * 16 * NRG,
                "the merge's (max, sum) table fits the staging area");
  using U = Unit<FMT, SF32, D, NRG>;
  using Regs = typename U::Regs;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;
  constexpr int W = kStepWaves;
  constexpr int PB = C::PB;
  constexpr int QUNIT = NRG * NP * 64;
  __shared__ SH sh;

  const StepRec rec = load_step((const sconst_step*)p.recs + blockIdx.x);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // the first batch's page ids, requested with the record (no dependence on it)
  static_assert(PB * W <= kStepFirstIds, "first-batch ids");
  const sconst_int* fids = (const sconst_int*)(p.first_ids + (size_t)blockIdx.x * kStepFirstIds);
  int first_ids[PB];
#pragma unroll
  for (int i = 0; i < PB; ++i) first_ids[i] = fids[i * W + wave];
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int group = p.group;
  const int kv_heads = p.app.kv_heads;
  const int dims = p.app.dims;  // the head's own dims (rows of q, k, v, out)
  const int kv_dim = kv_heads * dims;
  const int q_stride = p.app.q_heads * dims;
  const int rows = rec.n_new * group;
  // the block geometry is fixed by the kernel's format and head size: taken
  // as constants (no argument load, which the compiler would defer to the
  // first use, costing a memory round trip there)
  AppendParams app = p.app;
  app.geom = block_geom(FMT, D, SF32);
  app.head_dim = D;
  app.scale_f32 = SF32;
  const char* pool = static_cast<const char*>(app.pool);
  const uint32_t bb = (uint32_t)app.geom.block_bytes;
  const sconst_int* table = (const sconst_int*)(p.tables + rec.table_off);
  // the step's partials (byte offsets below 2^31: at most 64 slots per
  // segment and 4096 page blocks per step)
  const auto rs_o = make_rsrc(p.part_o, 0x7fffffff);
  const auto rs_ml = make_rsrc(p.part_ml, 0x7fffffff);
  // ---- the new rows of this KV head (in the piece holding the new
  // positions): the first round's values are requested first, so their
  // round trip overlaps the others
  constexpr int nb = D / 32;
  const int lanes = rec.append ? rec.n_new * 2 * nb * 4 : 0;  // 4 lanes per (row, K|V, 32 values)
  struct Job {
    float x[8];
    RowRec rr;
    int which, b, quarter;
    bool live;  // dead lanes still take part in the shuffles
  };
  const float* const kbase = p.app.k;  // (selected per lane below as values,
  const float* const vbase = p.app.v;  // not by indexing the argument block)
  auto fetch_job = [&](int base, Job& jb) __attribute__((always_inline)) {
    const int idx = base + threadIdx.x;
    jb.live = idx < lanes;
    const int id = jb.live ? idx : lanes - 1;
    jb.quarter = id & 3;
    int rest = id >> 2;
    jb.b = rest % nb;
    rest /= nb;
    jb.which = rest & 1;
    const int j = rest >> 1;
    const int pos = rec.ctx + j;
    jb.rr = RowRec{p.tables[rec.table_off + pos / 16], pos % 16, pos};
    const int d0 = jb.b * 32 + jb.quarter * 8;  // (dims past the head's own store zeros)
    const size_t off = (size_t)(rec.q_row + j) * kv_dim + rec.kv_head * dims;
    if ((dims & 7) == 0) {
      // (the load is issued for every lane, at dim 0 past the head's end)
      load8(jb.x, (jb.which ? vbase : kbase) + off + (d0 < dims ? d0 : 0));
      if (d0 >= dims) {
#pragma unroll
        for (int i = 0; i < 8; ++i) jb.x[i] = 0.0f;
      }
    } else {
      load8_head(jb.x, (jb.which ? vbase : kbase) + off, d0, dims);
    }
  };
  Job job;
  if (lanes > 0) fetch_job(0, job);

  // ---- Q^T operands of the rows (log2(e)/sqrt(D) folded in, f16): the
  // loads first, their conversion into the LDS table after the page loads
  // are on their way (so waiting for Q does not wait for the pages)
  constexpr int QPER = (QUNIT + 64 * W - 1) / (64 * W);
  float4 qa[QPER], qb[QPER];
#pragma unroll
  for (int k = 0; k < QPER; ++k) {
    const int idx = threadIdx.x + k * 64 * W;
    const int l = idx & 63;
    const int blk = idx >> 6;
    const int pp = blk % NP;
    const int rg = blk / NP;
    const int r = rg * 16 + (l & 15);
    const int d = 32 * pp + 4 * (l >> 4);  // (dims past the head's own read as zeros)
    if (idx < QUNIT && r < rows) {
      const int qi = r / group;
      const int head = rec.kv_head * group + r % group;
      const float* qp = p.q + (size_t)(rec.q_row + qi) * q_stride + (size_t)head * dims + d;
      qa[k] = d < dims ? *reinterpret_cast<const float4*>(qp) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      qb[k] = d + 16 < dims ? *reinterpret_cast<const float4*>(qp + 16) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
      qa[k] = qb[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }

  // ---- first batch of pages: wave w takes pages begin+w, begin+w+W, ... ----
  // Every load of the batch is issued, without branches (a page past the
  // piece loads the piece's last page instead and is not used), so the wait
  // for the Q loads issued before them can leave them in flight.
  // The appending piece issues its batch only after the new rows are stored
  // (besides the ordering, a store queued behind the compute unit's batch of
  // page loads waits for the whole batch); the planner keeps that piece to
  // the pages the new rows go to when the context has several pieces.
  const int j0 = rec.page_begin + wave;
  Regs r[PB];
  auto first_batch = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PB; ++i)
      load_page<FMT, SF32, D>(r[i], pool + ((size_t)first_ids[i] * kv_heads + rec.kv_head) * bb, lane,
                              grp);
  };
  // (an appending piece whose first batch ends before the new positions
  // issues it now as well)
  const bool early = !rec.append || rec.page_begin + W * PB <= rec.ctx / 16;
  if (early) first_batch();

#pragma unroll
  for (int k = 0; k < QPER; ++k) {
    const int idx = threadIdx.x + k * 64 * W;
    if (idx < QUNIT) {
      const float c = p.scale_log2;
      const float4 a = qa[k], b = qb[k];
      sh.q[idx] = half8_t{(_Float16)(a.x * c), (_Float16)(a.y * c), (_Float16)(a.z * c), (_Float16)(a.w * c),
                          (_Float16)(b.x * c), (_Float16)(b.y * c), (_Float16)(b.z * c), (_Float16)(b.w * c)};
    }
  }

  if (lanes > 0) {
    for (int base = 0; base < lanes; base += 64 * W) {
      if (base > 0) fetch_job(base, job);
      store_lane<FMT>(app, job.x, job.rr, job.which, rec.kv_head, job.b, job.quarter, job.live);
    }
    __threadfence_block();  // the stored rows before any wave reads their page
  }
  __syncthreads();  // the Q table is written (and the new rows stored)
  if (!early) first_batch();

  // ---- the piece's pages ---------------------------------------------------
  U u;
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    u.lim[rg] = r < rows ? rec.ctx + r / group : -1;
    u.base[rg] = 0.0f;
    u.thr[rg] = -INFINITY;
    u.l4[rg] = float4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] = float4_t{0, 0, 0, 0};
  }
  if constexpr (SP) u.set_sparse(p.sp_sink, p.sp_window, p.sp_stride, rec.ctx + rec.n_new);
  const int unmasked = (rec.ctx + 1) / 16;  // pages every row sees whole
  const half8_t* qt = sh.q + lane;
  auto qf = [&](int rg, int pp) __attribute__((always_inline)) { return qt[(rg * NP + pp) * 64]; };
  for (int jb = j0; jb < rec.page_end; jb += PB * W) {
    if (jb != j0) {
      int ids[PB];
#pragma unroll
      for (int i = 0; i < PB; ++i) ids[i] = table[min(jb + i * W, rec.page_end - 1)];
#pragma unroll
      for (int i = 0; i < PB; ++i)
        load_page<FMT, SF32, D>(r[i], pool + ((size_t)ids[i] * kv_heads + rec.kv_head) * bb, lane, grp);
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const int pi = jb + i * W;
      if (pi < rec.page_end) u.template consume_with<SP>(r[i], pi, grp, pi >= unmasked, qf);
    }
  }

  // ---- merge of the eight waves (fixed order) ------------------------------
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    if (grp == 0) {
      sh.m[wave][rg * 16 + col] = u.thr[rg] == -INFINITY ? -INFINITY : u.base[rg];
      sh.l[wave][rg * 16 + col] = u.l4[rg][0];
    }
  }
  __syncthreads();
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = rg * 16 + col;
    float mm = sh.m[0][r];
#pragma unroll
    for (int k = 1; k < W; ++k) mm = fmaxf(mm, sh.m[k][r]);
    const float mine = sh.m[wave][r];
    const float f = mine == -INFINITY ? 0.0f : pow2i(mine - mm);
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] *= f;
    if (wave == 0 && grp == 0) {
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const float mk = sh.m[k][r];
        if (mk != -INFINITY) sum += sh.l[k][r] * pow2i(mk - mm);
      }
      sh.mm[r] = mm;
      sh.sum[r] = sum;
    }
  }
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    float* dst = &sh.stage[wave][col][4 * grp];
#pragma unroll
    for (int t = 0; t < NT; ++t) *reinterpret_cast<float4_t*>(dst + 16 * t) = u.o[rg][t];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 16 * (D / 4); idx += 64 * W) {
      const int rr = idx / (D / 4);
      const int d4 = idx % (D / 4);
      const int r = rg * 16 + rr;
      float4_t acc = float4_t{0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < W; ++k) acc += *reinterpret_cast<const float4_t*>(&sh.stage[k][rr][4 * d4]);
      if (r < rows) {
        const float sum = sh.sum[r];
        if (rec.part < 0) {
          const int qi = r / group;
          const int head = rec.kv_head * group + r % group;
          float4_t res = float4_t{0, 0, 0, 0};
          if (sum > 0.0f) res = div4(acc, sum);
          if (4 * d4 < dims)
            *reinterpret_cast<float4_t*>(p.out + (size_t)(rec.q_row + qi) * q_stride + (size_t)head * dims +
                                         4 * d4) = res;
        } else {
          const uint32_t slot_row = (uint32_t)rec.part * p.rows_cap + r;
          store_partial(rs_o, (slot_row * D + 4 * d4) * 4, acc);
          if (d4 == 0) store_partial(rs_ml, slot_row * 8, sh.mm[r], sum);
        }
      }
    }
    __syncthreads();  // the staging area is free again
  }
  if (rec.part < 0) return;

  // ---- split segment: the last piece to arrive merges ---------------------
  if (threadIdx.x < C::ROWS) reinterpret_cast<unsigned*>(sh.mm)[threadIdx.x] = 0u;  // below every key
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  wait_vmcnt<0>();  // this wave's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev =
        __hip_atomic_fetch_add(p.counters + rec.seg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.last = prev == rec.seg_parts - 1;
  }
  __syncthreads();
  if (!sh.last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // merge_gqa_chunks over the segment's partials (pieces with no visible
  // position are skipped, none at all gives zeros):
  //   A. every slot's (max, sum) of every row into LDS, while the first
  //      accumulators are already on their way; each row's common base M
  //      (the largest max) by an LDS max over order-preserving integer keys;
  //   B. `slices` threads share each (row, 4 dims): slice s adds, slots
  //      [s*n/slices, (s+1)*n/slices) in order, each slot's accumulator and
  //      sum weighted by 2^(max - M) (MC loads in flight per thread); the
  //      slices are then added in order and the sum divides.
  constexpr int D4 = D / 4;
  constexpr int MC = NRG == 1 ? 20 : 8;
  const int n = rec.seg_parts;
  const int pairs = rows * D4;
  const int slices = max(1, min(n, (64 * W) / max(pairs, 1)));
  float* wml = &sh.stage[0][0][0];  // [n][rows] of (max, sum)
  unsigned* key = reinterpret_cast<unsigned*>(sh.mm);  // [rows] largest max, as a key
  for (int idx0 = 0; idx0 < slices * pairs; idx0 += 64 * W) {
    const int idx = idx0 + threadIdx.x;
    const bool act = idx < slices * pairs;
    const int sl = act ? idx / pairs : 0;
    const int pair = act ? idx - sl * pairs : 0;
    const int r = pair / D4;
    const int d4 = pair - r * D4;
    const int kb = act ? sl * n / slices : 0, ke = act ? (sl + 1) * n / slices : 0;
    float4_t v[MC];
    // slots past the slice reload its last slot (weight 0); no branches, so
    // every load is in flight at once
    auto fetch = [&](int k0) __attribute__((always_inline)) {
      if (ke > kb) {
#pragma unroll
        for (int i = 0; i < MC; ++i) {
          const int k = min(k0 + i, ke - 1);
          v[i] = load_partial4(rs_o, (((uint32_t)(rec.seg_first + k) * p.rows_cap + r) * D + 4 * d4) * 4);
        }
      } else {
#pragma unroll
        for (int i = 0; i < MC; ++i) v[i] = float4_t{0, 0, 0, 0};
      }
    };
    fetch(kb);
    if (idx0 == 0) {
      for (int i = threadIdx.x; i < n * rows; i += 64 * W) {
        const int k = i / rows;
        const float2 x = load_partial2(rs_ml, ((uint32_t)(rec.seg_first + k) * p.rows_cap + (i - k * rows)) * 8);
        wml[2 * i] = x.x;
        wml[2 * i + 1] = x.y;
        if (x.y > 0.0f) atomicMax(key + (i - k * rows), order_key(x.x));
      }
      __syncthreads();
    }
    const unsigned kr = key[r];
    const float mx = kr == 0u ? -INFINITY : key_value(kr);
    float4_t acc = float4_t{0, 0, 0, 0};
    float sum = 0.0f;
    for (int k0 = kb; k0 < ke; k0 += MC) {
      if (k0 != kb) fetch(k0);
      float m[MC], l[MC];
#pragma unroll
      for (int i = 0; i < MC; ++i) {
        const float2 e = *reinterpret_cast<const float2*>(wml + 2 * (min(k0 + i, ke - 1) * rows + r));
        m[i] = e.x;
        l[i] = e.y;
      }
#pragma unroll
      for (int i = 0; i < MC; ++i) {
        const float w = k0 + i < ke && l[i] > 0.0f ? pow2i(m[i] - mx) : 0.0f;
        acc += v[i] * w;
        sum += l[i] * w;
      }
    }
    if (slices == 1) {
      if (act) {
        const int qi = r / group;
        const int head = rec.kv_head * group + r % group;
        float4_t res = float4_t{0, 0, 0, 0};
        if (sum > 0.0f) res = div4(acc, sum);
        if (4 * d4 < dims)
          *reinterpret_cast<float4_t*>(p.out + (size_t)(rec.q_row + qi) * q_stride + (size_t)head * dims + 4 * d4) = res;
      }
    } else {
      // one pass (slices * pairs <= the workgroup): park the slice sums
      __syncthreads();  // every (max, sum) has been read
      if (act) {
        float* e = wml + 8 * (size_t)idx;
        *reinterpret_cast<float4_t*>(e) = acc;
        e[4] = sum;
      }
      __syncthreads();
      for (int pr = threadIdx.x; pr < pairs; pr += 64 * W) {
        const int rr = pr / D4;
        const int dd = pr - rr * D4;
        float4_t a = float4_t{0, 0, 0, 0};
        float su = 0.0f;
        for (int k = 0; k < slices; ++k) {
          const float* e = wml + 8 * (size_t)(k * pairs + pr);
          a += *reinterpret_cast<const float4_t*>(e);
          su += e[4];
        }
        const int qi = rr / group;
        const int head = rec.kv_head * group + rr % group;
        float4_t res = float4_t{0, 0, 0, 0};
        if (su > 0.0f) res = div4(a, su);
        if (4 * dd < dims)
          *reinterpret_cast<float4_t*>(p.out + (size_t)(rec.q_row + qi) * q_stride + (size_t)head * dims + 4 * dd) = res;
      }
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(p.counters + rec.seg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

template <int FMT, bool SF32, int D, bool SP>
hipError_t launch_step_v(int row_groups, int n, const StepParams& p, hipStream_t st) {
  const dim3 grid((unsigned)n), block(64 * kStepWaves);
  // variants that would spill are not built (step_fits keeps the planner
  // from asking for them)
  constexpr bool I8 = FMT == kI8;
  switch (row_groups) {
    case 1:
      if constexpr (step_fits(I8, SF32, D, 16, SP)) {
        hipLaunchKernelGGL((paged_step_kernel<FMT, SF32, D, 1, SP>), grid, block, 0, st, p);
        break;
      }
      return hipErrorInvalidValue;
    case 2:
      if constexpr (step_fits(I8, SF32, D, 32, SP)) {
        hipLaunchKernelGGL((paged_step_kernel<FMT, SF32, D, 2, SP>), grid, block, 0, st, p);
        break;
      }
      return hipErrorInvalidValue;
    case 3:
      if constexpr (step_fits(I8, SF32, D, 48, SP)) {
        hipLaunchKernelGGL((paged_step_kernel<FMT, SF32, D, 3, SP>), grid, block, 0, st, p);
        break;
      }
      return hipErrorInvalidValue;
    case 4:
      if constexpr (step_fits(I8, SF32, D, 64, SP)) {
        hipLaunchKernelGGL((paged_step_kernel<FMT, SF32, D, 4, SP>), grid, block, 0, st, p);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int FMT, bool SF32, int D>
hipError_t launch_step_d(int row_groups, int n, const StepParams& p, hipStream_t st) {
  return p.sp_stride > 0 ? launch_step_v<FMT, SF32, D, true>(row_groups, n, p, st)
                         : launch_step_v<FMT, SF32, D, false>(row_groups, n, p, st);
}

hipError_t launch_step(int format, int scale_f32, int head_dim, int row_groups, int n_recs,
                       const StepParams& p, hipStream_t stream) {
  if (n_recs <= 0) return hipSuccess;
  if (format == kF16) {
    if (head_dim == 64) return launch_step_d<kF16, false, 64>(row_groups, n_recs, p, stream);
    if (head_dim == 128) return launch_step_d<kF16, false, 128>(row_groups, n_recs, p, stream);
    if (head_dim == 256) return launch_step_d<kF16, false, 256>(row_groups, n_recs, p, stream);
  } else if (format == kI8) {
    if (head_dim == 64)
      return scale_f32 ? launch_step_d<kI8, true, 64>(row_groups, n_recs, p, stream)
                       : launch_step_d<kI8, false, 64>(row_groups, n_recs, p, stream);
    if (head_dim == 128)
      return scale_f32 ? launch_step_d<kI8, true, 128>(row_groups, n_recs, p, stream)
                       : launch_step_d<kI8, false, 128>(row_groups, n_recs, p, stream);
    if (head_dim == 256)
      return scale_f32 ? launch_step_d<kI8, true, 256>(row_groups, n_recs, p, stream)
                       : launch_step_d<kI8, false, 256>(row_groups, n_recs, p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace tge
