// Paged GQA attention on CDNA4 matrix cores: decode (one or a few new tokens
// per session, split-K over long contexts) and chunked prefill (a query tile
// against every prior page).
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
// Work unit: one session, one KV head, up to 16*NRG query rows, a range of
// logical pages. Rows are (query, head) pairs: decode packs the whole GQA
// group of every new token into the rows (each K/V page block is fetched
// once for the group), prefill packs the query group of consecutive
// queries. A page block (16 tokens of one KV head: K, V and int8 scales, one
// contiguous run of HBM) is fetched straight into LDS by 16-byte
// buffer_load ... lds instructions, each covering a contiguous KiB (piece i
// of every lane; layout in tge_common.h), and read back into the lane's MFMA
// operand registers.
//
// Per page, per 16-row group, per wave (lane = group g 0..3, column c 0..15):
//   S^T[token][row] = K (16 x D) . Q^T: one v_mfma_f32_16x16x32_f16 per 32-dim
//     block, Q rounded to f16 once;
//     int8 codes are exact in f16 and the block's per-token scale multiplies
//     the block's fp32 partial score. Lane (g, c) then holds row c,
//     tokens 4g..4g+3.
//   online softmax per row in the log2 domain; the row base only moves when
//     a score exceeds it by more than 2^8, so the accumulators are rescaled
//     rarely (weights stay <= 256, exact enough in f16).
//   O^T[dim][row] += V^T (D x 16) . P^T: v_mfma_f32_16x16x16_f16 per 16-dim
//     tile; lane (g, c) holds row c, dims 16j+4g..+3, the same row as its
//     softmax state. int8 V is dequantised in f16 (exact code times the f16
//     scale, one rounding).
// Waves that shared a unit merge through LDS in a fixed order (the output
// is bit-reproducible); units of a split context write partial
// (max, sum, acc) for the reduction kernel.

#include "append_common.h"
#include "attn_common.h"

namespace tge {

// Bounded waits inside the kernels (half_barrier) that ran out since the
// process started: a launch during which one expired may have wrong rows.
__device__ unsigned int g_wait_expired;

namespace {

// ---------------------------------------------------------------------------
// Decode kernel: persistent workgroups of W waves (DecodeCfg: 4 waves, two
// workgroups per CU for up to 32 rows per unit), each covering a contiguous
// share of the plan's page sequence (its work items in order).
//
// Within a unit the waves take pages round-robin (wave w: the unit's pages
// j with (j + item) mod W = w, item the unit's index in the plan, so the
// last pages of a share's units spread over the waves; with a static sparse
// subset that skips pages, the unit's kept pages, from wave 0). Each wave streams its pages through a private LDS ring of NB
// slots (NB-1 page blocks in flight while it consumes one) and crosses unit
// boundaries without draining: the next unit's first pages are already in
// flight while the current unit is merged. The Q^T operands of the share's
// units sit in an LDS table (f16, read per page), so no vector-memory wait
// for Q stalls the ring. A unit ends for a wave when its next page belongs
// to a later unit (or the share is exhausted); the W waves then merge their
// states for that unit in wave order, so every wave passes the same
// barriers. The page split is fixed by the plan, so results are
// bit-reproducible.
// ---------------------------------------------------------------------------
constexpr int kLdsBytes = 160 * 1024;  // LDS of one CU (gfx950)

#ifndef TGE_DECODE_WAVES
#define TGE_DECODE_WAVES 4
#endif
// Waves per SIMD of the dense decode kernel. A plain LDS-DMA ring over the
// c5 block pattern streams ~5.95 TB/s with three (twelve waves per CU)
// against ~5.4 with two, and the dense kernel fits the 168 registers three
// allow; but the whole kernel measured the same at three (132.4 against
// 131.5 us per c5 launch: the extra speed goes to cross-XCD imbalance that
// changes from launch to launch) while cutting a third more split partials.
// The static sparse variant stays at two in any case (its extra per-row
// state would spill at three).
#ifndef TGE_DECODE_WPE
#define TGE_DECODE_WPE 2
#endif
#ifndef TGE_DECODE_WPE_SPARSE
#define TGE_DECODE_WPE_SPARSE 2
#endif
#ifndef TGE_DECODE_MAX_SLOTS
#define TGE_DECODE_MAX_SLOTS 4
#endif

// Launch shape of a decode variant: W waves per workgroup at WPE waves per
// SIMD (PER_CU = 4*WPE/W workgroups per CU), NB ring slots per wave, and the
// Q^T operands of up to MAXU units resident in LDS.
// MIX: the decode role of the mixed-step kernel (paged_mixed_kernel below):
// always four waves (its workgroups are also block-prefill tiles of 256
// threads) at two per SIMD (one for more than 32 rows).
template <int FMT, bool SF32, int D, int NRG, bool SP = false, bool MIX = false>
struct DecodeCfg {
  static constexpr int WANT = SP ? TGE_DECODE_WPE_SPARSE : TGE_DECODE_WPE;
  static constexpr int SLOT = Ring<FMT, SF32, D>::SLOT;
  static constexpr int ROWS = 16 * NRG;
  static constexpr int QBYTES = NRG * (D / 32) * 64 * 16;  // one unit's Q^T operands (f16)
  static constexpr int merge_bytes(int w) { return 4 * (2 * w * ROWS + 2 * ROWS + w); }
  // Ring slots per wave that fit a workgroup of w waves at wpe waves per
  // SIMD, next to its merge area and one unit's Q^T operands.
  static constexpr int nb_fit(int w, int wpe) {
    return (kLdsBytes / (4 * wpe / w > 1 ? 4 * wpe / w : 1) - 256 - merge_bytes(w) - QBYTES) / (w * SLOT);
  }
  // More than 32 rows need a whole SIMD's registers per wave; otherwise the
  // configured shape, or eight waves at two per SIMD when its rings do not
  // fit (f16 pages at head_dim 128).
  static constexpr bool kBig = NRG > 2 || D > 128;  // (256-dim pages: 16 KB each)
  static constexpr bool kFits = nb_fit(TGE_DECODE_WAVES, WANT) >= 2;
  static constexpr int W = MIX ? 4 : (kBig ? 4 : (kFits ? TGE_DECODE_WAVES : 8));
  static constexpr int WPE = kBig ? 1 : (MIX ? 2 : (kFits ? WANT : 2));
  static constexpr int PER_CU = 4 * WPE / W > 1 ? 4 * WPE / W : 1;  // workgroups per CU
  static constexpr int LDS = kLdsBytes / PER_CU - 256;             // one workgroup's share
  static constexpr int NB = nb_fit(W, WPE) > TGE_DECODE_MAX_SLOTS ? TGE_DECODE_MAX_SLOTS : nb_fit(W, WPE);
  static constexpr int LEFT = LDS - merge_bytes(W) - W * NB * SLOT;
  static constexpr int MAXU = LEFT / QBYTES > 4 ? 4 : LEFT / QBYTES;
  static_assert(NB >= 2 && MAXU >= 1, "decode LDS plan");
  static_assert((W & (W - 1)) == 0, "the page split takes indices mod W");
  // The dense variants of up to 128 dims and 32 rows per unit can store a
  // decode step's new rows (their register budget holds a wave's encoded
  // rows through the page loop); rows per wave they hold: APP_ROWS.
  static constexpr bool kApp = !SP && !MIX && !kBig;
  static constexpr int APP_ROWS = decode_app_rows(D);
  // a merge pass stages 8 rows of D floats (row stride D+4) in one ring slot
  static_assert(8 * (D + 4) * 4 <= SLOT, "merge staging fits a slot");
};

template <int FMT, bool SF32, int D, int NRG, bool SP, bool MIX = false>
struct DecodeShared {
  using C = DecodeCfg<FMT, SF32, D, NRG, SP, MIX>;
  static constexpr int ROWS = 16 * NRG;
  static constexpr int MERGE_FLOATS = 2 * C::W * ROWS + 2 * ROWS + C::W;
  alignas(16) char ring[C::W * C::NB * C::SLOT];
  alignas(16) half8_t q[C::MAXU * NRG * (D / 32) * 64];  // [unit][rg][pp][lane]
  alignas(16) float merge[MERGE_FLOATS];
  int flag;  // arrival broadcast of the in-kernel split merge
};

// Wait for this wave's outstanding LDS and scalar-memory operations; a
// compiler barrier for memory accesses.
__device__ __forceinline__ void lgkm_wait_all() {
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0) only
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Workgroup barrier ordering LDS only: this wave's LDS accesses complete,
// then all waves meet. Direct-to-LDS page loads stay in flight across it
// (they fill the wave's own ring, which no other wave reads); the
// __syncthreads fence would wait for them.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}


// Share indices of the pages in a wave's ring, oldest first (a FIFO of at
// most N wave-uniform values; the constant-index loops keep it in scalar
// registers).
template <int N>
struct PageFifo {
  int t[N];
  __device__ __forceinline__ PageFifo() {
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = 0;
  }
  __device__ __forceinline__ void push(int n, int g) {  // n = entries before the push
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = n == i ? g : t[i];
  }
  __device__ __forceinline__ void pop() {
#pragma unroll
    for (int i = 0; i + 1 < N; ++i) t[i] = t[i + 1];
  }
  __device__ __forceinline__ int front() const { return t[0]; }
};

// Write one lane's encoded values (write_lane's pieces) into a landed page's
// ring slot, which holds the block in its memory layout: `offs` = block byte
// offsets (bits 0-15: the K run or first V element, 16 up: the scale),
// `rest` = the lane's index within its row. A K row's second run of 4 dims
// belongs to the lane 16 further on (256 bytes on in its piece), a V row's
// next dim to the next lane (16 bytes on).
template <int FMT, bool SF32, int D>
__device__ __forceinline__ void patch_slot(char* slot, const LaneCodes& c, int offs, int rest, int np) {
  char* const d = slot + (offs & 0xffff);
  if ((rest >> 2) / np == 0) {  // K
    if (FMT == kF16) {
      *reinterpret_cast<uint2*>(d) = make_uint2(c.w[0], c.w[1]);
      *reinterpret_cast<uint2*>(d + 256) = make_uint2(c.w[2], c.w[3]);
    } else {
      *reinterpret_cast<uint32_t*>(d) = c.w[0];
      *reinterpret_cast<uint32_t*>(d + 256) = c.w[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (FMT == kF16)
        *reinterpret_cast<uint16_t*>(d + 16 * i) = (uint16_t)(c.w[i >> 1] >> (16 * (i & 1)));
      else
        *reinterpret_cast<uint8_t*>(d + 16 * i) = (uint8_t)(c.w[i >> 2] >> (8 * (i & 3)));
    }
  }
  if (FMT != kF16 && (rest & 3) == 0) {
    char* const s = slot + (offs >> 16);
    if (SF32)
      *reinterpret_cast<uint32_t*>(s) = __float_as_uint(c.scale);
    else
      *reinterpret_cast<uint16_t*>(s) = float_to_half_ref(c.scale);
  }
}

// SKIP (static sparse, stride > 16 only): pages holding no kept position
// are never fetched. For strides of 16 or less every page holds one; that
// variant leaves the kept-page enumeration out of its issue path (with it
// compiled in, the c5 step at stride 4 took 1.22x the dense kernel's time,
// without 1.08x).
template <int FMT, bool SF32, int D, int NRG, int W, int WPE, bool SP, bool MIX, bool APP = false,
          bool SKIP = false>
__device__ __forceinline__ void decode_body(const AttnParams& p,
                                            DecodeShared<FMT, SF32, D, NRG, SP, MIX>& sh,
                                            const int group) {
  using CFG = DecodeCfg<FMT, SF32, D, NRG, SP, MIX>;
  using U = Unit<FMT, SF32, D, NRG>;
  using RG = Ring<FMT, SF32, D>;
  static_assert(CFG::W == W && CFG::WPE == WPE, "launch shape");
  constexpr int NB = CFG::NB;
  constexpr int MAXU = CFG::MAXU;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;
  constexpr int ROWS = 16 * NRG;
  constexpr int QUNIT = NRG * NP * 64;  // half8 entries of one unit's Q^T

  const int first = p.wg_first[group];
  const int last = p.wg_first[group + 1];
  if (first >= last) return;  // the whole workgroup leaves together

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  const sconst_work* work = (const sconst_work*)p.work;
  const int q_stride = p.q_heads * p.dims;

  char* ring = sh.ring + wave * NB * RG::SLOT;

  // ---- the step's new K/V rows (APP: the launch of tge_decode_step) --------
  // Each wave handles the new rows of the pages it reads itself (the plan
  // lists them per wave, at most APP_ROWS): their values are loaded beside
  // the Q table and encoded as the append encodes them; when such a page
  // lands in the ring, the wave writes the rows into the slot before reading
  // it (the page in memory does not hold them yet); after its last page the
  // wave stores them into the pool. No other wave or workgroup reads those
  // pages in this launch. Row r takes RL lanes: four per 32-value block of
  // the K row, then of the V row (encode_lane's lane order).
  constexpr bool kApp = APP;
  static_assert(!APP || CFG::kApp, "a variant that stores new rows");
  constexpr int RL = 8 * NP;
  constexpr int RJ = 64 / RL;                         // rows per 64-lane job
  constexpr int AJ = kApp ? CFG::APP_ROWS / RJ : 1;  // jobs
  static_assert(CFG::APP_ROWS <= kAppPad && CFG::APP_ROWS % RJ == 0, "app rows");
  // A job's state through the page loop: the encoded values, the lane's
  // slot offsets (K: first run, the second 256 bytes on; V: first element,
  // the next ones 16 bytes apart; bits 16 up: the scale, quarter-0 lanes)
  // and the row's key (work item << 16 | its page mod 2^16; -1: no row).
  struct AppJob {
    LaneCodes c;
    int offs;
    int key;
  };
  AppJob jobs[AJ];
#pragma unroll
  for (int a = 0; a < AJ; ++a) jobs[a].key = -1;
  int app_n = 0, app_off = 0;  // this wave's rows, its first record
  int arec[kApp ? CFG::APP_ROWS * kAppRecInts : 1];
  auto read_recs = [&]() __attribute__((always_inline)) -> void {
    // (records past the wave's own are the next wave's, or the zero padding
    // after the last list: never used)
    const sconst_int* rec = (const sconst_int*)p.app_recs + (size_t)app_off * kAppRecInts;
#pragma unroll
    for (int e = 0; e < (kApp ? CFG::APP_ROWS * kAppRecInts : 1); ++e) arec[e] = rec[e];
  };
  // record field e of the lane's row in job a
  auto rec_field = [&](int a, int e) __attribute__((always_inline)) -> int {
    int v = arec[(a * RJ) * kAppRecInts + e];
#pragma unroll
    for (int c = 1; c < RJ; ++c) v = lane / RL == c ? arec[(a * RJ + c) * kAppRecInts + e] : v;
    return v;
  };
  if constexpr (kApp) {
    // (read at kernel start: the scalar round trips end before the page ids
    // of the first fetches return)
    const sconst_int* af = (const sconst_int*)p.app_first + group * W + wave;
    app_off = af[0];
    app_n = af[1] - app_off;
    read_recs();
  }

  // ---- Q^T operands of units [qfirst, qfirst + MAXU) in LDS ----------------
  // Entry (u, rg, pp, l): lane l = 16g + c of row group rg holds row c, dims
  // {32pp+4g+e, 32pp+16+4g+e}, pre-multiplied by log2(e)/sqrt(D), in f16.
  // Each block of 64 entries is one wave's, so the unit is wave-uniform.
  int qfirst = first;
  auto fill_q = [&](int from) __attribute__((always_inline)) -> void {
    for (int idx = threadIdx.x; idx < MAXU * QUNIT; idx += 64 * W) {
      const int l = idx & 63;
      const int blk = __builtin_amdgcn_readfirstlane(idx >> 6);
      const int pp = blk % NP;
      const int rg = (blk / NP) % NRG;
      const int it = from + blk / (NP * NRG);
      half8_t h = {};
      if (it < last) {
        const WorkRec w = load_work(work + it);
        const int r = rg * 16 + (l & 15);
        if (r < w.rows) {
          const int qi = w.row_begin + r / w.rows_per_query;
          const int head = w.head_base + r % w.rows_per_query;
          const int d = 32 * pp + 4 * (l >> 4);  // (dims past the head's own read as zeros)
          const float* qp = p.q + (size_t)(w.q_row + qi) * q_stride + (size_t)head * p.dims + d;
          const float4 z = make_float4(0, 0, 0, 0);
          const float4 a = d < p.dims ? *reinterpret_cast<const float4*>(qp) : z;
          const float4 b = d + 16 < p.dims ? *reinterpret_cast<const float4*>(qp + 16) : z;
          const float c = p.scale_log2;
          h = half8_t{(_Float16)(a.x * c), (_Float16)(a.y * c), (_Float16)(a.z * c), (_Float16)(a.w * c),
                      (_Float16)(b.x * c), (_Float16)(b.y * c), (_Float16)(b.z * c), (_Float16)(b.w * c)};
        }
      }
      sh.q[idx] = h;
    }
  };
  // The same at kernel start, with every load of the table issued before
  // any is used (one memory round trip instead of one per pass); rows past
  // a unit's end read its row 0 (always present) and store zeros.
  auto fill_q_start = [&](int from) __attribute__((always_inline)) -> void {
    constexpr int TOTAL = MAXU * QUNIT;
    constexpr int PER = (TOTAL + 64 * W - 1) / (64 * W);
    float4 qa[PER], qb[PER];
    bool ok[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int idx = threadIdx.x + k * 64 * W;
      const int l = idx & 63;
      const int blk = __builtin_amdgcn_readfirstlane(idx >> 6);
      const int pp = blk % NP;
      const int rg = (blk / NP) % NRG;
      const int it = from + blk / (NP * NRG);
      const bool in = idx < TOTAL && it < last;
      const WorkRec w = load_work(work + (in ? it : from));
      const int r = rg * 16 + (l & 15);
      ok[k] = in && r < w.rows;
      const int rr = ok[k] ? r : 0;
      const int qi = w.row_begin + rr / w.rows_per_query;
      const int head = w.head_base + rr % w.rows_per_query;
      const int d = 32 * pp + 4 * (l >> 4);  // (dims past the head's own read as zeros)
      const float* qp = p.q + (size_t)(w.q_row + qi) * q_stride + (size_t)head * p.dims + d;
      qa[k] = d < p.dims ? *reinterpret_cast<const float4*>(qp) : make_float4(0, 0, 0, 0);
      qb[k] = d + 16 < p.dims ? *reinterpret_cast<const float4*>(qp + 16) : make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int idx = threadIdx.x + k * 64 * W;
      if (idx < TOTAL) {
        const float c = p.scale_log2;
        const float4 a = qa[k], b = qb[k];
        const half8_t h = {(_Float16)(a.x * c), (_Float16)(a.y * c), (_Float16)(a.z * c), (_Float16)(a.w * c),
                           (_Float16)(b.x * c), (_Float16)(b.y * c), (_Float16)(b.z * c), (_Float16)(b.w * c)};
        sh.q[idx] = ok[k] ? h : half8_t{};
      }
    }
  };

  // ---- issue side: this wave's next page, its block, its fetch -------------
  // Cursor over the share's units: unit `ik` covers share pages
  // [ibase, ibase + its page count); `jn` is this wave's next page in it
  // (wave w takes the unit's pages j = w - ik, w - ik + W, ... mod W: a
  // fixed split, so results are bit-reproducible and independent of where
  // the pages sit).
  int ik = first, ibase = 0, jn = (wave - first) & (W - 1);
  WorkRec iw = load_work(work + first);
  WorkRec iw_next = load_work(work + (first + 1 < last ? first + 1 : first));
  // Next page to fetch: share index (-1: none), page id and KV head. The id
  // is used only at the next fetch, so its scalar load is waited for there.
  int pend_g = -1, pend_id = 0, pend_head = 0;
  // Static sparse subsets with stride > 16 leave whole pages with nothing
  // kept for any row of a unit; those are never fetched. The unit's kept
  // pages are, in order: A, the pages holding a sink position; M, the pages
  // wholly inside every row's strided middle that hold a stride position
  // (one per stride step k: page (sink + k*stride)/16, since stride > 16);
  // C, the pages from the first row's window start on (row 0 has the
  // unit's smallest span). The waves split the kept ordinals round-robin
  // (wave w takes w, w+W, ...), so a periodic skip pattern never leaves
  // one wave all the work.
  static_assert(!SKIP || SP, "page skipping is a static sparse variant");
  const bool skipping = SKIP && p.sp_stride > 16;
  int ka0 = 0, kna = 0, kk0 = 0, knm = 0, kc0 = 0, knc = 0;  // A start/count, M first k/count, C
  auto kept_geometry = [&](const WorkRec& w) __attribute__((always_inline)) -> void {
    const int pb = w.page_begin, pe = w.page_end;
    const int span0 = w.ctx + w.row_begin + 1;
    const int mid0 = span0 > p.sp_sink + p.sp_window ? span0 - p.sp_window : p.sp_sink;
    const int ma = (p.sp_sink + 15) >> 4;    // pages below hold a sink position
    const int mb = max(ma, mid0 >> 4);       // pages from here reach row 0's window
    ka0 = pb;
    kna = max(0, min(pe, ma) - pb);
    const int lo = max(pb, ma), hi = min(pe, mb);
    knm = 0;
    if (hi > lo) {
      kk0 = (16 * lo - p.sp_sink + p.sp_stride - 1) / p.sp_stride;
      knm = (16 * hi - p.sp_sink + p.sp_stride - 1) / p.sp_stride - kk0;
    }
    kc0 = max(pb, mb);
    knc = max(0, pe - kc0);
  };
  auto kept_page = [&](int o) __attribute__((always_inline)) -> int {  // session page of ordinal o
    if (o < kna) return ka0 + o;
    o -= kna;
    if (o < knm) return (p.sp_sink + (kk0 + o) * p.sp_stride) >> 4;
    return kc0 + (o - knm);
  };
  int ko = wave;  // next kept ordinal of this wave in the issue unit
  if (skipping) kept_geometry(iw);
  auto request = [&]() __attribute__((always_inline)) -> void {
    bool ok = true;
    if (skipping) {
      while (ko >= kna + knm + knc) {
        if (ik + 1 >= last) {
          ok = false;
          break;
        }
        ibase += iw.page_end - iw.page_begin;
        ++ik;
        iw = iw_next;
        iw_next = load_work(work + (ik + 1 < last ? ik + 1 : ik));
        kept_geometry(iw);
        ko = wave;
      }
      jn = ok ? kept_page(ko) - iw.page_begin : 0;
      ko += W;
    } else {
      while (ok && jn >= iw.page_end - iw.page_begin) {
        if (ik + 1 >= last) {
          ok = false;  // past the share: the cursor stays on its last unit
        } else {
          ibase += iw.page_end - iw.page_begin;
          ++ik;
          jn = (wave - ik) & (W - 1);
          iw = iw_next;
          iw_next = load_work(work + (ik + 1 < last ? ik + 1 : ik));
        }
      }
    }
    // (index 0 when past the share keeps the table read inside the unit)
    const sconst_int* t = (const sconst_int*)(p.tables + iw.table_off + iw.page_begin);
    const int id = t[ok ? jn : 0];
    pend_g = ok ? ibase + jn : -1;
    pend_id = id;
    pend_head = iw.kv_head;
    if (!skipping) jn += W;
  };
  // Fetch the pending page into `slot`; returns the fetched page's share
  // index, or -1 when the share is exhausted. The caller then takes the
  // next page with request().
  auto issue = [&](int slot) __attribute__((always_inline)) -> int {
    const int g = pend_g;
    if (g >= 0) {
      const char* blk = static_cast<const char*>(p.pool) +
                        ((size_t)pend_id * p.kv_heads + pend_head) * p.block_bytes;
      fetch_page<FMT, SF32, D>(ring + slot * RG::SLOT, blk, p.block_bytes, lane);
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
    u.set_sparse(p.sp_sink, p.sp_window, p.sp_stride,
                 cw.ctx + cw.row_begin + (cw.rows - 1) / cw.rows_per_query + 1);
  };
  // Merge the W waves' states of unit `cw` and write the output rows (or the
  // unit's partial). Every wave calls this once per unit, at a point where
  // its ring has a free slot (slot `fs`: the ring holds `count` < NB pages).
  //   1. each wave publishes its rows' (base, sum) and its free slot; wave 0
  //      derives each row's common base and total sum; each wave rescales
  //      its accumulators to the common base;
  //   2. in passes of 8 rows, each wave stages its accumulators for those
  //      rows in its free slot, then the workgroup's threads add the W
  //      copies in wave order (a fixed order: results do not depend on
  //      timing) and write the rows out.
  constexpr int PASS_ROWS = 8;
  float* mbase = sh.merge;
  float (*lds_m)[ROWS] = reinterpret_cast<float (*)[ROWS]>(mbase);
  float (*lds_l)[ROWS] = reinterpret_cast<float (*)[ROWS]>(mbase + W * ROWS);
  float* lds_mm = mbase + 2 * W * ROWS;  // [ROWS] common base
  float* lds_sum = lds_mm + ROWS;         // [ROWS] total sum
  int* lds_fs = reinterpret_cast<int*>(lds_sum + ROWS);  // [W] free ring slot of each wave
  auto finalize = [&](int fs) __attribute__((always_inline)) -> void {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      if (grp == 0) {
        lds_m[wave][rg * 16 + col] = u.thr[rg] == -INFINITY ? -INFINITY : u.base[rg];
        lds_l[wave][rg * 16 + col] = u.l4[rg][0];
      }
    }
    if (lane == 0) lds_fs[wave] = fs;
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
      if (wave == 0 && grp == 0) {
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const float mk = lds_m[k][r];
          if (mk != -INFINITY) sum += lds_l[k][r] * pow2i(mk - mm);
        }
        lds_mm[r] = mm;
        lds_sum[r] = sum;
      }
    }
    constexpr int SPAD = D + 4;  // staged row stride (floats): rows fall on different banks
    float* stage = reinterpret_cast<float*>(ring + fs * RG::SLOT);  // [8 rows][SPAD]
#pragma unroll
    for (int ps = 0; ps < NRG * 16 / PASS_ROWS; ++ps) {
      const int rg = ps / (16 / PASS_ROWS);
      const int r0 = ps * PASS_ROWS;  // first row of the pass
      if (col - (r0 - rg * 16) >= 0 && col - (r0 - rg * 16) < PASS_ROWS) {
        float* dst = stage + (col - (r0 - rg * 16)) * SPAD + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; ++t) *reinterpret_cast<float4_t*>(dst + 16 * t) = u.o[rg][t];
      }
      lds_barrier();
      for (int idx = threadIdx.x; idx < PASS_ROWS * (D / 4); idx += 64 * W) {
        const int r = r0 + idx / (D / 4);
        const int d4 = idx % (D / 4);
        float4_t acc = float4_t{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const float* src = reinterpret_cast<const float*>(sh.ring + (k * NB + lds_fs[k]) * RG::SLOT);
          acc += *reinterpret_cast<const float4_t*>(src + (r - r0) * SPAD + 4 * d4);
        }
        if (r < cw.rows) {
          const float sum = lds_sum[r];
          if (cw.part < 0) {
            const int qi = cw.row_begin + r / cw.rows_per_query;
            const int head = cw.head_base + r % cw.rows_per_query;
            float4_t res = float4_t{0, 0, 0, 0};
            if (sum > 0.0f) res = div4(acc, sum);
            if (4 * d4 < p.dims)
              *reinterpret_cast<float4_t*>(p.out + (size_t)(cw.q_row + qi) * q_stride + (size_t)head * p.dims + 4 * d4) = res;
          } else if (MIX && p.counters) {  // merged in this launch: coherent stores
            store_partial_row<D>(p, cw.part, r, d4, acc);
            if (d4 == 0) store_partial_ml(p, cw.part, r, lds_mm[r], sum);
          } else {
            *reinterpret_cast<float4_t*>(p.part_o + ((size_t)cw.part * p.rows_cap + r) * D + 4 * d4) = acc;
            if (d4 == 0) {
              p.part_ml[((size_t)cw.part * p.rows_cap + r) * 2] = lds_mm[r];
              p.part_ml[((size_t)cw.part * p.rows_cap + r) * 2 + 1] = sum;
            }
          }
        }
      }
      lds_barrier();  // the slots (and, after the last pass, the merge area) are free again
    }
  };
  // Every wave passes the same unit boundaries in the same order (in the
  // page loop or in the closing loop below), so the barriers of finalize and
  // of a table reload pair up.
  auto next_unit = [&]() __attribute__((always_inline)) -> void {
    cbase += cw.page_end - cw.page_begin;
    ++ck;
    cw = load_work(work + (ck < last ? ck : last - 1));
    reset_unit();
    if (ck < last && ck >= qfirst + MAXU) {
      // (rare: more than MAXU units in one share) every wave has merged the
      // previous unit, so the table is free; the reload waits for this
      // wave's loads in flight.
      qfirst = ck;
      fill_q(qfirst);
      __syncthreads();
    }
  };

  // ---- the page loop -----------------------------------------------------------
  // The first pages are requested before the Q table is filled, so the
  // table's loads and the ring's first fetches share one memory round trip.
  request();
  PageFifo<NB> fifo;
  int head = 0, count = 0;
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) {
    if (count == b) {
      const int g = issue(b);
      if (g >= 0) {
        request();
        fifo.push(count, g);
        ++count;
      }
    }
  }
  float app_x[AJ][8];
  if constexpr (kApp) {
    if (app_n > 0) {
      const int rest = lane % RL;
      const int which = (rest >> 2) / NP, b = (rest >> 2) % NP, quarter = rest & 3;
      const int d0 = 32 * b + 8 * quarter;
      const float* src = which ? p.app_v : p.app_k;
      constexpr int E = FMT == kF16 ? 2 : 1;
      const BlockGeom geom = block_geom(FMT, D, SF32 ? 1 : 0);
#pragma unroll
      for (int a = 0; a < AJ; ++a) {
        const bool live = a * RJ + lane / RL < app_n;
        const int pos = rec_field(a, 1), kvrow = rec_field(a, 2), item = rec_field(a, 3);
        const int t = pos & 15;
        const int run = which ? geom.v_off() + v_index(t, d0, E) * E : k_index(t, d0, E) * E;
        const int sc = (which ? geom.vs_off() : geom.ks_off()) + scale_index_np(t, b, NP) * (SF32 ? 4 : 2);
        jobs[a].offs = run | (sc << 16);
        jobs[a].key = live ? (item << 16) | ((pos >> 4) & 0xffff) : -1;
#pragma unroll
        for (int i = 0; i < 8; ++i) app_x[a][i] = 0.0f;  // (dims past the head's own store zeros)
        if (live && (p.dims & 7) == 0) {
          if (d0 < p.dims) load8(app_x[a], src + (size_t)kvrow * p.dims + d0);
        } else if (live) {
          load8_head(app_x[a], src + (size_t)kvrow * p.dims, d0, p.dims);
        }
      }
    }
  }
  fill_q_start(qfirst);
  if constexpr (kApp) {
    if (app_n > 0) {
#pragma unroll
      for (int a = 0; a < AJ; ++a)
        if (a * RJ < app_n) jobs[a].c = encode_lane<FMT>(app_x[a]);  // (wave-uniform: shuffles)
    }
  }
  reset_unit();
  __syncthreads();  // the Q table is written
  // Close every unit that ends before this wave's next page (all of them
  // once the share is exhausted). Called with a free ring slot.
  auto close_units = [&]() __attribute__((always_inline)) -> void {
    while (ck < last && (count == 0 || fifo.front() >= cbase + (cw.page_end - cw.page_begin))) {
      int fs = head + count;
      fs = fs >= NB ? fs - NB : fs;
      finalize(fs);
      next_unit();
    }
  };
  close_units();
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
    const int g = fifo.front();
    const int pi = cw.page_begin + (g - cbase);
    if constexpr (kApp) {
      if (pi >= (cw.ctx >> 4)) {  // a page with new rows (a lane's key matches: its row)
        const int key = (ck << 16) | (pi & 0xffff);
        char* const slot = ring + head * RG::SLOT;
#pragma unroll
        for (int a = 0; a < AJ; ++a)
          if (jobs[a].key == key) patch_slot<FMT, SF32, D>(slot, jobs[a].c, jobs[a].offs, lane % RL, NP);
      }
    }
    const half8_t* qt = sh.q + (ck - qfirst) * QUNIT + lane;
    u.template consume_slot<SP>(
        ring + head * RG::SLOT, lane, pi, grp, pi >= unmasked,
        [&](int rg, int pp) __attribute__((always_inline)) { return qt[(rg * NP + pp) * 64]; },
        [&]() __attribute__((always_inline)) {
          // The next page id is read through the scalar cache only now,
          // after the K half's LDS reads have completed (they share the lgkm
          // counter), so its latency hides behind this page's math instead
          // of stalling the wave.
          lgkm_wait_all();
          if (gn >= 0) request();
        });
    head = head + 1 == NB ? 0 : head + 1;
    --count;
    fifo.pop();
    close_units();  // the slot just read is free
  }
  if constexpr (MIX) {
    // The split pieces of the share count in (and the last piece of a
    // record merges it) once the whole share is done: the ring is empty
    // then, so waiting for the coherent partial stores drains nothing. (At
    // the end of each piece instead, the wait drained every wave's ring:
    // 135 against 131 us for a c5-shaped mixed step.) Only a share's first
    // and last items can be pieces.
    if (p.counters) {
      for (int it = first; it < last; ++it) {
        const WorkRec w = load_work(work + it);
        if (w.part >= 0) arrive_and_merge<D, ROWS>(p, w.red, &sh.flag, sh.merge);
      }
    }
  }
  if constexpr (kApp) {
    // the rows into the pool (for the launches after this one); the list
    // bounds and records are read again (the empty asm keeps the compiler
    // from holding the first reads' registers through the page loop)
    int gw = group * W + wave;
    asm volatile("" : "+s"(gw));
    const sconst_int* af = (const sconst_int*)p.app_first + gw;
    app_off = af[0];
    app_n = af[1] - app_off;
    if (app_n > 0) {
      read_recs();
      const int rest = lane % RL;
      const BlockGeom geom = block_geom(FMT, D, SF32 ? 1 : 0);
      char* const pool = static_cast<char*>(const_cast<void*>(p.pool));
#pragma unroll
      for (int a = 0; a < AJ; ++a) {
        const int page = rec_field(a, 0), pos = rec_field(a, 1), kvrow = rec_field(a, 2);
        if (a * RJ + lane / RL < app_n)
          write_lane<FMT>(GlobalPut{pool + ((size_t)page * p.kv_heads + kvrow % p.kv_heads) * p.block_bytes},
                          geom, NP, SF32, jobs[a].c, pos & 15, (rest >> 2) / NP, (rest >> 2) % NP, rest & 3);
      }
    }
  }
}


// APP: the launch also encodes, attends to and stores the step's new rows
// (p.app_k, tge_decode_step).
template <int FMT, bool SF32, int D, int NRG, int W, int WPE, bool SP, bool APP = false, bool SKIP = false>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void paged_decode_kernel(AttnParams p) {
  __shared__ DecodeShared<FMT, SF32, D, NRG, SP> sh;
  decode_body<FMT, SF32, D, NRG, W, WPE, SP, false, APP, SKIP>(p, sh, blockIdx.x);
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
// NRGP: 16-row groups per wave (2, or 1 for 64-row tiles: the 256-dim
// kernels, and the narrow 128-dim tiles of steps too small to fill the
// compute units with 128-row tiles).
template <int FMT, bool SF32, int D, int WPE, int HALVES = 1, int NRGP = (D > 128 ? 1 : 2)>
struct PrefillShared {
  static constexpr int SLOT = Ring<FMT, SF32, D>::SLOT;
  static constexpr int TILE = kWaves * SLOT;  // four pages
  static constexpr int NB_FIT = (160 * 1024 / WPE - 64) / TILE;
  static constexpr int NB = NB_FIT > 4 ? 4 : NB_FIT;
  static_assert(NB >= 2, "the prefill ring needs two tiles");
  // one ring per half; afterwards the second half's states pass through it
  static constexpr int NRG = NRGP;  // row groups of 16 per wave
  static constexpr int XO = kWaves * NRG * (D / 16) * 64 * 16;  // accumulators (bytes)
  static constexpr int XS = kWaves * NRG * 3 * 64 * 4;          // base, sum, empty flag
  static_assert(HALVES == 1 || XO + XS <= HALVES * NB * TILE, "state exchange fits the rings");
  alignas(16) char ring[HALVES * NB * TILE];
  int flag;      // arrival broadcast of the in-kernel split merge
  int hbar[2];   // per-half tile barriers (arrivals, counting up)
};

// Waves of 32 rows per block-prefill workgroup, in halves of four: with two
// halves (eight waves, one workgroup per CU at two waves per SIMD) each half
// takes half of the item's pages for the same rows, and the halves' states
// are merged through LDS at the end (no partial slots, no merge launch).
template <int WPE>
constexpr int halves_for_wpe() {
  return WPE == 2 ? 2 : 1;
}

// Tile barrier of one half's four waves (the two halves run their tile
// loops independently): this wave's LDS reads are complete, it counts in,
// and waits until all four have counted `target` arrivals in total. The
// wait is bounded (about 0.2 s): past the bound the wave goes on, the
// launch completes with wrong rows instead of hanging, and the expiry is
// counted in g_wait_expired (tge_wait_expiries reads it).
__device__ __forceinline__ void half_barrier(int* ctr, int target) {
  bounded_barrier(ctr, target, &g_wait_expired);
}

// MERGE: split tiles are merged in the launch (the mixed-step kernel).
// HALVES: 1 or 2 groups of four waves sharing the item's rows (see above).
template <int FMT, bool SF32, int D, int WPE, bool SP, bool MERGE = false, int HALVES = 1,
          int NRGP = (D > 128 ? 1 : 2)>
__device__ __forceinline__ void prefill_body(const AttnParams& p,
                                             PrefillShared<FMT, SF32, D, WPE, HALVES, NRGP>& sh,
                                             const int item) {
  static_assert(HALVES == 1 || !MERGE, "the in-launch merge runs on four-wave workgroups");
  using SH = PrefillShared<FMT, SF32, D, WPE, HALVES, NRGP>;
  constexpr int NRG = SH::NRG;  // 32 rows per wave (16 in 64-row tiles)
  using U = Unit<FMT, SF32, D, NRG>;
  using Regs = typename U::Regs;
  using RG = Ring<FMT, SF32, D>;
  constexpr int NB = SH::NB;
  constexpr int NP = D / 32;
  constexpr int NT = D / 16;

  const WorkRec w = load_work((const sconst_work*)p.work + item);
  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = HALVES == 1 ? 0 : wave_all / kWaves;
  const int wave = HALVES == 1 ? wave_all : wave_all % kWaves;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int q_stride = p.q_heads * p.dims;
  const int row0 = wave * 16 * NRG;
  const bool has_rows = row0 < w.rows;

  // This half's pages: the first half takes whole tiles of four.
  const int all_pages = w.page_end - w.page_begin;
  const int cut = HALVES == 1 ? all_pages : min(all_pages, ((all_pages + 1) / 2 + 3) / 4 * 4);
  const int first_page = w.page_begin + (half == 0 ? 0 : cut);
  const int npages = half == 0 ? cut : all_pages - cut;
  const int ntiles = (npages + kWaves - 1) / kWaves;
  char* const ring = sh.ring + half * NB * SH::TILE;
  const sconst_int* table = (const sconst_int*)(p.tables + w.table_off + first_page);
  // Tile k, page `wave` of it: fetched by this wave (nothing past the range).
  auto fetch_tile = [&](int k) __attribute__((always_inline)) -> void {
    const int j = k * kWaves + wave;
    if (j < npages) {
      const char* blk = static_cast<const char*>(p.pool) +
                        ((size_t)table[j] * p.kv_heads + w.kv_head) * p.block_bytes;
      fetch_page<FMT, SF32, D, kPageReusePolicy>(ring + (k % NB) * SH::TILE + wave * RG::SLOT, blk,
                                                 p.block_bytes, lane);
    }
  };
  // The first tiles' fetches go out before the Q loads (both latencies overlap).
#pragma unroll
  for (int k = 0; k < NB - 1; ++k) {
    if (k < ntiles) fetch_tile(k);
  }

  // This wave's rows: Q^T operands (as in attend_unit) and visible limits.
  U u;
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const int r = row0 + rg * 16 + col;
    const bool valid = r < w.rows;
    const int qi = w.row_begin + (valid ? r / w.rows_per_query : 0);
    const int head = w.head_base + (valid ? r % w.rows_per_query : 0);
    const float* qp = p.q + (size_t)(w.q_row + qi) * q_stride + (size_t)head * p.dims + 4 * grp;
    if (half == 0) {  // (the second half takes the first half's operands, below)
#pragma unroll
      for (int pp = 0; pp < NP; ++pp) {
        // (dims past the head's own read as zeros)
        float4 a = make_float4(0, 0, 0, 0), b = make_float4(0, 0, 0, 0);
        if (valid && 32 * pp + 4 * grp < p.dims) a = *reinterpret_cast<const float4*>(qp + 32 * pp);
        if (valid && 32 * pp + 16 + 4 * grp < p.dims) b = *reinterpret_cast<const float4*>(qp + 32 * pp + 16);
        const float c = p.scale_log2;
        const float x[8] = {a.x * c, a.y * c, a.z * c, a.w * c, b.x * c, b.y * c, b.z * c, b.w * c};
#pragma unroll
        for (int j = 0; j < 8; ++j) u.q[rg][pp][j] = (_Float16)x[j];
      }
    }
    u.lim[rg] = valid ? w.ctx + w.row_begin + r / w.rows_per_query : -1;
    u.base[rg] = 0.0f;
    u.thr[rg] = -INFINITY;
    u.l4[rg] = float4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NT; ++t) u.o[rg][t] = float4_t{0, 0, 0, 0};
  }
  if constexpr (HALVES == 2) {
    // The first half's waves pass their f16 Q^T operands to the second
    // half's through LDS (half the Q reads): each half's last ring slot is
    // free until the loop's first fetch, two waves' operands to a slot.
    static_assert(2 * NRG * NP * 64 * 16 <= SH::TILE, "two waves' Q operands fit a ring slot");
    half8_t* stage = reinterpret_cast<half8_t*>(sh.ring + (wave / 2) * NB * SH::TILE +
                                                (NB - 1) * SH::TILE) +
                     (wave % 2) * NRG * NP * 64;
    if (half == 0) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) stage[(rg * NP + pp) * 64 + lane] = u.q[rg][pp];
      }
    }
    if (threadIdx.x < 2) sh.hbar[threadIdx.x] = 0;
    lds_barrier();
    if (half == 1) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) u.q[rg][pp] = stage[(rg * NP + pp) * 64 + lane];
      }
    }
    // Every second-half wave holds its operands before either half's first
    // in-loop fetch refills the staging slots (the first half's tile
    // barrier does not wait for the second half's reads).
    lds_barrier();
  }
  u.set_sparse(p.sp_sink, p.sp_window, p.sp_stride,
               w.ctx + w.row_begin + (w.rows - 1) / w.rows_per_query + 1);
  // Pages at or past `unmasked` hold a position some row of the wave may not see.
  const int unmasked =
      __builtin_amdgcn_readfirstlane((w.ctx + w.row_begin + row0 / w.rows_per_query + 1) / 16);

  // Last tile holding a page of this wave.
  const int t_last = wave < npages ? (npages - 1 - wave) / kWaves : -1;
  // Start of tile k: this wave's page of it has landed (its pages of up to
  // NB - 2 younger tiles may still be in flight), then every wave's has, and
  // every wave is done with tile k - 1, whose slot the fetch refills.
  auto tile_sync = [&](int k) __attribute__((always_inline)) {
    if (k <= t_last) {
      const int younger = (k + NB - 2 < t_last ? k + NB - 2 : t_last) - k;
      wait_vmcnt_pages<NB - 2, RG::LOADS>(younger);
    }
    if constexpr (HALVES == 2) {
      half_barrier(&sh.hbar[half], kWaves * (k + 1));
    } else {
      lds_barrier();
    }
    if (k + NB - 1 < ntiles) fetch_tile(k + NB - 1);
  };
  const auto qf = [&](int rg, int pp) __attribute__((always_inline)) { return u.qop(rg, pp); };
  // Pages j and j + 1 of the tile in LDS at `tile` (logical page pi first).
  auto pair = [&](const char* tile, int j, int pi) __attribute__((always_inline)) {
    if constexpr (FMT == kF16) {
      u.consume2_slots(tile + j * RG::SLOT, tile + (j + 1) * RG::SLOT, lane, pi, pi + 1, grp,
                       pi >= unmasked, pi + 1 >= unmasked, qf);
    } else {
      Regs ra, rb;
      read_page<FMT, SF32, D>(ra, tile + j * RG::SLOT, lane, grp);
      read_page<FMT, SF32, D>(rb, tile + (j + 1) * RG::SLOT, lane, grp);
      u.consume2(ra, rb, pi, pi + 1, grp, pi >= unmasked, pi + 1 >= unmasked, qf);
    }
  };
  // Tiles whose four pages all lie in the range take a straight path with
  // no per-page range test (the accumulators then keep their registers
  // from one page pair to the next, with no copies between them); the
  // last, partial tile and static sparse subsets take the general one.
  const int nfull = SP ? 0 : npages / kWaves;
  if (!has_rows) {
    for (int k = 0; k < ntiles; ++k) tile_sync(k);
  } else {
    int k = 0;
    for (; k < nfull; ++k) {
      tile_sync(k);
      const char* tile = ring + (k % NB) * SH::TILE;
      const int pi = first_page + k * kWaves;
      pair(tile, 0, pi);
      pair(tile, 2, pi + 2);
    }
    for (; k < ntiles; ++k) {
      tile_sync(k);
      const char* tile = ring + (k % NB) * SH::TILE;
#pragma unroll
      for (int j = 0; j < kWaves; j += 2) {
        const int pg = k * kWaves + j;
        const int pi = first_page + pg;
        if (SP) {  // static sparse subsets take the pages one by one
          for (int jj = j; jj < j + 2 && k * kWaves + jj < npages; ++jj) {
            Regs r;
            read_page<FMT, SF32, D>(r, tile + jj * RG::SLOT, lane, grp);
            u.template consume<true>(r, first_page + k * kWaves + jj, grp,
                                     first_page + k * kWaves + jj >= unmasked);
          }
        } else if (pg + 1 < npages) {
          pair(tile, j, pi);
        } else if (pg < npages) {
          Regs r;
          read_page<FMT, SF32, D>(r, tile + j * RG::SLOT, lane, grp);
          u.template consume<false>(r, pi, grp, pi >= unmasked);
        }
      }
    }
  }
  if constexpr (HALVES == 2) {
    // The second half hands its states to the first through the rings'
    // LDS (lane l of wave w holds the same rows and dims in both halves).
    __syncthreads();  // every wave is done with the rings
    float4_t* xo = reinterpret_cast<float4_t*>(sh.ring) + wave * NRG * NT * 64;
    float* xs = reinterpret_cast<float*>(sh.ring + SH::XO) + wave * NRG * 3 * 64;
    if (half == 1 && has_rows) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
        for (int t = 0; t < NT; ++t) xo[(rg * NT + t) * 64 + lane] = u.o[rg][t];
        xs[(rg * 3 + 0) * 64 + lane] = u.base[rg];
        xs[(rg * 3 + 1) * 64 + lane] = u.l4[rg][0];
        xs[(rg * 3 + 2) * 64 + lane] = u.thr[rg] == -INFINITY ? 0.0f : 1.0f;
      }
    }
    __syncthreads();
    if (half == 1) return;
    if (has_rows) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        if (xs[(rg * 3 + 2) * 64 + lane] == 0.0f) continue;  // the second half saw nothing
        const float b1 = xs[(rg * 3 + 0) * 64 + lane], l1 = xs[(rg * 3 + 1) * 64 + lane];
        const bool empty0 = u.thr[rg] == -INFINITY;
        const float m = empty0 ? b1 : fmaxf(u.base[rg], b1);
        const float a0 = empty0 ? 0.0f : pow2i(u.base[rg] - m), a1 = pow2i(b1 - m);
        const float l = u.l4[rg][0] * a0 + l1 * a1;
        u.l4[rg] = float4_t{l, l, l, l};
#pragma unroll
        for (int t = 0; t < NT; ++t) u.o[rg][t] = u.o[rg][t] * a0 + xo[(rg * NT + t) * 64 + lane] * a1;
        u.base[rg] = m;
        u.thr[rg] = kLazyMax;
      }
    }
  }
  // Write this wave's rows: normalised output, or the split's partial state.
  if (has_rows) {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const int r = row0 + rg * 16 + col;
      if (r >= w.rows) continue;
      const float sum = u.l4[rg][0];
      const float mx = u.thr[rg] == -INFINITY ? -INFINITY : u.base[rg];
      if (w.part < 0) {
        const int qi = w.row_begin + r / w.rows_per_query;
        const int head = w.head_base + r % w.rows_per_query;
        float* op = p.out + (size_t)(w.q_row + qi) * q_stride + (size_t)head * p.dims + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          float4_t res = float4_t{0, 0, 0, 0};
          if (sum > 0.0f) res = div4(u.o[rg][t], sum);
          if (16 * t + 4 * grp < p.dims) *reinterpret_cast<float4_t*>(op + 16 * t) = res;
        }
      } else if (MERGE && p.counters) {  // merged in this launch: coherent stores
#pragma unroll
        for (int t = 0; t < NT; ++t) store_partial_row<D>(p, w.part, r, 4 * t + grp, u.o[rg][t]);
        if (grp == 0) store_partial_ml(p, w.part, r, mx, sum);
      } else {
        float* po = p.part_o + ((size_t)w.part * p.rows_cap + r) * D + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; ++t) *reinterpret_cast<float4_t*>(po + 16 * t) = u.o[rg][t];
        if (grp == 0) {
          p.part_ml[((size_t)w.part * p.rows_cap + r) * 2] = mx;
          p.part_ml[((size_t)w.part * p.rows_cap + r) * 2 + 1] = sum;
        }
      }
    }
  }
  // the last piece of a split tile merges it (every wave takes part)
  if constexpr (MERGE) {
    // (every tile of the ring is consumed: its LDS is the merge scratch)
    if (p.counters && w.part >= 0)
      arrive_and_merge<D, kPrefillRows>(p, w.red, &sh.flag, reinterpret_cast<float*>(sh.ring));
  }
}

template <int FMT, bool SF32, int D, int WPE, bool SP, int NRGP = (D > 128 ? 1 : 2)>
__global__ __launch_bounds__(256 * halves_for_wpe<WPE>()) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void paged_prefill_kernel(AttnParams p) {
  constexpr int H = halves_for_wpe<WPE>();
  __shared__ PrefillShared<FMT, SF32, D, WPE, H, NRGP> sh;
  prefill_body<FMT, SF32, D, WPE, SP, false, H, NRGP>(p, sh, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Mixed-step kernel (continuous batching: some sessions decoding, some
// prefilling a chunk, forward_batch qwen2.cpp:1613-1747): one launch whose
// first n_dec workgroups (one per CU) run the decode role over the decode
// plan's persistent shares and whose remaining workgroups are block-prefill
// tiles of the prefill plan; the tiles take each CU's other slot from the
// start and its decode slot once the share is done, so the HBM-bound decode
// runs under the MFMA-bound tiles. Split pieces of either kind are merged in
// the same launch by the last piece to arrive.
// The two roles share the workgroup's LDS (a union) and its register budget.
// ---------------------------------------------------------------------------
// SP: both roles apply the static sparse subset (the decode role reads
// every page of its units, as the sparse decode kernel does for strides up
// to 16).
template <int FMT, bool SF32, int D, int NRG, bool SP = false>
struct MixCfg {
  using DC = DecodeCfg<FMT, SF32, D, NRG, SP, true>;
  static constexpr int WPE = DC::WPE;
};

template <int FMT, bool SF32, int D, int NRG, bool SP = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MixCfg<FMT, SF32, D, NRG, SP>::WPE,
                                                                     MixCfg<FMT, SF32, D, NRG, SP>::WPE)))
void paged_mixed_kernel(AttnParams dec, AttnParams pf, int n_dec) {
  using DC = typename MixCfg<FMT, SF32, D, NRG, SP>::DC;
  constexpr int WPE = MixCfg<FMT, SF32, D, NRG, SP>::WPE;
  static_assert(DC::W == 4, "both roles run 256 threads");
  static_assert(DecodeShared<FMT, SF32, D, NRG, SP, true>::MERGE_FLOATS >= 10 * 16 * NRG,
                "the decode merge area holds the split merge's scratch");
  static_assert(sizeof(PrefillShared<FMT, SF32, D, WPE>::ring) >= 10 * kPrefillRows * sizeof(float),
                "the prefill ring holds the split merge's scratch");
  __shared__ union {
    DecodeShared<FMT, SF32, D, NRG, SP, true> d;
    PrefillShared<FMT, SF32, D, WPE> p;
  } sh;
  if ((int)blockIdx.x < n_dec) {
    decode_body<FMT, SF32, D, NRG, 4, WPE, SP, true>(dec, sh.d, blockIdx.x);
  } else {
    prefill_body<FMT, SF32, D, WPE, SP, true>(pf, sh.p, blockIdx.x - n_dec);
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
  if (4 * d4 >= p.dims) return;  // a dim past the head's own
  const int q_stride = p.q_heads * p.dims;
  const int qi = it.row_begin + r / it.rows_per_query;
  const int head = it.head_base + r % it.rows_per_query;
  float4_t res = float4_t{0, 0, 0, 0};
  if (sum > 0.0f) res = div4(acc, sum);
  *reinterpret_cast<float4_t*>(p.out + (size_t)(it.q_row + qi) * q_stride + (size_t)head * p.dims + 4 * d4) = res;
}

}  // namespace

// Row groups a decode unit may hold at a block width (max_unit_rows / 16).
template <int D>
constexpr int max_row_groups() {
  return max_unit_rows(D) / 16;
}

template <int FMT, bool SF32, int D>
hipError_t launch_decode_d(int row_groups, int n_groups, const AttnParams& p, hipStream_t stream) {
  switch (row_groups) {
#define TGE_DEC(n)                                                                          \
  case n: {                                                                                 \
    if constexpr (n <= max_row_groups<D>()) {                                               \
      using C = DecodeCfg<FMT, SF32, D, n, false>;                                          \
      using CS = DecodeCfg<FMT, SF32, D, n, true>;                                          \
      if (p.sp_stride > 16) {                                                               \
        hipLaunchKernelGGL((paged_decode_kernel<FMT, SF32, D, n, CS::W, CS::WPE, true, false,  \
                                                true>),                                     \
                           dim3((unsigned)n_groups), dim3(64 * CS::W), 0, stream, p);       \
      } else if (p.sp_stride > 0) {                                                         \
        hipLaunchKernelGGL((paged_decode_kernel<FMT, SF32, D, n, CS::W, CS::WPE, true>),    \
                           dim3((unsigned)n_groups), dim3(64 * CS::W), 0, stream, p);       \
      } else if (p.app_k) {                                                                 \
        if constexpr (C::kApp)                                                              \
          hipLaunchKernelGGL((paged_decode_kernel<FMT, SF32, D, n, C::W, C::WPE, false,     \
                                                  C::kApp>),                                \
                             dim3((unsigned)n_groups), dim3(64 * C::W), 0, stream, p);      \
        else                                                                                \
          return hipErrorInvalidValue;                                                      \
      } else {                                                                              \
        hipLaunchKernelGGL((paged_decode_kernel<FMT, SF32, D, n, C::W, C::WPE, false>),     \
                           dim3((unsigned)n_groups), dim3(64 * C::W), 0, stream, p);        \
      }                                                                                     \
      break;                                                                                \
    } else {                                                                                \
      return hipErrorInvalidValue;                                                          \
    }                                                                                       \
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
int decode_blocks_d(int row_groups, bool sparse) {
  int n = 0;
  hipError_t e = hipErrorInvalidValue;
  switch (row_groups) {
#define TGE_DOCC(r)                                                                        \
  case r: {                                                                                \
    if constexpr (r <= max_row_groups<D>()) {                                              \
      using C = DecodeCfg<FMT, SF32, D, r, false>;                                         \
      using CS = DecodeCfg<FMT, SF32, D, r, true>;                                         \
      e = sparse ? hipOccupancyMaxActiveBlocksPerMultiprocessor(                           \
                       &n, paged_decode_kernel<FMT, SF32, D, r, CS::W, CS::WPE, true>,     \
                       64 * CS::W, 0)                                                      \
                 : hipOccupancyMaxActiveBlocksPerMultiprocessor(                           \
                       &n, paged_decode_kernel<FMT, SF32, D, r, C::W, C::WPE, false>,      \
                       64 * C::W, 0);                                                      \
    }                                                                                      \
    break;                                                                                 \
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

// Calls f.template operator()<FMT, SF32, D>() for a pool's format, scale
// format and block width (64, 128 or 256); `bad` for any other.
template <class R, class F>
R with_variant(int format, int scale_f32, int head_dim, R bad, F&& f) {
  if (format == kF16) {
    if (head_dim == 64) return f.template operator()<kF16, false, 64>();
    if (head_dim == 128) return f.template operator()<kF16, false, 128>();
    if (head_dim == 256) return f.template operator()<kF16, false, 256>();
  } else if (format == kI8) {
    if (head_dim == 64)
      return scale_f32 ? f.template operator()<kI8, true, 64>() : f.template operator()<kI8, false, 64>();
    if (head_dim == 128)
      return scale_f32 ? f.template operator()<kI8, true, 128>() : f.template operator()<kI8, false, 128>();
    if (head_dim == 256)
      return scale_f32 ? f.template operator()<kI8, true, 256>() : f.template operator()<kI8, false, 256>();
  }
  return bad;
}

hipError_t launch_decode(int format, int scale_f32, int head_dim, int row_groups, int n_groups,
                         const AttnParams& p, hipStream_t stream) {
  if (n_groups <= 0) return hipSuccess;
  if (!p.wg_first) return hipErrorInvalidValue;
  return with_variant(format, scale_f32, head_dim, hipErrorInvalidValue,
                      [&]<int FMT, bool SF32, int D>() {
                        return launch_decode_d<FMT, SF32, D>(row_groups, n_groups, p, stream);
                      });
}

int decode_blocks_per_cu(int format, int scale_f32, int head_dim, int row_groups, bool sparse) {
  return with_variant(format, scale_f32, head_dim, 0, [&]<int FMT, bool SF32, int D>() {
    return decode_blocks_d<FMT, SF32, D>(row_groups, sparse);
  });
}

template <int FMT, bool SF32, int D, int R>
constexpr int decode_app_waves_r() {
  if constexpr (R <= max_row_groups<D>()) {
    using C = DecodeCfg<FMT, SF32, D, R>;
    return C::kApp ? C::W : 0;
  } else {
    return 0;
  }
}

int decode_app_waves(int format, int scale_f32, int head_dim, int row_groups) {
  return with_variant(format, scale_f32, head_dim, 0, [&]<int FMT, bool SF32, int D>() {
    switch (row_groups) {
      case 1: return decode_app_waves_r<FMT, SF32, D, 1>();
      case 2: return decode_app_waves_r<FMT, SF32, D, 2>();
      case 3: return decode_app_waves_r<FMT, SF32, D, 3>();
      case 4: return decode_app_waves_r<FMT, SF32, D, 4>();
      default: return 0;
    }
  });
}

template <int FMT, int D>
constexpr int prefill_wpe() {
#ifdef TGE_PREFILL_WPE
  return TGE_PREFILL_WPE;
#else
  return waves_per_eu<FMT, D, 2>();
#endif
}

// tile_rows: rows of the plan's tiles (128, or 64: one 16-row group per
// wave; always 64 at 256 dims).
template <int FMT, bool SF32, int D>
hipError_t launch_prefill_d(int n_units, int tile_rows, const AttnParams& p, hipStream_t stream) {
  constexpr int wpe = prefill_wpe<FMT, D>();
  const dim3 block(256 * halves_for_wpe<wpe>()), grid((unsigned)n_units);
  const bool sp = p.sp_stride > 0;
  if (tile_rows == prefill_tile_rows(D)) {
    if (sp) {
      hipLaunchKernelGGL((paged_prefill_kernel<FMT, SF32, D, wpe, true>), grid, block, 0, stream, p);
    } else {
      hipLaunchKernelGGL((paged_prefill_kernel<FMT, SF32, D, wpe, false>), grid, block, 0, stream, p);
    }
  } else if constexpr (D == 128) {
    if (tile_rows != 64) return hipErrorInvalidValue;
    if (sp) {
      hipLaunchKernelGGL((paged_prefill_kernel<FMT, SF32, D, wpe, true, 1>), grid, block, 0, stream, p);
    } else {
      hipLaunchKernelGGL((paged_prefill_kernel<FMT, SF32, D, wpe, false, 1>), grid, block, 0, stream, p);
    }
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int FMT, bool SF32, int D>
hipError_t launch_mixed_d(int row_groups, int n_dec, int n_pf, const AttnParams& dec,
                          const AttnParams& pf, hipStream_t stream) {
  const dim3 grid((unsigned)(n_dec + n_pf)), block(256);
  switch (row_groups) {
#define TGE_MIX(n)                                                                                \
  case n:                                                                                         \
    if constexpr (n <= max_row_groups<D>()) {                                                     \
      if (dec.sp_stride > 0)                                                                      \
        hipLaunchKernelGGL((paged_mixed_kernel<FMT, SF32, D, n, true>), grid, block, 0, stream, dec, \
                           pf, n_dec);                                                            \
      else                                                                                        \
        hipLaunchKernelGGL((paged_mixed_kernel<FMT, SF32, D, n>), grid, block, 0, stream, dec, pf, \
                           n_dec);                                                                \
      break;                                                                                      \
    } else {                                                                                      \
      return hipErrorInvalidValue;                                                                \
    }
    TGE_MIX(1)
    TGE_MIX(2)
    TGE_MIX(3)
    TGE_MIX(4)
#undef TGE_MIX
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_mixed(int format, int scale_f32, int head_dim, int row_groups, int n_dec,
                        int n_pf, const AttnParams& dec, const AttnParams& pf, hipStream_t stream) {
  if (n_dec + n_pf <= 0) return hipSuccess;
  if (!dec.wg_first || !dec.counters || !pf.counters) return hipErrorInvalidValue;
  return with_variant(format, scale_f32, head_dim, hipErrorInvalidValue,
                      [&]<int FMT, bool SF32, int D>() {
                        return launch_mixed_d<FMT, SF32, D>(row_groups, n_dec, n_pf, dec, pf, stream);
                      });
}


int prefill_halves(int format, int head_dim) {
  return with_variant(format, 0, head_dim, 1, [&]<int FMT, bool SF32, int D>() {
    return halves_for_wpe<prefill_wpe<FMT, D>()>();
  });
}

hipError_t launch_prefill(int format, int scale_f32, int head_dim, int n_units, int tile_rows,
                          const AttnParams& p, hipStream_t stream) {
  if (n_units <= 0) return hipSuccess;
  return with_variant(format, scale_f32, head_dim, hipErrorInvalidValue,
                      [&]<int FMT, bool SF32, int D>() {
                        return launch_prefill_d<FMT, SF32, D>(n_units, tile_rows, p, stream);
                      });
}

template <int D>
hipError_t launch_reduce_d(int n_items, int max_parts, const ReduceParams& p, hipStream_t stream) {
  // Slots per row: one per batch of 8 splits (one round of loads), at most 8
  // (4 at 256 dims: a row's 64 (4-dim) lanes times the slots fill the 256
  // threads).
  constexpr int kMaxSlots = D > 128 ? 4 : 8;
  const int want = (max_parts + 7) / 8;
  const int slots = want <= 1 ? 1 : (want <= 2 ? 2 : (want <= 4 || kMaxSlots == 4 ? 4 : 8));
  const int rpb = 256 / (D / 4 * slots);
  const dim3 grid((unsigned)n_items, (unsigned)((p.rows_cap + rpb - 1) / rpb)), block(256);
  switch (slots) {
    case 1: hipLaunchKernelGGL((split_reduce_kernel<D, 1>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((split_reduce_kernel<D, 2>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((split_reduce_kernel<D, 4>), grid, block, 0, stream, p); break;
    default:
      if constexpr (kMaxSlots == 8) hipLaunchKernelGGL((split_reduce_kernel<D, 8>), grid, block, 0, stream, p);
      break;
  }
  return hipGetLastError();
}

hipError_t read_wait_expiries(unsigned int* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_wait_expired), sizeof(unsigned int), 0,
                             hipMemcpyDeviceToHost);
}

hipError_t launch_reduce(int head_dim, int n_items, int max_parts, const ReduceParams& p,
                         hipStream_t stream) {
  if (n_items == 0) return hipSuccess;
  if (head_dim == 64) return launch_reduce_d<64>(n_items, max_parts, p, stream);
  if (head_dim == 128) return launch_reduce_d<128>(n_items, max_parts, p, stream);
  if (head_dim == 256) return launch_reduce_d<256>(n_items, max_parts, p, stream);
  return hipErrorInvalidValue;
}

}  // namespace tge
