// C ABI of the gfx950 paged-KV path: backend bring-up, page pools, per-step
// batch plans and the kernel entry points. See include/tge_kv.h.
#include "tge_kv.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <array>
#include <vector>

#include "tge_common.h"
#include "tge_error.h"
#include "tge_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

}  // namespace

void tge::set_last_error(const std::string& message) { g_last_error = message; }

namespace {

#define TGE_HIP(call)                                                          \
  do {                                                                         \
    const hipError_t e_ = (call);                                              \
    if (e_ != hipSuccess)                                                      \
      return fail(TGE_ERR_DEVICE, std::string(#call ": ") + hipGetErrorString(e_)); \
  } while (0)

struct Backend {
  std::once_flag once;
  int status = TGE_ERR_UNAVAILABLE;
  std::string arch;
};
Backend g_backend;

int backend_ready() {
  std::call_once(g_backend.once, [] {
    const char* force = std::getenv("TGE_FORCE_UNAVAILABLE");
    if (force && force[0] && std::strcmp(force, "0") != 0) {
      g_backend.status = TGE_ERR_UNAVAILABLE;
      return;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return;
    g_backend.arch = prop.gcnArchName;
    if (g_backend.arch.rfind("gfx950", 0) == 0) g_backend.status = TGE_OK;
  });
  return g_backend.status;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

struct tge_kv_pool {
  tge_kv_pool_desc desc{};
  void* blocks = nullptr;   // layers x (pages * kv_heads) page blocks
  tge::BlockGeom geom{};
  size_t layer_blocks = 0;  // pages * kv_heads
  size_t bytes = 0;
};

// Work lists of one attention kind (decode or prefill) for the current plan.
struct AttnPlan {
  std::vector<tge::WorkRec> work;
  std::vector<tge::ReduceRec> reduce;
  std::vector<int> wg_first;  // empty: one item per workgroup
  int groups = 0;             // workgroups of the launch
  int row_groups = 1;
  int parts = 0;
  int max_splits = 0;
  bool built = false;
  // device image: work | reduce | wg_first
  char* dev = nullptr;
  size_t dev_bytes = 0;
  size_t off_reduce = 0;
  size_t off_first = 0;
  char* host = nullptr;
  size_t host_bytes = 0;
  hipEvent_t staged = nullptr;
  float* part_o = nullptr;
  float* part_ml = nullptr;
  size_t part_floats = 0;

  ~AttnPlan() {
    if (dev) (void)hipFree(dev);
    if (host) (void)hipHostFree(host);
    if (staged) (void)hipEventDestroy(staged);
    if (part_o) (void)hipFree(part_o);
    if (part_ml) (void)hipFree(part_ml);
  }
};

struct tge_batch {
  // Host copy of the plan.
  std::vector<tge::SessionRec> sessions;
  std::vector<int> tables;
  std::vector<tge::RowRec> rows;
  int kv_heads = 0, head_dim = 0, q_heads = 0, pages = 0, group = 1;
  int max_rows = 0;  // largest n_new * group
  bool planned = false;
  AttnPlan decode, prefill;
  // Mixed steps (tge_batch_attention): the decode kernel over the sessions
  // whose rows fit a decode unit, the prefill kernel over the others.
  AttnPlan mix_decode, mix_prefill;
  bool mix_built = false;
  // Static sparse subset of every attention call (stride 0: dense).
  int sp_sink = 0, sp_window = 0, sp_stride = 0;

  // Device image: sessions | tables | rows (one allocation), pinned staging.
  char* dev = nullptr;
  size_t dev_bytes = 0;
  char* host = nullptr;
  size_t host_bytes = 0;
  hipEvent_t staged = nullptr;
  size_t off_sessions = 0, off_tables = 0, off_rows = 0;

  // Kernel timing (tge_batch_set_profiling): per attention call since
  // enabling, events before the attention kernel, between it and the merge,
  // and after the merge. Triples are created on demand and reused.
  bool profiling = false;
  std::vector<std::array<hipEvent_t, 3>> prof;
  size_t prof_used = 0;

  ~tge_batch() {
    if (dev) (void)hipFree(dev);
    if (host) (void)hipHostFree(host);
    if (staged) (void)hipEventDestroy(staged);
    for (auto& t : prof)
      for (hipEvent_t e : t)
        if (e) (void)hipEventDestroy(e);
  }
};

extern "C" {

const char* tge_status_string(int status) {
  switch (status) {
    case TGE_OK: return "ok";
    case TGE_ERR_INVALID: return "invalid argument";
    case TGE_ERR_RUNTIME: return "runtime error";
    case TGE_ERR_UNAVAILABLE: return "backend unavailable";
    case TGE_ERR_DEVICE: return "device error";
    case TGE_ERR_CAPACITY: return "capacity exceeded";
    default: return "unknown status";
  }
}

const char* tge_last_error(void) { return g_last_error.c_str(); }

int tge_backend_init(void) {
  const int s = backend_ready();
  if (s != TGE_OK) return fail(s, "no gfx950 device available");
  return TGE_OK;
}

const char* tge_backend_arch(void) {
  backend_ready();
  return g_backend.arch.c_str();
}

int tge_kv_k_index(int token, int dim, int head_dim) {
  return tge::k_index_np(token, dim, head_dim / 32);
}
int tge_kv_v_index(int token, int dim, int head_dim) {
  return tge::v_index_np(token, dim, head_dim / 32);
}
int tge_kv_scale_index(int token, int block, int head_dim) {
  return tge::scale_index_np(token, block, head_dim / 32);
}

// ---------------------------------------------------------------------------
// Pool
// ---------------------------------------------------------------------------
int tge_kv_pool_create(const tge_kv_pool_desc* desc, tge_kv_pool** out) {
  if (!desc || !out) return fail(TGE_ERR_INVALID, "kv_pool_create: null argument");
  const tge_kv_pool_desc& d = *desc;
  if (d.layers <= 0 || d.pages <= 0 || d.kv_heads <= 0)
    return fail(TGE_ERR_INVALID, "kv_pool_create: non-positive size");
  if (d.head_dim != 64 && d.head_dim != 128)
    return fail(TGE_ERR_INVALID, "kv_pool_create: head_dim must be 64 or 128");
  if (d.format != TGE_KV_F16 && d.format != TGE_KV_I8)
    return fail(TGE_ERR_INVALID, "kv_pool_create: unknown format");
  if (d.format == TGE_KV_I8 && d.scale_format != TGE_SCALE_F16 &&
      d.scale_format != TGE_SCALE_F32)
    return fail(TGE_ERR_INVALID, "kv_pool_create: unknown scale format");
  const int s = backend_ready();
  if (s != TGE_OK) return fail(s, "kv_pool_create: backend unavailable");

  auto* p = new tge_kv_pool;
  p->desc = d;
  p->geom = tge::block_geom(d.format, d.head_dim, d.format == TGE_KV_I8 && d.scale_format == TGE_SCALE_F32);
  p->layer_blocks = (size_t)d.pages * d.kv_heads;
  // Kernels address a page block by its 64-bit address (one buffer
  // resource per block), so a layer's array has no 32-bit limit.
  const size_t layer_bytes = (size_t)p->geom.block_bytes * p->layer_blocks;
  const size_t total = layer_bytes * d.layers;
  hipError_t e = hipMalloc(&p->blocks, total);
  if (e == hipSuccess) e = hipMemset(p->blocks, 0, total);
  if (e != hipSuccess) {
    tge_kv_pool_destroy(p);
    return fail(e == hipErrorOutOfMemory ? TGE_ERR_CAPACITY : TGE_ERR_DEVICE,
                std::string("kv_pool_create: ") + hipGetErrorString(e));
  }
  p->bytes = total;
  *out = p;
  return TGE_OK;
}

void tge_kv_pool_destroy(tge_kv_pool* p) {
  if (!p) return;
  if (p->blocks) (void)hipFree(p->blocks);
  delete p;
}

size_t tge_kv_pool_bytes(const tge_kv_pool* p) { return p ? p->bytes : 0; }

int tge_kv_pool_layer(const tge_kv_pool* p, int layer, tge_kv_layer_view* out) {
  if (!p || !out) return fail(TGE_ERR_INVALID, "kv_pool_layer: null argument");
  if (layer < 0 || layer >= p->desc.layers)
    return fail(TGE_ERR_INVALID, "kv_pool_layer: layer out of range");
  char* base = static_cast<char*>(p->blocks) + (size_t)p->geom.block_bytes * p->layer_blocks * layer;
  const bool i8 = p->desc.format == TGE_KV_I8;
  out->k = base;
  out->v = base + p->geom.v_off();
  out->k_scales = i8 ? base + p->geom.ks_off() : nullptr;
  out->v_scales = i8 ? base + p->geom.vs_off() : nullptr;
  out->kv_block_bytes = (size_t)p->geom.kv_bytes;
  out->scale_block_bytes = (size_t)p->geom.scale_bytes;
  out->block_bytes = (size_t)p->geom.block_bytes;
  return TGE_OK;
}

int tge_kv_copy_page(tge_kv_pool* p, int src_page, int dst_page, void* stream) {
  if (!p) return fail(TGE_ERR_INVALID, "kv_copy_page: null pool");
  if (src_page < 0 || src_page >= p->desc.pages || dst_page < 0 || dst_page >= p->desc.pages)
    return fail(TGE_ERR_INVALID, "kv_copy_page: page outside the pool");
  if (src_page == dst_page) return TGE_OK;
  // A page's blocks are kv_heads consecutive blocks in every layer's array:
  // one strided copy of `layers` rows.
  const size_t row = (size_t)p->geom.block_bytes * p->desc.kv_heads;
  const size_t pitch = (size_t)p->geom.block_bytes * p->layer_blocks;
  char* base = static_cast<char*>(p->blocks);
  TGE_HIP(hipMemcpy2DAsync(base + row * dst_page, pitch, base + row * src_page, pitch, row,
                           (size_t)p->desc.layers, hipMemcpyDeviceToDevice,
                           static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

// ---------------------------------------------------------------------------
// Batch plan
// ---------------------------------------------------------------------------
int tge_batch_create(tge_batch** out) {
  if (!out) return fail(TGE_ERR_INVALID, "batch_create: null argument");
  *out = new tge_batch;
  return TGE_OK;
}

void tge_batch_destroy(tge_batch* b) { delete b; }

namespace {

// Splits [0, pages) into n nearly equal ranges and appends one unit each.
void add_units(std::vector<tge::WorkRec>& work, std::vector<tge::ReduceRec>& red,
               int& parts, int& max_splits, tge::WorkRec base, int pages, int pps) {
  const int n = std::max(1, (pages + pps - 1) / pps);
  max_splits = std::max(max_splits, n);
  if (n == 1) {
    base.page_begin = 0;
    base.page_end = pages;
    base.part = -1;
    work.push_back(base);
    return;
  }
  const int chunk = (pages + n - 1) / n;
  tge::ReduceRec r{};
  r.session = base.session;
  r.row_begin = base.row_begin;
  r.rows = base.rows;
  r.rows_per_query = base.rows_per_query;
  r.head_base = base.head_base;
  r.first_part = parts;
  r.n_parts = 0;
  for (int b = 0; b < pages; b += chunk) {
    tge::WorkRec w = base;
    w.page_begin = b;
    w.page_end = std::min(pages, b + chunk);
    w.part = parts++;
    work.push_back(w);
    ++r.n_parts;
  }
  red.push_back(r);
}


// Copies `bytes` from pinned staging to device memory on `st`, growing both
// buffers as needed; waits for the previous copy out of the staging buffer
// before overwriting it.
int stage_upload(char*& host, size_t& host_bytes, char*& dev, size_t& dev_bytes,
                 hipEvent_t& staged, size_t bytes, hipStream_t st,
                 const std::function<void(char*)>& fill) {
  bytes = std::max<size_t>(bytes, 256);
  if (staged) TGE_HIP(hipEventSynchronize(staged));
  if (bytes > host_bytes) {
    if (host) TGE_HIP(hipHostFree(host));
    host = nullptr;
    TGE_HIP(hipHostMalloc(&host, bytes));
    host_bytes = bytes;
  }
  if (bytes > dev_bytes) {
    if (dev) {
      TGE_HIP(hipStreamSynchronize(st));
      TGE_HIP(hipFree(dev));
    }
    dev = nullptr;
    TGE_HIP(hipMalloc(&dev, bytes));
    dev_bytes = bytes;
  }
  fill(host);
  TGE_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, st));
  if (!staged) TGE_HIP(hipEventCreateWithFlags(&staged, hipEventDisableTiming));
  TGE_HIP(hipEventRecord(staged, st));
  return TGE_OK;
}

// Uploads an attention plan's lists and sizes its split-K partial buffers.
int upload_plan(AttnPlan& pl, int head_dim, hipStream_t st) {
  const size_t wbytes = pl.work.size() * sizeof(tge::WorkRec);
  pl.off_reduce = align256(wbytes);
  pl.off_first = align256(pl.off_reduce + pl.reduce.size() * sizeof(tge::ReduceRec));
  const size_t total = pl.off_first + pl.wg_first.size() * sizeof(int);
  if (pl.groups == 0) pl.groups = (int)pl.work.size();
  int s = stage_upload(pl.host, pl.host_bytes, pl.dev, pl.dev_bytes, pl.staged, total, st,
                       [&](char* h) {
                         if (wbytes) std::memcpy(h, pl.work.data(), wbytes);
                         if (!pl.reduce.empty())
                           std::memcpy(h + pl.off_reduce, pl.reduce.data(),
                                       pl.reduce.size() * sizeof(tge::ReduceRec));
                         if (!pl.wg_first.empty())
                           std::memcpy(h + pl.off_first, pl.wg_first.data(),
                                       pl.wg_first.size() * sizeof(int));
                       });
  if (s != TGE_OK) return s;
  const size_t rows_cap = 16 * (size_t)pl.row_groups;
  const size_t need = (size_t)std::max(pl.parts, 1) * rows_cap * head_dim;
  if (need > pl.part_floats) {
    if (pl.part_o) {
      TGE_HIP(hipStreamSynchronize(st));
      TGE_HIP(hipFree(pl.part_o));
      TGE_HIP(hipFree(pl.part_ml));
    }
    pl.part_o = pl.part_ml = nullptr;
    TGE_HIP(hipMalloc(&pl.part_o, need * sizeof(float)));
    TGE_HIP(hipMalloc(&pl.part_ml, need / head_dim * 2 * sizeof(float)));
    pl.part_floats = need;
  }
  pl.built = true;
  return TGE_OK;
}

// Resident workgroups of an attention variant on this device (cached).
// Workgroups of a decode launch: one per CU (the decode kernel's workgroup
// holds all of a CU's waves), times what the occupancy query allows.
struct Residency {
  int groups;  // resident workgroups of the launch
  int cus;     // compute units
};

Residency resident_groups(int format, int scale_f32, int head_dim, int row_groups) {
  static std::mutex mu;
  static std::vector<std::pair<int, Residency>> cache;  // key -> residency
  const int key = ((format * 2 + scale_f32) * 256 + head_dim) * 8 + row_groups;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& kv : cache)
    if (kv.first == key) return kv.second;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  int per_cu = tge::decode_blocks_per_cu(format, scale_f32, head_dim, row_groups);
  if (per_cu <= 0) per_cu = 1;
  const Residency r{per_cu * cus, cus};
  cache.emplace_back(key, r);
  return r;
}

// Relative speed of the k-th workgroup that lands on a CU. Workgroups are
// dispatched one per CU before a CU gets a second, and on a shared SIMD the
// older wave wins issue, so equal page shares finish far apart (measured:
// ~25 % slower for the second). Shares are weighted by rank^k.
#ifndef TGE_DECODE_RANK_WEIGHT
#define TGE_DECODE_RANK_WEIGHT 0.76
#endif
// Fixed cost of one unit of a share (start-up and merge), in pages.
#ifndef TGE_DECODE_UNIT_COST
#define TGE_DECODE_UNIT_COST 22
#endif

// Decode schedule. Every (session, kv head) is a segment of pages whose rows
// are the GQA group of each new token. The segments are laid end to end and
// cut into one equal share of pages per resident workgroup, so all
// workgroups of the launch finish together; a segment cut into several
// items is merged by the split reduction.
// Sessions of a mixed step that the decode kernel takes: rows fit one unit.
bool decode_session(const tge_batch* b, const tge::SessionRec& sr) {
  return sr.n_new * b->group <= tge::kMaxRows;
}

// `only`: 0 every session, 1 decode sessions only, 2 the others only.
bool take_session(const tge_batch* b, const tge::SessionRec& sr, int only) {
  return only == 0 || (only == 1) == decode_session(b, sr);
}

void build_decode(tge_batch* b, Residency res, AttnPlan& pl, int only) {
  pl.work.clear();
  pl.reduce.clear();
  pl.wg_first.clear();
  pl.parts = pl.max_splits = 0;
  int max_rows = 0;
  for (const auto& sr : b->sessions)
    if (take_session(b, sr, only)) max_rows = std::max(max_rows, sr.n_new * b->group);
  pl.row_groups = std::max(1, std::min(4, (max_rows + 15) / 16));

  struct Seg {
    int session, head, pages;
  };
  std::vector<Seg> segs;
  long total = 0;
  for (int s = 0; s < (int)b->sessions.size(); ++s) {
    const tge::SessionRec& sr = b->sessions[s];
    if (!take_session(b, sr, only)) continue;
    const int pages = (sr.ctx + sr.n_new + 15) / 16;
    for (int h = 0; h < b->kv_heads; ++h) segs.push_back(Seg{s, h, pages});
    total += (long)pages * b->kv_heads;
  }
  // At least 8 pages per workgroup: on small steps (one to four sessions
  // of 1k-8k positions) shorter chains win over fewer split merges down to
  // 8 pages (c1-c3: 5-7 % per layer-step against 16; 4 is slower again).
#ifndef TGE_DECODE_MIN_PAGES
#define TGE_DECODE_MIN_PAGES 8
#endif
  const long g_eff = std::max<long>(
      1, std::min<long>(res.groups, (total + TGE_DECODE_MIN_PAGES - 1) / TGE_DECODE_MIN_PAGES));
  std::vector<double> w((size_t)g_eff);
  double wrem = 0.0;
  for (long g = 0; g < g_eff; ++g) {
    w[(size_t)g] = std::pow(TGE_DECODE_RANK_WEIGHT, (double)(g / std::max(1, res.cus)));
    wrem += w[(size_t)g];
  }

  // Cut the segments, end to end, into one share per workgroup. A share's
  // cost is its pages plus TGE_DECODE_UNIT_COST per piece (the fixed cost
  // of starting and merging a unit); each share gets the remaining cost in
  // proportion to its rank weight, the last one takes what is left.
  const double unit_cost = TGE_DECODE_UNIT_COST;
  std::vector<int> seg_of;  // segment of each work item
  long pages_rem = total, segs_rem = (long)segs.size();
  size_t si = 0;
  int pos = 0;
  pl.wg_first.push_back(0);
  for (long g = 0; g < g_eff && si < segs.size(); ++g) {
    const bool last_wg = g + 1 == g_eff;
    double target =
        ((double)pages_rem + unit_cost * (double)(segs_rem + (g_eff - g))) * w[(size_t)g] / wrem;
    wrem -= w[(size_t)g];
    bool started = false;
    while (si < segs.size()) {
      const Seg& sg = segs[si];
      const int left = sg.pages - pos;
      int take = left;
      if (!last_wg) {
        const double room = target - unit_cost;
        if (started && room < 1.0) break;
        take = (int)std::min<double>(left, std::max(1.0, std::floor(room)));
      }
      const tge::SessionRec& sr = b->sessions[sg.session];
      tge::WorkRec it{};
      it.session = sg.session;
      it.kv_head = sg.head;
      it.page_begin = pos;
      it.page_end = pos + take;
      it.part = -1;
      it.row_begin = 0;
      it.rows = sr.n_new * b->group;
      it.rows_per_query = b->group;
      it.head_base = sg.head * b->group;
      it.ctx = sr.ctx;
      it.q_row = sr.q_row;
      it.table_off = sr.table_off;
      pl.work.push_back(it);
      seg_of.push_back((int)si);
      started = true;
      target -= take + unit_cost;
      pos += take;
      pages_rem -= take;
      if (pos == sg.pages) {
        ++si;
        pos = 0;
        --segs_rem;
      }
      if (!last_wg && target < unit_cost + 1.0) break;
    }
    pl.wg_first.push_back((int)pl.work.size());
  }

  // Segments cut into several items are merged by the split reduction.
  for (size_t i = 0; i < pl.work.size();) {
    size_t j = i + 1;
    while (j < pl.work.size() && seg_of[j] == seg_of[i]) ++j;
    const int n = (int)(j - i);
    pl.max_splits = std::max(pl.max_splits, n);
    if (n > 1) {
      const tge::WorkRec& w0 = pl.work[i];
      tge::ReduceRec r{};
      r.session = w0.session;
      r.row_begin = w0.row_begin;
      r.rows = w0.rows;
      r.rows_per_query = w0.rows_per_query;
      r.head_base = w0.head_base;
      r.first_part = pl.parts;
      r.n_parts = n;
      for (size_t k = i; k < j; ++k) pl.work[k].part = pl.parts++;
      pl.reduce.push_back(r);
    }
    i = j;
  }
  pl.groups = (int)pl.wg_first.size() - 1;
}

// Prefill units: (session, KV head, query tile) x page splits. A tile takes
// as many whole queries as fit 128 rows of (query, head) pairs of the KV
// head's query group, so every K/V page a tile reads serves the whole group.
// Long spans are split so the launch has work for every CU; items are
// ordered longest first.
void build_prefill(tge_batch* b, AttnPlan& pl, int only) {
  pl.work.clear();
  pl.reduce.clear();
  pl.wg_first.clear();
  pl.groups = 0;
  pl.parts = pl.max_splits = 0;
  pl.row_groups = tge::kPrefillRows / 16;
  const int tq = std::max(1, tge::kPrefillRows / b->group);
  // Page-split size: enough items for about two rounds of two workgroups
  // on each of 256 CUs, at least 32 pages (eight tiles of four).
  long pages_total = 0;
  for (const auto& sr : b->sessions) {
    if (!take_session(b, sr, only)) continue;
    for (int a = 0; a < sr.n_new; a += tq)
      pages_total += (long)((sr.ctx + std::min(sr.n_new, a + tq) + 15) / 16) * b->kv_heads;
  }
#ifndef TGE_PREFILL_MIN_SPLIT
#define TGE_PREFILL_MIN_SPLIT 32
#endif
  const long target_units = 2L * 256 * 2;
  const int pps = (int)std::max<long>(TGE_PREFILL_MIN_SPLIT,
                                      ((pages_total + target_units - 1) / target_units + 3) / 4 * 4);
  for (int s = 0; s < (int)b->sessions.size(); ++s) {
    const tge::SessionRec& sr = b->sessions[s];
    if (!take_session(b, sr, only)) continue;
    for (int h = 0; h < b->kv_heads; ++h) {
      for (int a = 0; a < sr.n_new; a += tq) {
        tge::WorkRec w{};
        w.session = s;
        w.kv_head = h;
        w.ctx = sr.ctx;
        w.q_row = sr.q_row;
        w.table_off = sr.table_off;
        w.row_begin = a;
        w.rows = std::min(tq, sr.n_new - a) * b->group;
        w.rows_per_query = b->group;
        w.head_base = h * b->group;
        const int pages = (sr.ctx + a + std::min(tq, sr.n_new - a) + 15) / 16;
        add_units(pl.work, pl.reduce, pl.parts, pl.max_splits, w, pages, pps);
      }
    }
  }
  // Longest items first (partial slots are fixed per item, so order is free).
  std::stable_sort(pl.work.begin(), pl.work.end(), [](const tge::WorkRec& x, const tge::WorkRec& y) {
    return x.page_end - x.page_begin > y.page_end - y.page_begin;
  });
}

}  // namespace

int tge_batch_plan(tge_batch* b, const tge_kv_pool* pool, const tge_batch_desc* d,
                   void* stream) {
  if (!b || !pool || !d) return fail(TGE_ERR_INVALID, "batch_plan: null argument");
  const int ns = d->n_sessions;
  if (ns <= 0 || !d->ctx || !d->n_new || !d->table_offsets || !d->page_ids)
    return fail(TGE_ERR_INVALID, "batch_plan: empty or incomplete description");
  const int hkv = pool->desc.kv_heads, hd = pool->desc.head_dim;
  if (d->q_heads <= 0 || d->q_heads % hkv != 0)
    return fail(TGE_ERR_INVALID, "batch_plan: q_heads must be a multiple of kv_heads");
  const int group = d->q_heads / hkv;
  if (d->table_offsets[0] != 0)
    return fail(TGE_ERR_INVALID, "batch_plan: table_offsets[0] must be 0");
  const int n_entries = d->table_offsets[ns];
  if (n_entries < 0) return fail(TGE_ERR_INVALID, "batch_plan: negative table size");

  // Validate first: a failed plan leaves the batch unplanned, never half-built.
  int max_rows = 0;
  for (int s = 0; s < ns; ++s) {
    const int ctx = d->ctx[s], nn = d->n_new[s];
    const int lo = d->table_offsets[s], hi = d->table_offsets[s + 1];
    if (ctx < 0 || nn < 1)
      return fail(TGE_ERR_INVALID, "batch_plan: ctx must be >= 0 and n_new >= 1");
    if (hi < lo || hi > n_entries)
      return fail(TGE_ERR_INVALID, "batch_plan: table_offsets must not decrease");
    const long need = ((long)ctx + nn + 15) / 16;
    if (hi - lo < need)
      return fail(TGE_ERR_INVALID, "batch_plan: block table shorter than the context");
    for (long i = 0; i < need; ++i) {
      const int id = d->page_ids[lo + i];
      if (id < 0 || id >= pool->desc.pages)
        return fail(TGE_ERR_INVALID, "batch_plan: page id outside the pool");
    }
    max_rows = std::max(max_rows, nn * group);
  }

  b->planned = false;
  b->sessions.assign(ns, {});
  b->rows.clear();
  b->tables.assign(d->page_ids, d->page_ids + n_entries);
  int q_row = 0;
  for (int s = 0; s < ns; ++s) {
    const int ctx = d->ctx[s], nn = d->n_new[s], lo = d->table_offsets[s];
    b->sessions[s] = tge::SessionRec{ctx, nn, q_row, lo};
    for (int j = 0; j < nn; ++j) {
      const int pos = ctx + j;
      b->rows.push_back(tge::RowRec{d->page_ids[lo + pos / 16], pos % 16, pos});
    }
    q_row += nn;
  }
  b->kv_heads = hkv;
  b->head_dim = hd;
  b->q_heads = d->q_heads;
  b->group = group;
  b->pages = pool->desc.pages;
  b->max_rows = max_rows;
  b->prefill.built = false;
  b->decode.built = false;
  b->mix_built = false;

  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t o_sess = 0;
  const size_t o_tab = align256(o_sess + b->sessions.size() * sizeof(tge::SessionRec));
  const size_t o_rows = align256(o_tab + b->tables.size() * sizeof(int));
  const size_t total = o_rows + b->rows.size() * sizeof(tge::RowRec);
  int s = stage_upload(b->host, b->host_bytes, b->dev, b->dev_bytes, b->staged, total, st,
                       [&](char* h) {
                         std::memcpy(h + o_sess, b->sessions.data(),
                                     b->sessions.size() * sizeof(tge::SessionRec));
                         if (!b->tables.empty())
                           std::memcpy(h + o_tab, b->tables.data(), b->tables.size() * sizeof(int));
                         std::memcpy(h + o_rows, b->rows.data(),
                                     b->rows.size() * sizeof(tge::RowRec));
                       });
  if (s != TGE_OK) return s;
  b->off_sessions = o_sess;
  b->off_tables = o_tab;
  b->off_rows = o_rows;
  // Decode lists are built eagerly when the rows fit a decode unit (the
  // common case: one upload per step serves every layer).
  if (max_rows <= tge::kMaxRows) {
    const int rg = std::max(1, std::min(4, (max_rows + 15) / 16));
    build_decode(b, resident_groups(pool->desc.format, pool->desc.scale_format == TGE_SCALE_F32,
                                    hd, rg),
                 b->decode, 0);
    s = upload_plan(b->decode, hd, st);
    if (s != TGE_OK) return s;
  }
  b->planned = true;
  return TGE_OK;
}

int tge_batch_info(const tge_batch* b, int* rows, int* work_items, int* max_splits) {
  if (!b || !b->planned) return fail(TGE_ERR_INVALID, "batch_info: batch not planned");
  if (rows) *rows = (int)b->rows.size();
  if (work_items) *work_items = (int)b->decode.work.size();
  // (workgroups of the decode launch: b->decode.groups)
  if (max_splits) *max_splits = b->decode.max_splits;
  return TGE_OK;
}

int tge_batch_set_sparse(tge_batch* b, int enabled, int sink, int window, int stride) {
  if (!b) return fail(TGE_ERR_INVALID, "batch_set_sparse: null batch");
  if (!enabled) {
    b->sp_sink = b->sp_window = b->sp_stride = 0;
    return TGE_OK;
  }
  // set_sparse_config's rules (qwen2.cpp:182-189)
  if (stride < 2) return fail(TGE_ERR_RUNTIME, "sparse: stride must be >= 2");
  if (sink < 0 || window < 1) return fail(TGE_ERR_RUNTIME, "sparse: sink must be >= 0 and window >= 1");
  b->sp_sink = sink;
  b->sp_window = window;
  b->sp_stride = stride;
  return TGE_OK;
}

int tge_batch_set_profiling(tge_batch* b, int enable) {
  if (!b) return fail(TGE_ERR_INVALID, "batch_set_profiling: null batch");
  b->profiling = enable != 0;
  b->prof_used = 0;
  return TGE_OK;
}

int tge_batch_kernel_times(const tge_batch* b, int* calls, float* attention_us,
                           float* merge_us) {
  if (!b || !calls || !attention_us || !merge_us)
    return fail(TGE_ERR_INVALID, "batch_kernel_times: null argument");
  double att = 0.0, mrg = 0.0;
  for (size_t i = 0; i < b->prof_used; ++i) {
    const auto& t = b->prof[i];
    TGE_HIP(hipEventSynchronize(t[2]));
    float x = 0.0f, y = 0.0f;
    TGE_HIP(hipEventElapsedTime(&x, t[0], t[1]));
    TGE_HIP(hipEventElapsedTime(&y, t[1], t[2]));
    att += x;
    mrg += y;
  }
  *calls = (int)b->prof_used;
  *attention_us = (float)(1e3 * att);
  *merge_us = (float)(1e3 * mrg);
  return TGE_OK;
}

namespace {

int check_use(const tge_batch* b, const tge_kv_pool* p, int layer, const char* who) {
  if (!b || !p) return fail(TGE_ERR_INVALID, std::string(who) + ": null argument");
  if (!b->planned) return fail(TGE_ERR_INVALID, std::string(who) + ": batch not planned");
  if (b->kv_heads != p->desc.kv_heads || b->head_dim != p->desc.head_dim ||
      b->pages != p->desc.pages)
    return fail(TGE_ERR_INVALID, std::string(who) + ": batch planned for another pool");
  if (layer < 0 || layer >= p->desc.layers)
    return fail(TGE_ERR_INVALID, std::string(who) + ": layer out of range");
  return TGE_OK;
}

tge::AttnParams attn_params(const tge_batch* b, const tge_kv_pool* p, int layer,
                            const float* q, float* out, const AttnPlan& pl) {
  tge_kv_layer_view v{};
  tge_kv_pool_layer(p, layer, &v);
  tge::AttnParams a{};
  a.pool = v.k;
  a.block_bytes = (uint32_t)p->geom.block_bytes;
  a.sessions = reinterpret_cast<const tge::SessionRec*>(b->dev + b->off_sessions);
  a.work = reinterpret_cast<const tge::WorkRec*>(pl.dev);
  a.wg_first = pl.wg_first.empty() ? nullptr : reinterpret_cast<const int*>(pl.dev + pl.off_first);
  a.tables = reinterpret_cast<const int*>(b->dev + b->off_tables);
  a.sp_sink = b->sp_sink;
  a.sp_window = b->sp_window;
  a.sp_stride = b->sp_stride;
  a.q = q;
  a.out = out;
  a.part_o = pl.part_o;
  a.part_ml = pl.part_ml;
  a.rows_cap = 16 * pl.row_groups;
  a.kv_heads = b->kv_heads;
  a.q_heads = b->q_heads;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)b->head_dim));
  return a;
}

int run_attention(const tge_batch* b, const tge_kv_pool* p, int layer, const float* q,
                  float* out, void* stream, const AttnPlan& pl, bool decode) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  const tge::AttnParams a = attn_params(b, p, layer, q, out, pl);
  std::array<hipEvent_t, 3>* ev = nullptr;
  if (b->profiling) {
    tge_batch* mb = const_cast<tge_batch*>(b);
    if (mb->prof_used == mb->prof.size()) {
      std::array<hipEvent_t, 3> t{nullptr, nullptr, nullptr};
      for (hipEvent_t& e : t) {
        const hipError_t err = hipEventCreate(&e);
        if (err != hipSuccess) {
          for (hipEvent_t x : t)
            if (x) (void)hipEventDestroy(x);
          return fail(TGE_ERR_DEVICE, std::string("hipEventCreate: ") + hipGetErrorString(err));
        }
      }
      mb->prof.push_back(t);
    }
    ev = &mb->prof[mb->prof_used++];
    TGE_HIP(hipEventRecord((*ev)[0], st));
  }
  if (decode) {
    TGE_HIP(tge::launch_decode(p->desc.format, p->desc.scale_format == TGE_SCALE_F32, b->head_dim,
                               pl.row_groups, pl.groups, a, st));
  } else {
    TGE_HIP(tge::launch_prefill(p->desc.format, p->desc.scale_format == TGE_SCALE_F32,
                                b->head_dim, (int)pl.work.size(), a, st));
  }
  if (ev) TGE_HIP(hipEventRecord((*ev)[1], st));
  if (!pl.reduce.empty()) {
    tge::ReduceParams r{};
    r.sessions = a.sessions;
    r.items = reinterpret_cast<const tge::ReduceRec*>(pl.dev + pl.off_reduce);
    r.part_o = pl.part_o;
    r.part_ml = pl.part_ml;
    r.out = out;
    r.rows_cap = a.rows_cap;
    r.q_heads = b->q_heads;
    TGE_HIP(tge::launch_reduce(b->head_dim, (int)pl.reduce.size(), pl.max_splits, r, st));
  }
  if (ev) TGE_HIP(hipEventRecord((*ev)[2], st));
  return TGE_OK;
}

}  // namespace

int tge_kv_append(const tge_batch* b, tge_kv_pool* p, int layer, const float* k,
                  const float* v, void* stream) {
  int s = check_use(b, p, layer, "kv_append");
  if (s != TGE_OK) return s;
  if (!k || !v) return fail(TGE_ERR_INVALID, "kv_append: null k/v");
  tge_kv_layer_view view{};
  tge_kv_pool_layer(p, layer, &view);
  tge::AppendParams a{};
  a.k = k;
  a.v = v;
  a.pool = view.k;
  a.geom = p->geom;
  a.rows = reinterpret_cast<const tge::RowRec*>(b->dev + b->off_rows);
  a.n_rows = (int)b->rows.size();
  a.kv_heads = b->kv_heads;
  a.head_dim = b->head_dim;
  a.scale_f32 = p->desc.scale_format == TGE_SCALE_F32;
  TGE_HIP(tge::launch_kv_append(p->desc.format, a, static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

int tge_kv_append_rope(const tge_batch* b, tge_kv_pool* p, int layer,
                       const tge_rope_append_args* r, void* stream) {
  int s = check_use(b, p, layer, "kv_append_rope");
  if (s != TGE_OK) return s;
  if (!r || !r->k || !r->v || !r->rope_cos || !r->rope_sin)
    return fail(TGE_ERR_INVALID, "kv_append_rope: null k/v/tables");
  if (r->q && !r->q_out) return fail(TGE_ERR_INVALID, "kv_append_rope: q without q_out");
  int max_pos = -1;
  for (const auto& row : b->rows) max_pos = std::max(max_pos, row.pos);
  if (max_pos >= r->rope_positions)
    return fail(TGE_ERR_INVALID, "kv_append_rope: a position is past the rotary tables");
  tge_kv_layer_view view{};
  tge_kv_pool_layer(p, layer, &view);
  tge::AppendParams a{};
  a.k = r->k;
  a.v = r->v;
  a.pool = view.k;
  a.geom = p->geom;
  a.rows = reinterpret_cast<const tge::RowRec*>(b->dev + b->off_rows);
  a.n_rows = (int)b->rows.size();
  a.kv_heads = b->kv_heads;
  a.head_dim = b->head_dim;
  a.scale_f32 = p->desc.scale_format == TGE_SCALE_F32;
  a.q = r->q;
  a.q_out = r->q_out;
  a.q_bias = r->q_bias;
  a.k_bias = r->k_bias;
  a.v_bias = r->v_bias;
  a.rope_cos = r->rope_cos;
  a.rope_sin = r->rope_sin;
  a.q_heads = b->q_heads;
  a.rope_fma = r->rope_fma ? 1 : 0;
  TGE_HIP(tge::launch_kv_append_rope(p->desc.format, a, static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

int tge_rope_tables(int head_dim, int positions, float theta, float attn_factor,
                    const float* factors, float* cos_out, float* sin_out) {
  if (head_dim <= 0 || (head_dim & 1) || positions < 0 || !cos_out || !sin_out)
    return fail(TGE_ERR_INVALID, "rope_tables: bad arguments");
  const int half = head_dim / 2;
  std::vector<float> freq((size_t)half);
  for (int i = 0; i < half; ++i) {
    freq[(size_t)i] = std::pow(theta, -2.0f * (float)i / (float)head_dim);
    if (factors) {
      if (!(factors[i] > 0.0f)) return fail(TGE_ERR_INVALID, "rope_tables: non-positive factor");
      freq[(size_t)i] /= factors[i];
    }
  }
  for (int pos = 0; pos < positions; ++pos) {
    for (int i = 0; i < half; ++i) {
      const float angle = (float)pos * freq[(size_t)i];
      cos_out[(size_t)pos * half + i] = std::cos(angle) * attn_factor;
      sin_out[(size_t)pos * half + i] = std::sin(angle) * attn_factor;
    }
  }
  return TGE_OK;
}

int tge_decode_attention(const tge_batch* b, const tge_kv_pool* p, int layer,
                         const float* q, float* out, void* stream) {
  int s = check_use(b, p, layer, "decode_attention");
  if (s != TGE_OK) return s;
  if (!q || !out) return fail(TGE_ERR_INVALID, "decode_attention: null q/out");
  if (!b->decode.built)
    return fail(TGE_ERR_INVALID, "decode_attention: n_new * group exceeds 64 rows");
  return run_attention(b, p, layer, q, out, stream, b->decode, true);
}

int tge_prefill_attention(const tge_batch* b, const tge_kv_pool* p, int layer,
                          const float* q, float* out, void* stream) {
  int s = check_use(b, p, layer, "prefill_attention");
  if (s != TGE_OK) return s;
  if (!q || !out) return fail(TGE_ERR_INVALID, "prefill_attention: null q/out");
  // The prefill lists are built on first use after each plan (decode-only
  // steps never pay for them) and reused by every layer.
  tge_batch* mb = const_cast<tge_batch*>(b);
  if (!mb->prefill.built) {
    build_prefill(mb, mb->prefill, 0);
    s = upload_plan(mb->prefill, b->head_dim, static_cast<hipStream_t>(stream));
    if (s != TGE_OK) return s;
  }
  return run_attention(b, p, layer, q, out, stream, b->prefill, false);
}

int tge_batch_attention(const tge_batch* b, const tge_kv_pool* p, int layer, const float* q,
                        float* out, void* stream) {
  int s = check_use(b, p, layer, "batch_attention");
  if (s != TGE_OK) return s;
  if (!q || !out) return fail(TGE_ERR_INVALID, "batch_attention: null q/out");
  tge_batch* mb = const_cast<tge_batch*>(b);
  int n_dec = 0, n_pf = 0;
  for (const auto& sr : b->sessions) (decode_session(b, sr) ? n_dec : n_pf)++;
  if (n_pf == 0) return tge_decode_attention(b, p, layer, q, out, stream);
  if (n_dec == 0) return tge_prefill_attention(b, p, layer, q, out, stream);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!mb->mix_built) {
    // Built on first use after each plan, reused by every layer.
    int max_rows = 0;
    for (const auto& sr : b->sessions)
      if (decode_session(b, sr)) max_rows = std::max(max_rows, sr.n_new * b->group);
    const int rg = std::max(1, std::min(4, (max_rows + 15) / 16));
    build_decode(mb, resident_groups(p->desc.format, p->desc.scale_format == TGE_SCALE_F32,
                                     b->head_dim, rg),
                 mb->mix_decode, 1);
    s = upload_plan(mb->mix_decode, b->head_dim, st);
    if (s != TGE_OK) return s;
    build_prefill(mb, mb->mix_prefill, 2);
    s = upload_plan(mb->mix_prefill, b->head_dim, st);
    if (s != TGE_OK) return s;
    mb->mix_built = true;
  }
  // Long chunks first: the prefill tiles are MFMA-bound, the persistent
  // decode workgroups HBM-bound; both write disjoint rows of `out`.
  s = run_attention(b, p, layer, q, out, stream, b->mix_prefill, false);
  if (s != TGE_OK) return s;
  return run_attention(b, p, layer, q, out, stream, b->mix_decode, true);
}

int tge_kv_gather(const tge_batch* b, const tge_kv_pool* p, int layer, int session,
                  int count, void* k_rows, void* v_rows, void* k_scales, void* v_scales,
                  void* stream) {
  int s = check_use(b, p, layer, "kv_gather");
  if (s != TGE_OK) return s;
  if (session < 0 || session >= (int)b->sessions.size())
    return fail(TGE_ERR_INVALID, "kv_gather: session out of range");
  const tge::SessionRec& sr = b->sessions[session];
  if (count < 0 || count > sr.ctx + sr.n_new)
    return fail(TGE_ERR_INVALID, "kv_gather: count beyond the session's positions");
  if (!k_rows || !v_rows) return fail(TGE_ERR_INVALID, "kv_gather: null rows");
  const bool i8 = p->desc.format == TGE_KV_I8;
  if (i8 && (!k_scales || !v_scales)) return fail(TGE_ERR_INVALID, "kv_gather: null scales");
  tge_kv_layer_view view{};
  tge_kv_pool_layer(p, layer, &view);
  tge::GatherParams g{};
  g.pool = view.k;
  g.geom = p->geom;
  g.table = reinterpret_cast<const int*>(b->dev + b->off_tables) + sr.table_off;
  g.count = count;
  g.kv_heads = b->kv_heads;
  g.head_dim = b->head_dim;
  g.scale_bytes = p->desc.scale_format == TGE_SCALE_F32 ? 4 : 2;
  g.k_rows = k_rows;
  g.v_rows = v_rows;
  g.k_scales = i8 ? k_scales : nullptr;
  g.v_scales = i8 ? v_scales : nullptr;
  TGE_HIP(tge::launch_kv_gather(p->desc.format, g, static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

}  // extern "C"
