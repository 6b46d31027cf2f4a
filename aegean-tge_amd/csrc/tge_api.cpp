// C ABI of the gfx950 paged-KV path: backend bring-up, page pools, per-step
// batch plans and the kernel entry points. See include/tge_kv.h.
#include "tge_kv.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <array>
#include <vector>

#include "../host/plan.hpp"
#include "tge_common.h"
#include "tge_error.h"
#include "tge_kernels.h"

namespace {

thread_local std::string g_last_error;

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

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

}  // namespace

struct tge_kv_pool {
  tge_kv_pool_desc desc{};
  void* blocks = nullptr;   // layers x (pages * kv_heads) page blocks
  int bd = 0;               // block width (dims per token of a page block)
  tge::BlockGeom geom{};
  size_t layer_blocks = 0;  // pages * kv_heads
  size_t bytes = 0;
};

namespace {

// HIP behind the planner's memory interface: allocation failures for lack
// of memory report TGE_ERR_CAPACITY, other HIP failures TGE_ERR_DEVICE.
struct HipMem final : tge::plan::MemOps {
  static int status(hipError_t e, const char* what) {
    if (e == hipSuccess) return TGE_OK;
    return fail(e == hipErrorOutOfMemory ? TGE_ERR_CAPACITY : TGE_ERR_DEVICE,
                std::string(what) + ": " + hipGetErrorString(e));
  }
  // (coherent: the plan upload kernel reads it over the bus)
  int host_alloc(char** p, size_t n) override {
    return status(hipHostMalloc(reinterpret_cast<void**>(p), n, hipHostMallocCoherent),
                  "hipHostMalloc");
  }
  void host_free(char* p) override { (void)hipHostFree(p); }
  int dev_alloc(char** p, size_t n) override {
    return status(hipMalloc(reinterpret_cast<void**>(p), n), "hipMalloc");
  }
  void dev_free(char* p) override { (void)hipFree(p); }
  // A kernel copies the pinned staging buffer (no DMA-engine hand-offs on
  // the launch stream); where the runtime gives no device address for it,
  // a DMA copy.
  int copy_to_device(char* d, const char* h, size_t n, void* st) override {
    void* hd = nullptr;
    if (hipHostGetDevicePointer(&hd, const_cast<char*>(h), 0) == hipSuccess && hd)
      return status(tge::launch_upload(d, static_cast<const char*>(hd), n, static_cast<hipStream_t>(st)),
                    "plan upload");
    (void)hipGetLastError();  // (clear the failed lookup)
    return status(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, static_cast<hipStream_t>(st)),
                  "hipMemcpyAsync");
  }
  int record(void** ev, void* st) override {
    if (!*ev) {
      hipEvent_t e = nullptr;
      const int s = status(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
      if (s != TGE_OK) return s;
      *ev = e;
    }
    return status(hipEventRecord(static_cast<hipEvent_t>(*ev), static_cast<hipStream_t>(st)),
                  "hipEventRecord");
  }
  int wait_event(void* ev) override {
    return status(hipEventSynchronize(static_cast<hipEvent_t>(ev)), "hipEventSynchronize");
  }
  int wait_stream(void* st) override {
    return status(hipStreamSynchronize(static_cast<hipStream_t>(st)), "hipStreamSynchronize");
  }
  void event_free(void* ev) override { (void)hipEventDestroy(static_cast<hipEvent_t>(ev)); }
};
HipMem g_mem;

// Work lists of one attention kind (decode or prefill) for the current plan,
// their device image and the split-K partial buffers.
struct AttnPlan {
  tge::plan::AttnLists lists;
  bool built = false;
  bool sparse = false;  // decode lists balanced for the static sparse kernel
  tge::plan::Staged image;  // work | reduce | wg_first (plans built after tge_batch_plan)
  // Device base of the lists: `image`, or the batch image's region for the
  // plans tge_batch_plan uploads with the step (one copy per step).
  char* dev = nullptr;
  size_t off_reduce = 0;
  size_t off_first = 0;
  size_t off_app = 0;  // app_first, then app_recs (decode plans that store the new rows)
  tge::plan::Scratch part_o;   // [parts][rows_cap][block width] fp32
  tge::plan::Scratch part_ml;  // [parts][rows_cap][2] fp32
  ~AttnPlan() {
    image.release(g_mem);
    part_o.release(g_mem);
    part_ml.release(g_mem);
  }
};

// A small decode step in one launch (paged_step_kernel): its records, the
// split partials and the per-segment arrival counters (zero between
// launches: each launch's last piece of a segment resets its counter).
struct StepPlan {
  tge::plan::StepLists lists;
  bool built = false;
  char* dev = nullptr;  // records | first-batch page ids, in the batch image
  tge::plan::Scratch part_o, part_ml, counters;
  ~StepPlan() {
    part_o.release(g_mem);
    part_ml.release(g_mem);
    counters.release(g_mem);
  }
};

}  // namespace

struct tge_batch {
  tge::plan::Step step;  // host copy of the plan
  StepPlan small;        // one-launch decode steps (tge_decode_step)
  bool planned = false;
  // The pool's storage the plan was built for (the one-launch step's page
  // batches depend on it).
  int format = 0, scale_format = 0;
  AttnPlan decode, prefill;
  // Mixed steps (tge_batch_attention): the decode kernel over the sessions
  // whose rows fit a decode unit, the prefill kernel over the others.
  AttnPlan mix_decode, mix_prefill;
  bool mix_built = false;
  // arrival counters of the mixed launch: the decode plan's records, then
  // the prefill plan's (zero between launches)
  tge::plan::Scratch mix_counters;
  // Static sparse subset of every attention call (stride 0: dense).
  int sp_sink = 0, sp_window = 0, sp_stride = 0;

  // Device image: sessions | tables | rows (one allocation), pinned staging.
  tge::plan::Staged image;
  size_t off_sessions = 0, off_tables = 0, off_rows = 0;

  // Kernel timing (tge_batch_set_profiling): per attention call since
  // enabling, events before the attention kernel, between it and the merge,
  // and after the merge. Triples are created on demand and reused.
  bool profiling = false;
  std::vector<std::array<hipEvent_t, 3>> prof;
  std::vector<char> prof_merged;  // whether the call launched the split merge kernel
  size_t prof_used = 0;

  ~tge_batch() {
    image.release(g_mem);
    mix_counters.release(g_mem);
    for (auto& t : prof)
      for (hipEvent_t e : t)
        if (e) (void)hipEventDestroy(e);
  }
};

namespace {

// Whether tge_decode_step runs the current plan as one kernel: a small step
// (its lists built), and with a static sparse subset only where the sparse
// variant of the kernel fits its registers.
bool one_kernel_step(const tge_batch* b) {
  return b->small.built &&
         (b->sp_stride == 0 || tge::step_fits(b->format == TGE_KV_I8, b->scale_format == TGE_SCALE_F32,
                                              b->step.block_dims, b->step.max_rows, true));
}

}  // namespace

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

int tge_kv_k_index(int token, int dim, int format) {
  if (format != TGE_KV_F16 && format != TGE_KV_I8) return -1;
  return tge::k_index(token, dim, format == TGE_KV_F16 ? 2 : 1);
}
int tge_kv_v_index(int token, int dim, int format) {
  if (format != TGE_KV_F16 && format != TGE_KV_I8) return -1;
  return tge::v_index(token, dim, format == TGE_KV_F16 ? 2 : 1);
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
  if (d.format != TGE_KV_F16 && d.format != TGE_KV_I8)
    return fail(TGE_ERR_INVALID, "kv_pool_create: unknown format");
  if (tge::block_dims_for(d.head_dim, d.format) == 0)
    return fail(TGE_ERR_INVALID, d.format == TGE_KV_I8
                                     ? "kv_pool_create: int8 head_dim must be a multiple of 32 up to 256"
                                     : "kv_pool_create: head_dim must be a multiple of 4 up to 256");
  if (d.format == TGE_KV_I8 && d.scale_format != TGE_SCALE_F16 &&
      d.scale_format != TGE_SCALE_F32)
    return fail(TGE_ERR_INVALID, "kv_pool_create: unknown scale format");
  const int s = backend_ready();
  if (s != TGE_OK) return fail(s, "kv_pool_create: backend unavailable");

  auto* p = new tge_kv_pool;
  p->desc = d;
  p->bd = tge::block_dims_for(d.head_dim, d.format);
  p->geom = tge::block_geom(d.format, p->bd, d.format == TGE_KV_I8 && d.scale_format == TGE_SCALE_F32);
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
  out->block_dims = p->bd;
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

// Sizes an attention plan's split-K partial buffers (rows of the page
// blocks' width) once its lists are on the device at pl.dev.
int finish_plan(AttnPlan& pl, int block_dims, hipStream_t st) {
  const size_t rows_cap = 16 * (size_t)pl.lists.row_groups;
  const size_t parts = (size_t)std::max(pl.lists.parts, 1);
  int s = pl.part_o.reserve(g_mem, parts * rows_cap * block_dims * sizeof(float), st);
  if (s == TGE_OK) s = pl.part_ml.reserve(g_mem, parts * rows_cap * 2 * sizeof(float), st);
  if (s != TGE_OK) return s;
  pl.built = true;
  return TGE_OK;
}

// Uploads an attention plan's lists on their own (the plans built after
// tge_batch_plan) and sizes its partial buffers.
int upload_plan(AttnPlan& pl, int block_dims, hipStream_t st) {
  pl.built = false;
  const size_t total = tge::plan::image_layout(pl.lists, &pl.off_reduce, &pl.off_first, &pl.off_app);
  int s = pl.image.upload(g_mem, total, st, [&](char* h) {
    tge::plan::write_image(pl.lists, pl.off_reduce, pl.off_first, h, pl.off_app);
  });
  if (s != TGE_OK) return s;
  pl.dev = pl.image.dev;
  return finish_plan(pl, block_dims, st);
}

int device_cus() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

// Resident workgroups of a decode variant on this device (cached): the
// compute units times what the occupancy query allows per unit.
tge::plan::Residency resident_groups(int format, int scale_f32, int head_dim, int row_groups,
                                     bool sparse) {
  static std::mutex mu;
  static std::vector<std::pair<int, tge::plan::Residency>> cache;  // key -> residency
  const int key = (((format * 2 + scale_f32) * 256 + head_dim) * 8 + row_groups) * 2 + sparse;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& kv : cache)
    if (kv.first == key) return kv.second;
  const int cus = device_cus();
  int per_cu = tge::decode_blocks_per_cu(format, scale_f32, head_dim, row_groups, sparse);
  if (per_cu <= 0) per_cu = 1;
  const tge::plan::Residency r{per_cu * cus, cus};
  cache.emplace_back(key, r);
  return r;
}

// Workgroups of the mixed-step kernel's decode role: one per CU. The
// launch lists the decode shares first, so each CU takes one share and its
// other workgroup slot runs prefill tiles from the start: the HBM-bound
// decode streams under the MFMA-bound tiles. (Shares for every slot, two
// decode workgroups per CU, left the tiles to run after the decode: 131-135
// us against 125 us for the c5-shaped mixed step.)
tge::plan::Residency resident_groups_mixed() {
  const int cus = device_cus();
  return tge::plan::Residency{cus, cus};
}

// Builds the lists of a decode plan over the sessions `only` selects
// (0 all, 1 those a decode unit holds), balanced for the decode kernel the
// batch's current sparse setting launches (`mixed`: the decode role of the
// mixed-step kernel).
void build_decode_lists(tge_batch* b, const tge_kv_pool* p, AttnPlan& pl, int only, bool mixed) {
  pl.built = false;
  int max_rows = 0;
  for (const auto& sr : b->step.sessions)
    if (tge::plan::take_session(b->step, sr, only))
      max_rows = std::max(max_rows, sr.n_new * b->step.group);
  const int rg = std::max(1, std::min(4, (max_rows + 15) / 16));
  const bool sparse = b->sp_stride > 0;
  const int sf32 = p->desc.scale_format == TGE_SCALE_F32;
  tge::plan::build_decode(b->step,
                          mixed ? resident_groups_mixed()
                                : resident_groups(p->desc.format, sf32, b->step.block_dims, rg, sparse),
                          pl.lists, only);
  // (the dense decode kernel of tge_decode_step stores the step's new rows
  // where its variant can)
  if (!mixed && !sparse)
    tge::plan::build_decode_appends(b->step, pl.lists,
                                    tge::decode_app_waves(p->desc.format, sf32, b->step.block_dims, rg),
                                    tge::decode_app_rows(b->step.block_dims));
  pl.sparse = sparse;
}

// The same, uploaded on its own (a plan built after tge_batch_plan).
int build_decode_plan(tge_batch* b, const tge_kv_pool* p, AttnPlan& pl, int only, hipStream_t st,
                      bool mixed = false) {
  build_decode_lists(b, p, pl, only, mixed);
  return upload_plan(pl, b->step.block_dims, st);
}

}  // namespace

namespace {

// The partial and counter buffers of a small decode step's one-launch
// lists, once the lists are on the device at sp.dev (counters zeroed when
// allocated).
int finish_step_plan(tge_batch* b, hipStream_t st) {
  StepPlan& sp = b->small;
  const auto& L = sp.lists;
  const size_t rows_cap = 16 * (size_t)L.row_groups;
  int s = TGE_OK;
  const size_t parts = (size_t)std::max(L.parts, 1);
  s = sp.part_o.reserve(g_mem, parts * rows_cap * b->step.block_dims * sizeof(float), st);
  if (s == TGE_OK) s = sp.part_ml.reserve(g_mem, parts * rows_cap * 2 * sizeof(float), st);
  if (s != TGE_OK) return s;
  const size_t had = sp.counters.bytes;
  s = sp.counters.reserve(g_mem, (size_t)std::max(L.segments, 1) * sizeof(int), st);
  if (s != TGE_OK) return s;
  if (sp.counters.bytes != had)
    TGE_HIP(hipMemsetAsync(sp.counters.dev, 0, sp.counters.bytes, st));
  sp.built = true;
  return TGE_OK;
}

}  // namespace

int tge_batch_plan(tge_batch* b, const tge_kv_pool* pool, const tge_batch_desc* d,
                   void* stream) {
  if (!b || !pool || !d) return fail(TGE_ERR_INVALID, "batch_plan: null argument");
  const int hd = pool->desc.head_dim;
  const char* msg = nullptr;
  b->planned = false;
  int s = tge::plan::build_step(b->step, d->n_sessions, d->ctx, d->n_new, d->table_offsets,
                                d->page_ids, d->q_heads, pool->desc.kv_heads, hd,
                                pool->desc.pages, &msg);
  if (s != TGE_OK) return fail(s, msg ? msg : "batch_plan: invalid description");
  tge::plan::Step& st = b->step;
  b->format = pool->desc.format;
  b->scale_format = pool->desc.scale_format;
  b->prefill.built = false;
  b->decode.built = false;
  b->mix_built = false;

  hipStream_t hs = static_cast<hipStream_t>(stream);
  // The step's lists are built on the host first and go up in one copy:
  // [ sessions | tables | rows | attention lists | step records |
  // first-batch page ids ]. The attention lists are the decode lists when
  // every session's rows fit a decode unit (one upload per step serves every
  // layer), the block-prefill lists when none does (a prompt chunk); a step
  // mixing both builds its plans on first use.
  const bool dec = st.max_rows <= tge::max_unit_rows(st.block_dims);
  bool pre = !dec;
  for (const auto& sr : st.sessions) pre = pre && !tge::plan::decode_session(st, sr);
  if (dec) build_decode_lists(b, pool, b->decode, 0, false);
  if (pre) {
    b->prefill.built = false;
    tge::plan::build_prefill(st, device_cus(), b->prefill.lists, 0,
                             tge::prefill_halves(pool->desc.format, st.block_dims),
                             pool->desc.format == TGE_KV_I8);
  }
  b->small.built = false;
  const bool small = tge::plan::build_step_lists(st, pool->desc.format == TGE_KV_I8,
                                                 pool->desc.scale_format == TGE_SCALE_F32,
                                                 b->small.lists);
  const auto& SL = b->small.lists;
  const size_t o_sess = 0;
  const size_t o_tab = align_up(o_sess + st.sessions.size() * sizeof(tge::SessionRec));
  const size_t o_rows = align_up(o_tab + st.tables.size() * sizeof(int));
  const size_t o_dec = align_up(o_rows + st.rows.size() * sizeof(tge::RowRec));
  AttnPlan& dp = dec ? b->decode : b->prefill;  // (the eager attention plan, if any)
  const bool eager = dec || pre;
  const size_t dec_bytes =
      eager ? tge::plan::image_layout(dp.lists, &dp.off_reduce, &dp.off_first, &dp.off_app) : 0;
  const size_t o_step = align_up(o_dec + dec_bytes);
  const size_t rbytes = small ? SL.recs.size() * sizeof(tge::StepRec) : 0;
  const size_t ibytes = small ? SL.first_ids.size() * sizeof(int) : 0;
  const size_t total = o_step + rbytes + ibytes;
  s = b->image.upload(g_mem, total, hs, [&](char* h) {
    std::memcpy(h + o_sess, st.sessions.data(), st.sessions.size() * sizeof(tge::SessionRec));
    if (!st.tables.empty()) std::memcpy(h + o_tab, st.tables.data(), st.tables.size() * sizeof(int));
    std::memcpy(h + o_rows, st.rows.data(), st.rows.size() * sizeof(tge::RowRec));
    if (eager) tge::plan::write_image(dp.lists, dp.off_reduce, dp.off_first, h + o_dec, dp.off_app);
    if (small) {
      std::memcpy(h + o_step, SL.recs.data(), rbytes);
      std::memcpy(h + o_step + rbytes, SL.first_ids.data(), ibytes);
    }
  });
  if (s != TGE_OK) return s;
  b->off_sessions = o_sess;
  b->off_tables = o_tab;
  b->off_rows = o_rows;
  if (eager) {
    dp.dev = b->image.dev + o_dec;
    s = finish_plan(dp, st.block_dims, hs);
    if (s != TGE_OK) return s;
  }
  if (small) {
    b->small.dev = b->image.dev + o_step;
    s = finish_step_plan(b, hs);
    if (s != TGE_OK) return s;
  }
  b->planned = true;
  return TGE_OK;
}

int tge_batch_info(const tge_batch* b, int* rows, int* work_items, int* max_splits) {
  if (!b || !b->planned) return fail(TGE_ERR_INVALID, "batch_info: batch not planned");
  // Decode figures of the current plan; a plan whose rows exceed a decode
  // unit has none (0, 0).
  const bool dec = b->decode.built;
  if (rows) *rows = (int)b->step.rows.size();
  if (work_items) *work_items = dec ? (int)b->decode.lists.work.size() : 0;
  if (max_splits) *max_splits = dec ? b->decode.lists.max_splits : 0;
  return TGE_OK;
}

int tge_batch_step_info(const tge_batch* b, int* workgroups, int* max_pieces) {
  if (!b || !b->planned) return fail(TGE_ERR_INVALID, "batch_step_info: batch not planned");
  const bool one = one_kernel_step(b);
  if (workgroups) *workgroups = one ? (int)b->small.lists.recs.size() : 0;
  if (max_pieces) *max_pieces = one ? b->small.lists.max_pieces : 0;
  return TGE_OK;
}

int tge_batch_decode_stores_rows(const tge_batch* b, int* stores) {
  if (!b || !b->planned || !stores) return fail(TGE_ERR_INVALID, "batch_decode_stores_rows: batch not planned");
  *stores = !b->small.built && b->sp_stride == 0 && b->decode.built && b->decode.lists.app_waves > 0;
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
    if (b->prof_merged[i]) TGE_HIP(hipEventElapsedTime(&y, t[1], t[2]));
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
  if (b->step.kv_heads != p->desc.kv_heads || b->step.head_dim != p->desc.head_dim ||
      b->step.pages != p->desc.pages || b->format != p->desc.format ||
      b->scale_format != p->desc.scale_format)
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
  a.sessions = reinterpret_cast<const tge::SessionRec*>(b->image.dev + b->off_sessions);
  a.work = reinterpret_cast<const tge::WorkRec*>(pl.dev);
  a.wg_first = pl.lists.wg_first.empty() ? nullptr : reinterpret_cast<const int*>(pl.dev + pl.off_first);
  a.tables = reinterpret_cast<const int*>(b->image.dev + b->off_tables);
  a.sp_sink = b->sp_sink;
  a.sp_window = b->sp_window;
  a.sp_stride = b->sp_stride;
  a.q = q;
  a.out = out;
  a.part_o = reinterpret_cast<float*>(pl.part_o.dev);
  a.part_ml = reinterpret_cast<float*>(pl.part_ml.dev);
  a.rows_cap = 16 * pl.lists.row_groups;
  a.kv_heads = b->step.kv_heads;
  a.q_heads = b->step.q_heads;
  a.dims = b->step.head_dim;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)b->step.head_dim));
  return a;
}

// The next triple of timing events of an attention call while profiling is
// on (created on demand and reused), else null.
int profile_events(tge_batch* b, std::array<hipEvent_t, 3>** ev) {
  *ev = nullptr;
  if (!b->profiling) return TGE_OK;
  if (b->prof_used == b->prof.size()) {
    std::array<hipEvent_t, 3> t{nullptr, nullptr, nullptr};
    for (hipEvent_t& e : t) {
      const hipError_t err = hipEventCreate(&e);
      if (err != hipSuccess) {
        for (hipEvent_t x : t)
          if (x) (void)hipEventDestroy(x);
        return fail(TGE_ERR_DEVICE, std::string("hipEventCreate: ") + hipGetErrorString(err));
      }
    }
    b->prof.push_back(t);
    b->prof_merged.push_back(0);
  }
  b->prof_merged[b->prof_used] = 0;
  *ev = &b->prof[b->prof_used++];
  return TGE_OK;
}

// app_k/app_v (dense decode only): the step's new K/V rows, stored by the
// decode launch itself (tge_decode_step).
int run_attention(const tge_batch* b, const tge_kv_pool* p, int layer, const float* q,
                  float* out, void* stream, const AttnPlan& pl, bool decode,
                  const float* app_k = nullptr, const float* app_v = nullptr) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  tge::AttnParams a = attn_params(b, p, layer, q, out, pl);
  if (app_k) {
    a.app_k = app_k;
    a.app_v = app_v;
    a.app_first = reinterpret_cast<const int*>(pl.dev + pl.off_app);
    a.app_recs = a.app_first + pl.lists.app_first.size();
  }
  std::array<hipEvent_t, 3>* ev = nullptr;
  const int ps = profile_events(const_cast<tge_batch*>(b), &ev);
  if (ps != TGE_OK) return ps;
  if (ev) TGE_HIP(hipEventRecord((*ev)[0], st));
  const bool merge_kernel = !pl.lists.reduce.empty();
  if (decode) {
    TGE_HIP(tge::launch_decode(p->desc.format, p->desc.scale_format == TGE_SCALE_F32, b->step.block_dims,
                               pl.lists.row_groups, pl.lists.groups, a, st));
  } else {
    TGE_HIP(tge::launch_prefill(p->desc.format, p->desc.scale_format == TGE_SCALE_F32,
                                b->step.block_dims, (int)pl.lists.work.size(), pl.lists.tile_rows,
                                a, st));
  }
  if (ev) {
    TGE_HIP(hipEventRecord((*ev)[1], st));
    const_cast<tge_batch*>(b)->prof_merged[b->prof_used - 1] = merge_kernel;
  }
  if (merge_kernel) {
    tge::ReduceParams r{};
    r.items = reinterpret_cast<const tge::ReduceRec*>(pl.dev + pl.off_reduce);
    r.part_o = reinterpret_cast<const float*>(pl.part_o.dev);
    r.part_ml = reinterpret_cast<const float*>(pl.part_ml.dev);
    r.out = out;
    r.rows_cap = a.rows_cap;
    r.q_heads = b->step.q_heads;
    r.dims = b->step.head_dim;
    TGE_HIP(tge::launch_reduce(b->step.block_dims, (int)pl.lists.reduce.size(), pl.lists.max_splits, r, st));
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
  a.rows = reinterpret_cast<const tge::RowRec*>(b->image.dev + b->off_rows);
  a.n_rows = (int)b->step.rows.size();
  a.kv_heads = b->step.kv_heads;
  a.head_dim = p->bd;
  a.dims = b->step.head_dim;
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
  // (a lane rotates 8 dims against the 8 half a head away: the halves must
  // be whole runs of 8)
  if (b->step.head_dim % 16 != 0)
    return fail(TGE_ERR_INVALID, "kv_append_rope: head_dim must be a multiple of 16");
  int max_pos = -1;
  for (const auto& row : b->step.rows) max_pos = std::max(max_pos, row.pos);
  if (max_pos >= r->rope_positions)
    return fail(TGE_ERR_INVALID, "kv_append_rope: a position is past the rotary tables");
  tge_kv_layer_view view{};
  tge_kv_pool_layer(p, layer, &view);
  tge::AppendParams a{};
  a.k = r->k;
  a.v = r->v;
  a.pool = view.k;
  a.geom = p->geom;
  a.rows = reinterpret_cast<const tge::RowRec*>(b->image.dev + b->off_rows);
  a.n_rows = (int)b->step.rows.size();
  a.kv_heads = b->step.kv_heads;
  a.head_dim = p->bd;
  a.dims = b->step.head_dim;
  a.scale_f32 = p->desc.scale_format == TGE_SCALE_F32;
  a.q = r->q;
  a.q_out = r->q_out;
  a.q_bias = r->q_bias;
  a.k_bias = r->k_bias;
  a.v_bias = r->v_bias;
  a.rope_cos = r->rope_cos;
  a.rope_sin = r->rope_sin;
  a.q_heads = b->step.q_heads;
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
    return fail(TGE_ERR_INVALID, "decode_attention: n_new * group exceeds a decode unit (64 rows, 48 at head_dim > 128)");
  if (b->decode.sparse != (b->sp_stride > 0)) {
    // the sparse setting changed after planning: rebalance for its kernel
    s = build_decode_plan(const_cast<tge_batch*>(b), p, const_cast<tge_batch*>(b)->decode, 0,
                          static_cast<hipStream_t>(stream));
    if (s != TGE_OK) return s;
  }
  return run_attention(b, p, layer, q, out, stream, b->decode, true);
}

int tge_decode_step(const tge_batch* b, tge_kv_pool* p, int layer, const float* q,
                    const float* k, const float* v, float* out, void* stream) {
  int s = check_use(b, p, layer, "decode_step");
  if (s != TGE_OK) return s;
  if (!q || !k || !v || !out) return fail(TGE_ERR_INVALID, "decode_step: null q/k/v/out");
  if (!b->decode.built)
    return fail(TGE_ERR_INVALID, "decode_step: n_new * group exceeds a decode unit (64 rows, 48 at head_dim > 128)");
  if (b->sp_stride > 0 && !one_kernel_step(b)) {
    // a static sparse step the one-launch kernel does not take: the append,
    // then the sparse decode kernel and its split merge
    s = tge_kv_append(b, p, layer, k, v, stream);
    if (s != TGE_OK) return s;
    return tge_decode_attention(b, p, layer, q, out, stream);
  }
  if (!b->small.built) {
    // a large step: the decode kernel, which writes the new rows into the
    // pages it reads as they land and stores them into the pool, then its
    // split merge
    if (b->decode.sparse) {
      s = build_decode_plan(const_cast<tge_batch*>(b), p, const_cast<tge_batch*>(b)->decode, 0,
                            static_cast<hipStream_t>(stream));
      if (s != TGE_OK) return s;
    }
    if (b->decode.lists.app_waves > 0)
      return run_attention(b, p, layer, q, out, stream, b->decode, true, k, v);
    s = tge_kv_append(b, p, layer, k, v, stream);  // (no new-row lists: the variant or rows per wave)
    if (s != TGE_OK) return s;
    return run_attention(b, p, layer, q, out, stream, b->decode, true);
  }
  const StepPlan& sp = b->small;
  tge_kv_layer_view view{};
  tge_kv_pool_layer(p, layer, &view);
  tge::StepParams a{};
  a.app.k = k;
  a.app.v = v;
  a.app.pool = view.k;
  a.app.geom = p->geom;
  a.app.kv_heads = b->step.kv_heads;
  a.app.head_dim = p->bd;
  a.app.dims = b->step.head_dim;
  a.app.scale_f32 = p->desc.scale_format == TGE_SCALE_F32;
  a.app.q_heads = b->step.q_heads;
  a.recs = reinterpret_cast<const tge::StepRec*>(sp.dev);
  a.first_ids = reinterpret_cast<const int*>(sp.dev + sp.lists.recs.size() * sizeof(tge::StepRec));
  a.tables = reinterpret_cast<const int*>(b->image.dev + b->off_tables);
  a.q = q;
  a.out = out;
  a.part_o = reinterpret_cast<float*>(sp.part_o.dev);
  a.part_ml = reinterpret_cast<float*>(sp.part_ml.dev);
  a.counters = reinterpret_cast<int*>(sp.counters.dev);
  a.rows_cap = 16 * sp.lists.row_groups;
  a.group = b->step.group;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)b->step.head_dim));
  a.sp_sink = b->sp_sink;
  a.sp_window = b->sp_window;
  a.sp_stride = b->sp_stride;
  TGE_HIP(tge::launch_step(p->desc.format, p->desc.scale_format == TGE_SCALE_F32,
                           b->step.block_dims, sp.lists.row_groups, (int)sp.lists.recs.size(), a,
                           static_cast<hipStream_t>(stream)));
  return TGE_OK;
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
    tge::plan::build_prefill(mb->step, device_cus(), mb->prefill.lists, 0,
                             tge::prefill_halves(p->desc.format, b->step.block_dims),
                             p->desc.format == TGE_KV_I8);
    s = upload_plan(mb->prefill, b->step.block_dims, static_cast<hipStream_t>(stream));
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
  for (const auto& sr : b->step.sessions) (tge::plan::decode_session(b->step, sr) ? n_dec : n_pf)++;
  if (n_pf == 0) return tge_decode_attention(b, p, layer, q, out, stream);
  if (n_dec == 0) return tge_prefill_attention(b, p, layer, q, out, stream);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool sparse = b->sp_stride > 0;
  if (!mb->mix_built || mb->mix_decode.sparse != sparse) {
    // Built on first use after each plan (and after the sparse setting
    // changes), reused by every layer: one launch, the decode shares
    // balanced for the mixed kernel.
    s = build_decode_plan(mb, p, mb->mix_decode, 1, st, true);
    if (s != TGE_OK) return s;
    tge::plan::build_prefill(mb->step, device_cus(), mb->mix_prefill.lists, 2);
    s = upload_plan(mb->mix_prefill, b->step.block_dims, st);
    if (s != TGE_OK) return s;
    const size_t n = mb->mix_decode.lists.reduce.size() + mb->mix_prefill.lists.reduce.size();
    const size_t had = mb->mix_counters.bytes;
    s = mb->mix_counters.reserve(g_mem, std::max<size_t>(n, 1) * sizeof(int), st);
    if (s != TGE_OK) return s;
    if (mb->mix_counters.bytes != had)
      TGE_HIP(hipMemsetAsync(mb->mix_counters.dev, 0, mb->mix_counters.bytes, st));
    mb->mix_built = true;
  }
  // One launch: the decode shares first, then the prefill tiles; each
  // plan's split records are merged in the launch (arrival counters).
  tge::AttnParams dec = attn_params(b, p, layer, q, out, b->mix_decode);
  tge::AttnParams pf = attn_params(b, p, layer, q, out, b->mix_prefill);
  int* counters = reinterpret_cast<int*>(b->mix_counters.dev);
  dec.reduce = reinterpret_cast<const tge::ReduceRec*>(b->mix_decode.dev + b->mix_decode.off_reduce);
  dec.counters = counters;
  pf.reduce = reinterpret_cast<const tge::ReduceRec*>(b->mix_prefill.dev + b->mix_prefill.off_reduce);
  pf.counters = counters + b->mix_decode.lists.reduce.size();
  std::array<hipEvent_t, 3>* ev = nullptr;
  s = profile_events(mb, &ev);
  if (s != TGE_OK) return s;
  if (ev) TGE_HIP(hipEventRecord((*ev)[0], st));
  TGE_HIP(tge::launch_mixed(p->desc.format, p->desc.scale_format == TGE_SCALE_F32, b->step.block_dims,
                            b->mix_decode.lists.row_groups, b->mix_decode.lists.groups,
                            (int)b->mix_prefill.lists.work.size(), dec, pf, st));
  if (ev) {
    TGE_HIP(hipEventRecord((*ev)[1], st));
    TGE_HIP(hipEventRecord((*ev)[2], st));
  }
  return TGE_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Decode attention that allocates nothing (tge_decode_attention_static): the
// step's plan image and its split-K partials live in `scratch`, one array
// per device that the library holds until the process ends. In host code
// `scratch` names a host-side stand-in, never device memory: every host use
// goes through the device address hipGetSymbolAddress returns for the
// current device (static_scratch below).
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kStaticImageBytes = size_t(4) << 20;    // sessions | tables | work lists
constexpr size_t kStaticScratchBytes = size_t(32) << 20;  // image, then partials
constexpr int kStaticDevices = 64;

__device__ __align__(256) char scratch[kStaticScratchBytes];

std::mutex g_static_mu;
char* g_static[kStaticDevices] = {};  // device address of `scratch` per device

// The device address of this device's `scratch`, looked up with that device
// current on the first call that succeeds (a failed lookup is not kept: the
// next call tries again).
int static_scratch(char** out) {
  int dev = 0;
  TGE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kStaticDevices)
    return fail(TGE_ERR_DEVICE, "decode_attention_static: device index beyond the table");
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (!g_static[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TGE_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") +
                                      hipGetErrorString(e));
    g_static[dev] = static_cast<char*>(p);
  }
  *out = g_static[dev];
  return TGE_OK;
}

}  // namespace

extern "C" {

int tge_decode_attention_static(const tge_batch_desc* d, const tge_kv_pool* p, int layer,
                                const float* q, float* out, void* stream) {
  if (!d || !p || !q || !out) return fail(TGE_ERR_INVALID, "decode_attention_static: null argument");
  if (layer < 0 || layer >= p->desc.layers)
    return fail(TGE_ERR_INVALID, "decode_attention_static: layer out of range");
  int s = backend_ready();
  if (s != TGE_OK) return fail(s, "decode_attention_static: backend unavailable");
  {
    // The plan is copied from host memory at each call: a captured copy
    // would replay whatever the buffer holds later, so capture is refused.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    TGE_HIP(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs));
    if (cs != hipStreamCaptureStatusNone)
      return fail(TGE_ERR_INVALID,
                  "decode_attention_static: the stream is capturing (the plan is uploaded from "
                  "host memory at each call, which a graph would replay stale)");
  }
  // Host-side plan in per-thread buffers that keep their capacity.
  thread_local tge::plan::Step step;
  thread_local tge::plan::AttnLists lists;
  thread_local std::vector<char> image;
  const int hd = p->desc.head_dim;
  const char* msg = nullptr;
  s = tge::plan::build_step(step, d->n_sessions, d->ctx, d->n_new, d->table_offsets, d->page_ids,
                            d->q_heads, p->desc.kv_heads, hd, p->desc.pages, &msg);
  if (s != TGE_OK) return fail(s, std::string(msg ? msg : "invalid description"));
  if (step.max_rows > tge::max_unit_rows(step.block_dims))
    return fail(TGE_ERR_INVALID, "decode_attention_static: n_new * group exceeds a decode unit (64 rows, 48 at head_dim > 128)");
  const int f = p->desc.format, sf32 = p->desc.scale_format == TGE_SCALE_F32;
  const int rg = std::max(1, std::min(4, (step.max_rows + 15) / 16));
  const int bd = p->bd;
  tge::plan::build_decode(step, resident_groups(f, sf32, bd, rg, false), lists, 0);

  // scratch: [ sessions | tables | work | reduce | wg_first ] in the first
  // kStaticImageBytes, then part_o [parts][rows_cap][hd] and part_ml
  // [parts][rows_cap][2].
  const size_t o_tab = align_up(step.sessions.size() * sizeof(tge::SessionRec));
  const size_t o_work = align_up(o_tab + step.tables.size() * sizeof(int));
  size_t l_red = 0, l_first = 0;
  const size_t l_total = tge::plan::image_layout(lists, &l_red, &l_first);
  const size_t total = o_work + l_total;
  const size_t rows_cap = 16 * (size_t)lists.row_groups;
  const size_t parts = (size_t)std::max(lists.parts, 1);
  const size_t part_floats = parts * rows_cap * bd;
  const size_t part_bytes = (part_floats + parts * rows_cap * 2) * sizeof(float);
  if (total > kStaticImageBytes)
    return fail(TGE_ERR_CAPACITY, "decode_attention_static: the step's plan (" +
                                      std::to_string(total) + " B) exceeds the static limit of " +
                                      std::to_string(kStaticImageBytes) + " B");
  if (part_bytes > kStaticScratchBytes - kStaticImageBytes)
    return fail(TGE_ERR_CAPACITY, "decode_attention_static: the step's split-K partials (" +
                                      std::to_string(part_bytes) +
                                      " B) exceed the static limit of " +
                                      std::to_string(kStaticScratchBytes - kStaticImageBytes) +
                                      " B");
  char* base = nullptr;
  s = static_scratch(&base);
  if (s != TGE_OK) return s;

  if (image.size() < total) image.resize(total);
  std::memcpy(image.data(), step.sessions.data(), step.sessions.size() * sizeof(tge::SessionRec));
  if (!step.tables.empty())
    std::memcpy(image.data() + o_tab, step.tables.data(), step.tables.size() * sizeof(int));
  tge::plan::write_image(lists, l_red, l_first, image.data() + o_work);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // From pageable memory: the copy is ordered after the stream's earlier
  // work, and the host buffer may be reused once the call returns.
  TGE_HIP(hipMemcpyAsync(base, image.data(), total, hipMemcpyHostToDevice, st));

  tge_kv_layer_view v{};
  tge_kv_pool_layer(p, layer, &v);
  tge::AttnParams a{};
  a.pool = v.k;
  a.block_bytes = (uint32_t)p->geom.block_bytes;
  a.sessions = reinterpret_cast<const tge::SessionRec*>(base);
  a.work = reinterpret_cast<const tge::WorkRec*>(base + o_work);
  a.wg_first = reinterpret_cast<const int*>(base + o_work + l_first);
  a.tables = reinterpret_cast<const int*>(base + o_tab);
  a.q = q;
  a.out = out;
  a.part_o = reinterpret_cast<float*>(base + kStaticImageBytes);
  a.part_ml = a.part_o + part_floats;
  a.rows_cap = (int)rows_cap;
  a.kv_heads = step.kv_heads;
  a.q_heads = step.q_heads;
  a.dims = hd;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)hd));
  TGE_HIP(tge::launch_decode(f, sf32, bd, lists.row_groups, lists.groups, a, st));
  if (!lists.reduce.empty()) {
    tge::ReduceParams r{};
    r.items = reinterpret_cast<const tge::ReduceRec*>(base + o_work + l_red);
    r.part_o = a.part_o;
    r.part_ml = a.part_ml;
    r.out = out;
    r.rows_cap = a.rows_cap;
    r.q_heads = step.q_heads;
    r.dims = hd;
    TGE_HIP(tge::launch_reduce(bd, (int)lists.reduce.size(), lists.max_splits, r, st));
  }
  return TGE_OK;
}

int tge_eligible_gqa(int requested, int span, int threads, int follows_schedule,
                     int dense_only) {
  // eligible_gqa = requested && want_gqa_gpu(span, threads) && follows && dense
  // (backend.hpp:170-174); want_gqa_gpu = threads > 1 && span >= kGqaMinSpan
  // (backend.hpp:124-126).
  return requested && threads > 1 && span >= TGE_GQA_MIN_SPAN && follows_schedule && dense_only
             ? 1
             : 0;
}

int tge_attention_group(const tge_attention_group_args* a, void* stream) {
  if (!a || !a->pool) return fail(TGE_ERR_INVALID, "attention_group: null argument");
  const tge_kv_pool* p = a->pool;
  if (a->layer < 0 || a->layer >= p->desc.layers)
    return fail(TGE_ERR_INVALID, "attention_group: layer out of range");
  if (a->kv_head < 0 || a->kv_head >= p->desc.kv_heads)
    return fail(TGE_ERR_INVALID, "attention_group: kv_head out of range");
  if (!a->page_ids || !a->queries || !a->maxima || !a->sums || !a->accumulators)
    return fail(TGE_ERR_INVALID, "attention_group: null pointer");
  if (a->first < 0 || a->count < 0)
    return fail(TGE_ERR_INVALID, "attention_group: first and count must be >= 0");
  if (a->first > INT_MAX - a->count)
    return fail(TGE_ERR_INVALID, "attention_group: first + count overflows int");
  if (a->group_heads < 1 || a->group_heads > tge::kPrefillRows)
    return fail(TGE_ERR_INVALID, "attention_group: group_heads must be 1..128");
  int s = backend_ready();
  if (s != TGE_OK) return fail(s, "attention_group: backend unavailable");
  tge_kv_layer_view v{};
  tge_kv_pool_layer(p, a->layer, &v);
  tge::GroupParams g{};
  g.pool = v.k;
  g.block_bytes = (uint32_t)p->geom.block_bytes;
  g.pages = p->desc.pages;
  g.kv_heads = p->desc.kv_heads;
  g.kv_head = a->kv_head;
  g.page_ids = a->page_ids;
  g.first = a->first;
  g.count = a->count;
  g.queries = a->queries;
  g.group_heads = a->group_heads;
  g.dims = p->desc.head_dim;
  g.scale = a->scale;
  g.maxima = a->maxima;
  g.sums = a->sums;
  g.accumulators = a->accumulators;
  TGE_HIP(tge::launch_attention_group(p->desc.format, p->desc.scale_format == TGE_SCALE_F32,
                                      p->bd, g, static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

int tge_kv_gather(const tge_batch* b, const tge_kv_pool* p, int layer, int session,
                  int count, void* k_rows, void* v_rows, void* k_scales, void* v_scales,
                  void* stream) {
  int s = check_use(b, p, layer, "kv_gather");
  if (s != TGE_OK) return s;
  if (session < 0 || session >= (int)b->step.sessions.size())
    return fail(TGE_ERR_INVALID, "kv_gather: session out of range");
  const tge::SessionRec& sr = b->step.sessions[session];
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
  g.table = reinterpret_cast<const int*>(b->image.dev + b->off_tables) + sr.table_off;
  g.count = count;
  g.kv_heads = b->step.kv_heads;
  g.head_dim = p->bd;
  g.dims = b->step.head_dim;
  g.scale_bytes = p->desc.scale_format == TGE_SCALE_F32 ? 4 : 2;
  g.k_rows = k_rows;
  g.v_rows = v_rows;
  g.k_scales = i8 ? k_scales : nullptr;
  g.v_scales = i8 ? v_scales : nullptr;
  TGE_HIP(tge::launch_kv_gather(p->desc.format, g, static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

int tge_wait_expiries(unsigned int* count) {
  if (!count) return fail(TGE_ERR_INVALID, "wait_expiries: null argument");
  int s = backend_ready();
  if (s != TGE_OK) return fail(s, "wait_expiries: backend unavailable");
  unsigned int n = 0;
  TGE_HIP(tge::read_wait_expiries(&n));
  *count = n;
  return TGE_OK;
}

int tge_read_ceiling(const void* buf, size_t bytes, int pattern, int workgroups_per_cu,
                     int block_bytes, void* stream) {
  if (!buf) return fail(TGE_ERR_INVALID, "read_ceiling: null buffer");
  if (workgroups_per_cu < 1 || workgroups_per_cu > 64)
    return fail(TGE_ERR_INVALID, "read_ceiling: workgroups_per_cu must be 1..64");
  if (pattern == TGE_READ_STREAM) {
    if (bytes < 4096 || bytes % 4096 != 0)
      return fail(TGE_ERR_INVALID, "read_ceiling: stream bytes must be a positive multiple of 4096");
  } else if (pattern == TGE_READ_BLOCKS) {
    if (block_bytes < 16 || block_bytes > 17 * 1024 || block_bytes % 16 != 0)
      return fail(TGE_ERR_INVALID, "read_ceiling: block_bytes must be a multiple of 16 in 16..17408");
    if (bytes < (size_t)block_bytes || bytes / (size_t)block_bytes > 0x7fffffffu)
      return fail(TGE_ERR_INVALID, "read_ceiling: 1..2^31-1 blocks");
  } else {
    return fail(TGE_ERR_INVALID, "read_ceiling: unknown pattern");
  }
  int s = backend_ready();
  if (s != TGE_OK) return fail(s, "read_ceiling: backend unavailable");
  int dev = 0, cus = 0;
  TGE_HIP(hipGetDevice(&dev));
  TGE_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  TGE_HIP(tge::launch_read_ceiling(buf, bytes, pattern, cus * workgroups_per_cu, block_bytes,
                                   static_cast<hipStream_t>(stream)));
  return TGE_OK;
}

}  // extern "C"
