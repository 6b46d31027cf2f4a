// Host-side planning of one step: see plan.hpp.
#include "plan.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "tge_kv.h"

namespace tge::plan {

namespace {
std::size_t align256(std::size_t x) { return (x + 255) & ~std::size_t(255); }
}  // namespace

int Staged::upload(MemOps& m, std::size_t bytes, void* stream,
                   const std::function<void(char*)>& fill) {
  bytes = std::max<std::size_t>(bytes, 256);
  if (staged) {
    const int s = m.wait_event(staged);
    if (s != TGE_OK) return s;
  }
  if (bytes > host_bytes) {
    if (host) m.host_free(host);
    host = nullptr;
    host_bytes = 0;
    const int s = m.host_alloc(&host, bytes);
    if (s != TGE_OK) {
      host = nullptr;
      return s;
    }
    host_bytes = bytes;
  }
  if (bytes > dev_bytes) {
    if (dev) {
      const int s = m.wait_stream(stream);  // queued kernels may still read it
      if (s != TGE_OK) return s;
      m.dev_free(dev);
    }
    dev = nullptr;
    dev_bytes = 0;
    const int s = m.dev_alloc(&dev, bytes);
    if (s != TGE_OK) {
      dev = nullptr;
      return s;
    }
    dev_bytes = bytes;
  }
  fill(host);
  int s = m.copy_to_device(dev, host, bytes, stream);
  if (s == TGE_OK) s = m.record(&staged, stream);
  return s;
}

void Staged::release(MemOps& m) {
  if (dev) m.dev_free(dev);
  if (host) m.host_free(host);
  if (staged) m.event_free(staged);
  dev = host = nullptr;
  staged = nullptr;
  dev_bytes = host_bytes = 0;
}

int Scratch::reserve(MemOps& m, std::size_t need, void* stream) {
  if (need <= bytes) return TGE_OK;
  if (dev) {
    const int s = m.wait_stream(stream);
    if (s != TGE_OK) return s;
    m.dev_free(dev);
  }
  dev = nullptr;
  bytes = 0;
  const int s = m.dev_alloc(&dev, need);
  if (s != TGE_OK) {
    dev = nullptr;
    return s;
  }
  bytes = need;
  return TGE_OK;
}

void Scratch::release(MemOps& m) {
  if (dev) m.dev_free(dev);
  dev = nullptr;
  bytes = 0;
}

int build_step(Step& step, int ns, const int* ctx, const int* n_new, const int* table_offsets,
               const int* page_ids, int q_heads, int kv_heads, int head_dim, int pool_pages,
               const char** message) {
  auto bad = [&](const char* m) {
    if (message) *message = m;
    return TGE_ERR_INVALID;
  };
  if (ns <= 0 || !ctx || !n_new || !table_offsets || !page_ids)
    return bad("batch_plan: empty or incomplete description");
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0)
    return bad("batch_plan: q_heads must be a multiple of kv_heads");
  const int group = q_heads / kv_heads;
  if (group > prefill_tile_rows(head_dim <= 128 ? 128 : 256))
    return bad("batch_plan: more than 128 query heads per KV head (64 at head_dim > 128)");
  if (table_offsets[0] != 0) return bad("batch_plan: table_offsets[0] must be 0");
  const int n_entries = table_offsets[ns];
  if (n_entries < 0) return bad("batch_plan: negative table size");

  // Validate first: a failed plan leaves the step untouched.
  int max_rows = 0;
  for (int s = 0; s < ns; ++s) {
    const int c = ctx[s], nn = n_new[s];
    const int lo = table_offsets[s], hi = table_offsets[s + 1];
    if (c < 0 || nn < 1) return bad("batch_plan: ctx must be >= 0 and n_new >= 1");
    if (hi < lo || hi > n_entries) return bad("batch_plan: table_offsets must not decrease");
    const long need = ((long)c + nn + 15) / 16;
    if (hi - lo < need) return bad("batch_plan: block table shorter than the context");
    for (long i = 0; i < need; ++i) {
      const int id = page_ids[lo + i];
      if (id < 0 || id >= pool_pages) return bad("batch_plan: page id outside the pool");
    }
    if ((long)nn * group > (1L << 30)) return bad("batch_plan: too many rows");
    max_rows = std::max(max_rows, nn * group);
  }

  step.sessions.assign((std::size_t)ns, {});
  step.rows.clear();
  step.tables.assign(page_ids, page_ids + n_entries);
  int q_row = 0;
  for (int s = 0; s < ns; ++s) {
    const int c = ctx[s], nn = n_new[s], lo = table_offsets[s];
    step.sessions[(std::size_t)s] = SessionRec{c, nn, q_row, lo};
    for (int j = 0; j < nn; ++j) {
      const int pos = c + j;
      step.rows.push_back(RowRec{page_ids[lo + pos / 16], pos % 16, pos});
    }
    q_row += nn;
  }
  step.kv_heads = kv_heads;
  step.head_dim = head_dim;
  step.block_dims = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
  step.q_heads = q_heads;
  step.group = group;
  step.pages = pool_pages;
  step.max_rows = max_rows;
  return TGE_OK;
}

bool decode_session(const Step& s, const SessionRec& r) {
  return r.n_new * s.group <= max_unit_rows(s.block_dims);
}

bool take_session(const Step& s, const SessionRec& r, int only) {
  return only == 0 || (only == 1) == decode_session(s, r);
}

// Relative speed of the k-th workgroup that lands on a CU. Workgroups are
// dispatched one per CU before a CU gets a second, and on a shared SIMD the
// older wave wins issue, so equal page shares finish far apart. Measured
// pages per microsecond of the c5 decode kernel by dispatch rank: 1 : 0.79
// with two workgroups per CU (1 : 0.75 before page loads read whole KiB
// runs), 1 : 0.775 : 0.54 with three (per-workgroup timestamps over whole
// launches); more ranks fall off by TGE_DECODE_RANK_WEIGHT.
#ifndef TGE_DECODE_RANK_WEIGHT
#define TGE_DECODE_RANK_WEIGHT 0.76
#endif

namespace {
double rank_weight(int rank, int per_cu) {
  if (per_cu == 2 && rank < 2) return rank == 0 ? 1.0 : 0.79;
  if (per_cu == 3 && rank < 3) return rank == 0 ? 1.0 : rank == 1 ? 0.775 : 0.54;
  return std::pow(TGE_DECODE_RANK_WEIGHT, (double)rank);
}
}  // namespace
// Fixed cost of one unit of a share (start-up and merge), in pages.
#ifndef TGE_DECODE_UNIT_COST
#define TGE_DECODE_UNIT_COST 22
#endif
// At least 8 pages per workgroup: on small steps (one to four sessions
// of 1k-8k positions) shorter chains win over fewer split merges down to
// 8 pages (c1-c3: 5-7 % per layer-step against 16; 4 is slower again).
#ifndef TGE_DECODE_MIN_PAGES
#define TGE_DECODE_MIN_PAGES 8
#endif

void build_decode(const Step& b, Residency res, AttnLists& pl, int only) {
  pl.work.clear();
  pl.reduce.clear();
  pl.wg_first.clear();
  pl.app_first.clear();
  pl.app_recs.clear();
  pl.app_waves = 0;
  pl.parts = pl.max_splits = 0;
  int max_rows = 0;
  for (const auto& sr : b.sessions)
    if (take_session(b, sr, only)) max_rows = std::max(max_rows, sr.n_new * b.group);
  pl.row_groups = std::max(1, std::min(4, (max_rows + 15) / 16));

  struct Seg {
    int session, head, pages;
  };
  std::vector<Seg> segs;
  long total = 0;
  for (int s = 0; s < (int)b.sessions.size(); ++s) {
    const SessionRec& sr = b.sessions[(std::size_t)s];
    if (!take_session(b, sr, only)) continue;
    const int pages = (sr.ctx + sr.n_new + 15) / 16;
    for (int h = 0; h < b.kv_heads; ++h) segs.push_back(Seg{s, h, pages});
    total += (long)pages * b.kv_heads;
  }
  const long g_eff = std::max<long>(
      1, std::min<long>(res.groups, (total + TGE_DECODE_MIN_PAGES - 1) / TGE_DECODE_MIN_PAGES));
  std::vector<double> w((std::size_t)g_eff);
  double wrem = 0.0;
  for (long g = 0; g < g_eff; ++g) {
    const int cus = std::max(1, res.cus);
    w[(std::size_t)g] = rank_weight((int)(g / cus), (res.groups + cus - 1) / cus);
    wrem += w[(std::size_t)g];
  }

  // Cut the segments, end to end, into one share per workgroup. A share's
  // cost is its pages plus TGE_DECODE_UNIT_COST per piece (the fixed cost
  // of starting and merging a unit); each share gets the remaining cost in
  // proportion to its rank weight, the last one takes what is left.
  const double unit_cost = TGE_DECODE_UNIT_COST;
  std::vector<int> seg_of;  // segment of each work item
  long pages_rem = total, segs_rem = (long)segs.size();
  std::size_t si = 0;
  int pos = 0;
  pl.wg_first.push_back(0);
  for (long g = 0; g < g_eff && si < segs.size(); ++g) {
    const bool last_wg = g + 1 == g_eff;
    double target =
        ((double)pages_rem + unit_cost * (double)(segs_rem + (g_eff - g))) * w[(std::size_t)g] / wrem;
    wrem -= w[(std::size_t)g];
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
      const SessionRec& sr = b.sessions[(std::size_t)sg.session];
      WorkRec it{};
      it.session = sg.session;
      it.kv_head = sg.head;
      it.page_begin = pos;
      it.page_end = pos + take;
      it.part = -1;
      it.row_begin = 0;
      it.rows = sr.n_new * b.group;
      it.rows_per_query = b.group;
      it.head_base = sg.head * b.group;
      it.ctx = sr.ctx;
      it.q_row = sr.q_row;
      it.table_off = sr.table_off;
      it.red = -1;
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
  for (std::size_t i = 0; i < pl.work.size();) {
    std::size_t j = i + 1;
    while (j < pl.work.size() && seg_of[j] == seg_of[i]) ++j;
    const int n = (int)(j - i);
    pl.max_splits = std::max(pl.max_splits, n);
    if (n > 1) {
      const WorkRec& w0 = pl.work[i];
      ReduceRec r{};
      r.session = w0.session;
      r.row_begin = w0.row_begin;
      r.rows = w0.rows;
      r.rows_per_query = w0.rows_per_query;
      r.head_base = w0.head_base;
      r.first_part = pl.parts;
      r.q_row = w0.q_row;
      r.n_parts = n;
      for (std::size_t k = i; k < j; ++k) {
        pl.work[k].part = pl.parts++;
        pl.work[k].red = (int)pl.reduce.size();
      }
      pl.reduce.push_back(r);
    }
    i = j;
  }
  pl.groups = (int)pl.wg_first.size() - 1;
}

namespace {

// Splits [0, pages) into n nearly equal ranges and appends one unit each.
void add_units(std::vector<WorkRec>& work, std::vector<ReduceRec>& red, int& parts,
               int& max_splits, WorkRec base, int pages, int pps) {
  const int n = std::max(1, (pages + pps - 1) / pps);
  max_splits = std::max(max_splits, n);
  if (n == 1) {
    base.page_begin = 0;
    base.page_end = pages;
    base.part = -1;
    base.red = -1;
    work.push_back(base);
    return;
  }
  const int chunk = (pages + n - 1) / n;
  ReduceRec r{};
  r.session = base.session;
  r.row_begin = base.row_begin;
  r.rows = base.rows;
  r.rows_per_query = base.rows_per_query;
  r.head_base = base.head_base;
  r.first_part = parts;
  r.q_row = base.q_row;
  r.n_parts = 0;
  for (int b = 0; b < pages; b += chunk) {
    WorkRec w = base;
    w.page_begin = b;
    w.page_end = std::min(pages, b + chunk);
    w.part = parts++;
    w.red = (int)red.size();
    work.push_back(w);
    ++r.n_parts;
  }
  red.push_back(r);
}

}  // namespace

#ifndef TGE_PREFILL_MIN_SPLIT
#define TGE_PREFILL_MIN_SPLIT 32
#endif

void build_prefill(const Step& b, int cus, AttnLists& pl, int only, int halves, bool i8) {
  pl.work.clear();
  pl.reduce.clear();
  pl.wg_first.clear();
  pl.groups = 0;
  pl.parts = pl.max_splits = 0;
  pl.row_groups = kPrefillRows / 16;
  halves = halves == 2 ? 2 : 1;
  // Page-split size for tiles of tq queries: enough items for about two
  // rounds of two four-wave workgroups on each compute unit (of one
  // eight-wave workgroup with two halves), at least 32 pages (eight tiles
  // of four) per half. `pieces` counts the workgroups that gives.
  const long target_units = 2L * std::max(1, cus) * (halves == 2 ? 1 : 2);
  auto split_size = [&](int tq, long* pieces) {
    long pages_total = 0;
    for (const auto& sr : b.sessions) {
      if (!take_session(b, sr, only)) continue;
      for (int a = 0; a < sr.n_new; a += tq)
        pages_total += (long)((sr.ctx + std::min(sr.n_new, a + tq) + 15) / 16) * b.kv_heads;
    }
    const int pps = (int)std::max<long>((long)TGE_PREFILL_MIN_SPLIT * halves,
                                        ((pages_total + target_units - 1) / target_units + 3) / 4 * 4);
    if (pieces) {
      *pieces = 0;
      for (const auto& sr : b.sessions) {
        if (!take_session(b, sr, only)) continue;
        for (int a = 0; a < sr.n_new; a += tq)
          *pieces += (long)(((sr.ctx + std::min(sr.n_new, a + tq) + 15) / 16 + pps - 1) / pps) *
                     b.kv_heads;
      }
    }
    return pps;
  };
  pl.tile_rows = prefill_tile_rows(b.block_dims);
  int tq = std::max(1, pl.tile_rows / b.group);
  int pps = split_size(tq, nullptr);
  // Narrow tiles: a 128-dim step whose 128-row tiles would leave half the
  // compute units idle (the two-halves kernel runs one workgroup per CU)
  // takes 64-row tiles (one 16-row group per wave) instead: twice the
  // workgroups, each with half the rows against the same pages. With f16
  // pages, so does a step whose 128-row tiles would be split and merged
  // while its 64-row tiles fit one round of workgroups unsplit.
  if (halves == 2 && b.block_dims == 128 && b.group <= 64) {
    long pieces = 0, items = 0;
    split_size(tq, &pieces);
    const int tq64 = std::max(1, 64 / b.group);
    for (const auto& sr : b.sessions)
      if (take_session(b, sr, only)) items += (long)((sr.n_new + tq64 - 1) / tq64) * b.kv_heads;
    if (2 * pieces <= std::max(1, cus)) {
      pl.tile_rows = 64;
      tq = tq64;
      pps = split_size(tq, nullptr);
    } else if (!i8 && items <= std::max(1, cus) && pieces > items / 2) {
      // the split 128-row tiles need a merge launch; one round of unsplit
      // 64-row tiles does not (f16 pages: with int8 ones the split
      // 128-row tiles measure faster)
      pl.tile_rows = 64;
      tq = tq64;
      pps = 1 << 30;
    }
  }
  for (int s = 0; s < (int)b.sessions.size(); ++s) {
    const SessionRec& sr = b.sessions[(std::size_t)s];
    if (!take_session(b, sr, only)) continue;
    for (int h = 0; h < b.kv_heads; ++h) {
      for (int a = 0; a < sr.n_new; a += tq) {
        WorkRec w{};
        w.session = s;
        w.kv_head = h;
        w.ctx = sr.ctx;
        w.q_row = sr.q_row;
        w.table_off = sr.table_off;
        w.row_begin = a;
        w.rows = std::min(tq, sr.n_new - a) * b.group;
        w.rows_per_query = b.group;
        w.head_base = h * b.group;
        const int pages = (sr.ctx + a + std::min(tq, sr.n_new - a) + 15) / 16;
        add_units(pl.work, pl.reduce, pl.parts, pl.max_splits, w, pages, pps);
      }
    }
  }
  // Longest items first (partial slots are fixed per item, so order is free).
  std::stable_sort(pl.work.begin(), pl.work.end(), [](const WorkRec& x, const WorkRec& y) {
    return x.page_end - x.page_begin > y.page_end - y.page_begin;
  });
  pl.groups = (int)pl.work.size();
}

// When every context of the step fits this many batches, each is one piece:
// a batch more per wave (about a microsecond) costs less than the split
// merge it saves (the partials' coherent stores, the arrival counter and
// the last piece's reads, 3-4 microseconds), and no piece waits for another.
constexpr int kStepUnsplitBatches = 3;

bool build_step_lists(const Step& b, bool i8, bool scale_f32, StepLists& out) {
  out = StepLists{};
  if (b.max_rows > max_unit_rows(b.block_dims) || b.sessions.empty()) return false;
  long blocks = 0;
  int max_pages = 0;
  for (const auto& sr : b.sessions) {
    const int pages = (sr.ctx + sr.n_new + 15) / 16;
    blocks += (long)pages * b.kv_heads;
    max_pages = std::max(max_pages, pages);
  }
  if (blocks > kStepMaxBlocks) return false;
  // 64 rows at head_dim 128 (48 with int8 K/V and fp32 scales) do not fit
  // the step kernel's registers beside its page images (it would spill);
  // those steps take the decode kernel
  if (!step_fits(i8, scale_f32, b.block_dims, b.max_rows)) return false;
  out.row_groups = std::max(1, std::min(4, (b.max_rows + 15) / 16));
  // A piece is a whole number of batches (every wave of the workgroup loads
  // one batch of pages at once), as few as keep every context within
  // kStepMaxParts pieces.
  const int batch = kStepWaves * step_batch_pages(i8, scale_f32, b.block_dims, out.row_groups);
  const int heads = kStepMaxParts - 1;  // pieces before the appending one
  const int piece = batch * std::max(1, (max_pages + batch * heads - 1) / (batch * heads));
  out.piece_pages = piece;
  const bool unsplit = max_pages <= kStepUnsplitBatches * batch;
  for (int s = 0; s < (int)b.sessions.size(); ++s) {
    const SessionRec& sr = b.sessions[(std::size_t)s];
    const int pages = (sr.ctx + sr.n_new + 15) / 16;
    // A context of more than one piece: the pages before the first new
    // position in pieces of `piece` pages cut from the end (the first takes
    // the remainder), then one piece of the pages the new positions fall in
    // (at most 5: n_new <= 64), which stores the new rows first.
    const int written = sr.ctx / 16;
    const int head = unsplit || pages <= piece ? 0 : (written + piece - 1) / piece;
    const int n = head + 1;
    out.max_pieces = std::max(out.max_pieces, n);
    for (int h = 0; h < b.kv_heads; ++h) {
      const int seg = out.segments++;
      const int first = n > 1 ? out.parts : -1;
      if (n > 1) out.parts += n;
      for (int k = 0; k < n; ++k) {
        StepRec r{};
        if (k < head) {
          const int end = written - (head - 1 - k) * piece;
          r.page_begin = std::max(0, end - piece);
          r.page_end = end;
        } else {
          r.page_begin = head > 0 ? written : 0;
          r.page_end = pages;
        }
        r.session = s;
        r.kv_head = h;
        r.part = n > 1 ? first + k : -1;
        r.seg = seg;
        r.seg_parts = n;
        r.seg_first = first;
        r.append = k == n - 1;
        r.ctx = sr.ctx;
        r.n_new = sr.n_new;
        r.q_row = sr.q_row;
        r.table_off = sr.table_off;
        out.recs.push_back(r);
        const int pb = batch / kStepWaves;
        for (int i = 0; i < kStepFirstIds / kStepWaves; ++i)
          for (int w = 0; w < kStepWaves; ++w) {
            const int pg = std::min(r.page_begin + w + i * kStepWaves, r.page_end - 1);
            out.first_ids.push_back(i < pb && pg >= 0
                                        ? b.tables[(std::size_t)(r.table_off + pg)]
                                        : 0);
          }
      }
    }
  }
  return true;
}

std::size_t image_layout(const AttnLists& pl, std::size_t* off_reduce, std::size_t* off_first,
                         std::size_t* off_app) {
  const std::size_t wbytes = pl.work.size() * sizeof(WorkRec);
  *off_reduce = align256(wbytes);
  *off_first = align256(*off_reduce + pl.reduce.size() * sizeof(ReduceRec));
  const std::size_t end = *off_first + pl.wg_first.size() * sizeof(int);
  if (!off_app) return end;
  *off_app = align256(end);
  return *off_app + (pl.app_first.size() + pl.app_recs.size()) * sizeof(int);
}

void write_image(const AttnLists& pl, std::size_t off_reduce, std::size_t off_first, char* h,
                 std::size_t off_app) {
  if (!pl.work.empty()) std::memcpy(h, pl.work.data(), pl.work.size() * sizeof(WorkRec));
  if (!pl.reduce.empty())
    std::memcpy(h + off_reduce, pl.reduce.data(), pl.reduce.size() * sizeof(ReduceRec));
  if (!pl.wg_first.empty())
    std::memcpy(h + off_first, pl.wg_first.data(), pl.wg_first.size() * sizeof(int));
  if (off_app && !pl.app_first.empty()) {
    std::memcpy(h + off_app, pl.app_first.data(), pl.app_first.size() * sizeof(int));
    std::memcpy(h + off_app + pl.app_first.size() * sizeof(int), pl.app_recs.data(),
                pl.app_recs.size() * sizeof(int));
  }
}

void build_decode_appends(const Step& b, AttnLists& pl, int waves, int max_rows) {
  pl.app_first.clear();
  pl.app_recs.clear();
  pl.app_waves = 0;
  // (the kernel keys a row by its work item, below 2^15)
  if (waves <= 0 || pl.work.size() >= (std::size_t)1 << 15) return;
  const int groups = (int)pl.wg_first.size() - 1;
  std::vector<std::vector<int>> per((std::size_t)waves);
  for (int g = 0; g < groups; ++g) {
    for (auto& v : per) v.clear();
    for (int it = pl.wg_first[(std::size_t)g]; it < pl.wg_first[(std::size_t)g + 1]; ++it) {
      const WorkRec& u = pl.work[(std::size_t)it];
      const SessionRec& sr = b.sessions[(std::size_t)u.session];
      const int j0 = std::max(0, 16 * u.page_begin - sr.ctx);
      const int j1 = std::min(sr.n_new, 16 * u.page_end - sr.ctx);
      for (int j = j0; j < j1; ++j) {
        const int pos = sr.ctx + j;
        auto& v = per[(std::size_t)((pos / 16 - u.page_begin + it) % waves)];
        v.push_back(b.tables[(std::size_t)sr.table_off + (std::size_t)(pos / 16)]);
        v.push_back(pos);
        v.push_back((sr.q_row + j) * b.kv_heads + u.kv_head);
        v.push_back(it);
      }
    }
    for (const auto& v : per) {
      if ((int)(v.size() / kAppRecInts) > max_rows) {  // more than a wave holds: no lists
        pl.app_first.clear();
        pl.app_recs.clear();
        return;
      }
      pl.app_first.push_back((int)(pl.app_recs.size() / kAppRecInts));
      pl.app_recs.insert(pl.app_recs.end(), v.begin(), v.end());
    }
  }
  pl.app_first.push_back((int)(pl.app_recs.size() / kAppRecInts));
  pl.app_recs.resize(pl.app_recs.size() + (std::size_t)kAppPad * kAppRecInts, 0);
  pl.app_waves = waves;
}

}  // namespace tge::plan
