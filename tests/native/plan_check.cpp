// Host check of the step planner (aegean-tge_amd/host/plan.cpp), built with
// the address and undefined-behaviour sanitizers by tests/test_host_plan.py.
//   - random steps: the decode and block-prefill work lists cover every
//     page of every (session, KV head[, query tile]) exactly once, in order;
//     split items own consecutive partial slots that one reduction record
//     lists; workgroup ranges tile the work list; rows fit the units;
//   - the decode lists' new-row records list every new row once, for the
//     wave that reads its page;
//   - the one-launch step lists are taken exactly when a step qualifies and
//     tile each (session, KV head) in order with one appending last piece;
//   - invalid descriptions are rejected and leave the step untouched;
//   - staged uploads and scratch buffers survive injected allocation
//     failures: after a failure the recorded capacity is zero, and a later
//     (smaller) request allocates again instead of using a freed buffer.
// Prints "plan_check ok" and exits 0, or prints the first failure and
// exits 1.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <random>
#include <tuple>
#include <vector>

#include "../../aegean-tge_amd/host/plan.hpp"
#include "tge_kv.h"

using namespace tge;
using namespace tge::plan;

#define REQUIRE(c, ...)                                       \
  do {                                                        \
    if (!(c)) {                                               \
      std::printf("FAIL %s:%d: %s: ", __FILE__, __LINE__, #c); \
      std::printf(__VA_ARGS__);                               \
      std::printf("\n");                                      \
      std::exit(1);                                           \
    }                                                         \
  } while (0)

// A MemOps over malloc whose allocation number `fail_at` (counting from 0)
// fails with TGE_ERR_CAPACITY. Tracks live blocks, copies and waits.
struct FakeMem final : MemOps {
  int allocs = 0, fail_at = -1, live = 0, copies = 0, events = 0;
  int take(char** p, std::size_t n) {
    if (allocs++ == fail_at) {
      *p = nullptr;
      return TGE_ERR_CAPACITY;
    }
    *p = static_cast<char*>(std::malloc(n));
    ++live;
    return TGE_OK;
  }
  int host_alloc(char** p, std::size_t n) override { return take(p, n); }
  void host_free(char* p) override { std::free(p), --live; }
  int dev_alloc(char** p, std::size_t n) override { return take(p, n); }
  void dev_free(char* p) override { std::free(p), --live; }
  int copy_to_device(char* d, const char* h, std::size_t n, void*) override {
    std::memcpy(d, h, n);
    ++copies;
    return TGE_OK;
  }
  int record(void** ev, void*) override {
    if (!*ev) {
      *ev = std::malloc(1);
      ++events;
    }
    return TGE_OK;
  }
  int wait_event(void*) override { return TGE_OK; }
  int wait_stream(void*) override { return TGE_OK; }
  void event_free(void* e) override { std::free(e), --events; }
};

struct Desc {
  std::vector<int> ctx, n_new, offsets, ids;
};

Desc random_desc(std::mt19937& rng, int ns, int group, int pool_pages, bool decode_rows) {
  Desc d;
  d.offsets.push_back(0);
  for (int s = 0; s < ns; ++s) {
    const int pick = (int)(rng() % 4);
    const int c = pick == 0 ? 0 : pick == 1 ? 16 * (int)(rng() % 200) : (int)(rng() % 40000);
    const int max_new = decode_rows ? std::max(1, 64 / group) : 700;
    const int nn = 1 + (int)(rng() % max_new);
    d.ctx.push_back(c);
    d.n_new.push_back(nn);
    const int pages = (c + nn + 15) / 16 + (int)(rng() % 3);
    for (int i = 0; i < pages; ++i) d.ids.push_back((int)(rng() % pool_pages));
    d.offsets.push_back((int)d.ids.size());
  }
  return d;
}

// Each (session, head[, tile]) key's items must tile its pages exactly.
void check_lists(const Step& st, const AttnLists& l, int only, bool prefill) {
  REQUIRE(l.row_groups >= 1, "row_groups %d", l.row_groups);
  if (!l.wg_first.empty()) {
    REQUIRE((int)l.wg_first.size() == l.groups + 1, "wg_first size %zu groups %d",
            l.wg_first.size(), l.groups);
    REQUIRE(l.wg_first.front() == 0 && l.wg_first.back() == (int)l.work.size(), "wg_first ends");
    for (std::size_t i = 1; i < l.wg_first.size(); ++i)
      REQUIRE(l.wg_first[i] >= l.wg_first[i - 1], "wg_first decreases at %zu", i);
  } else {
    REQUIRE(l.groups == (int)l.work.size(), "one workgroup per item");
  }
  // key -> items
  std::map<std::tuple<int, int, int>, std::vector<const WorkRec*>> by;
  for (const WorkRec& w : l.work) {
    REQUIRE(w.session >= 0 && w.session < (int)st.sessions.size(), "session %d", w.session);
    const SessionRec& sr = st.sessions[(std::size_t)w.session];
    REQUIRE(take_session(st, sr, only), "session %d should not be planned", w.session);
    REQUIRE(w.kv_head >= 0 && w.kv_head < st.kv_heads, "kv head %d", w.kv_head);
    REQUIRE(w.rows >= 1 && w.rows <= 16 * l.row_groups, "rows %d of %d", w.rows, 16 * l.row_groups);
    if (prefill)
      REQUIRE(w.rows <= std::max(l.tile_rows, st.group), "rows %d past the %d-row tile", w.rows,
              l.tile_rows);
    REQUIRE(w.rows_per_query == st.group && w.head_base == w.kv_head * st.group, "row mapping");
    REQUIRE(w.rows % st.group == 0 && w.row_begin + w.rows / st.group <= sr.n_new, "row range");
    REQUIRE(w.ctx == sr.ctx && w.q_row == sr.q_row && w.table_off == sr.table_off, "copies");
    REQUIRE(w.page_begin >= 0 && w.page_begin < w.page_end, "page range %d..%d", w.page_begin,
            w.page_end);
    by[{w.session, w.kv_head, w.row_begin}].push_back(&w);
  }
  int parts_seen = 0;
  int max_splits = 0;
  for (int s = 0; s < (int)st.sessions.size(); ++s) {
    const SessionRec& sr = st.sessions[(std::size_t)s];
    if (!take_session(st, sr, only)) continue;
    for (int h = 0; h < st.kv_heads; ++h) {
      const int tq = prefill ? std::max(1, l.tile_rows / st.group) : sr.n_new;
      for (int a = 0; a < sr.n_new; a += tq) {
        const auto it = by.find({s, h, a});
        REQUIRE(it != by.end(), "session %d head %d tile %d has no work", s, h, a);
        std::vector<const WorkRec*> items = it->second;
        std::sort(items.begin(), items.end(),
                  [](const WorkRec* x, const WorkRec* y) { return x->page_begin < y->page_begin; });
        const int pages = (sr.ctx + a + std::min(tq, sr.n_new - a) + 15) / 16;
        int at = 0;
        for (const WorkRec* w : items) {
          REQUIRE(w->page_begin == at, "gap or overlap at page %d (item starts %d)", at,
                  w->page_begin);
          REQUIRE(w->rows == std::min(tq, sr.n_new - a) * st.group, "tile rows");
          at = w->page_end;
        }
        REQUIRE(at == pages, "session %d head %d covers %d of %d pages", s, h, at, pages);
        const int n = (int)items.size();
        max_splits = std::max(max_splits, n);
        if (n == 1) {
          REQUIRE(items[0]->part == -1 && items[0]->red == -1, "an unsplit item writes the output");
        } else {
          // one reduction record with n consecutive partial slots
          const ReduceRec* rr = nullptr;
          for (const ReduceRec& r : l.reduce)
            if (r.session == s && r.head_base == h * st.group && r.row_begin == a) rr = &r;
          REQUIRE(rr, "split session %d head %d has no reduction record", s, h);
          REQUIRE(rr->n_parts == n && rr->rows == items[0]->rows, "reduction record shape");
          REQUIRE(rr->q_row == sr.q_row, "reduction record row");
          for (const WorkRec* w : items)
            REQUIRE(w->red >= 0 && w->red < (int)l.reduce.size() && &l.reduce[(std::size_t)w->red] == rr,
                    "split item names another reduction record");
          std::vector<int> got;
          for (const WorkRec* w : items) got.push_back(w->part);
          std::sort(got.begin(), got.end());
          for (int k = 0; k < n; ++k)
            REQUIRE(got[(std::size_t)k] == rr->first_part + k, "partial slots not consecutive");
          REQUIRE(rr->first_part + n <= l.parts, "partial slot past the plan's count");
          parts_seen += n;
        }
      }
    }
  }
  REQUIRE(parts_seen == l.parts, "parts %d listed %d", l.parts, parts_seen);
  REQUIRE(max_splits == l.max_splits, "max_splits %d want %d", l.max_splits, max_splits);
  if (prefill) {
    for (std::size_t i = 1; i < l.work.size(); ++i)
      REQUIRE(l.work[i - 1].page_end - l.work[i - 1].page_begin >=
                  l.work[i].page_end - l.work[i].page_begin,
              "prefill items are not longest first");
  }
}

// The one-launch step lists: taken exactly when the step qualifies; each
// (session, KV head) is one segment of at most kStepMaxParts pieces tiling
// its pages in order; only the last piece appends and it holds every new
// position (and, when there are several, nothing else); split pieces own
// consecutive partial slots, each slot once.
void check_step_lists(const Step& st, bool i8, bool sf32) {
  StepLists sl;
  const bool one = build_step_lists(st, i8, sf32, sl);
  long blocks = 0;
  for (const auto& r : st.sessions) blocks += (long)((r.ctx + r.n_new + 15) / 16) * st.kv_heads;
  const int row_cap = st.head_dim <= 64 ? 64 : (i8 && sf32 ? 32 : 48);
  const bool fits = st.max_rows <= row_cap && blocks <= kStepMaxBlocks && !st.sessions.empty();
  REQUIRE(one == fits, "one-launch %d, qualifies %d (rows %d blocks %ld)", one, fits, st.max_rows,
          blocks);
  if (!one) {
    REQUIRE(sl.recs.empty() && sl.parts == 0 && sl.segments == 0, "lists left behind");
    return;
  }
  REQUIRE(16 * sl.row_groups >= st.max_rows && sl.row_groups <= 4, "row groups %d", sl.row_groups);
  const int batch = kStepWaves * step_batch_pages(i8, sf32, st.block_dims, sl.row_groups);
  int step_pages = 0;  // the step's longest context, in pages
  for (const SessionRec& sr : st.sessions) step_pages = std::max(step_pages, (sr.ctx + sr.n_new + 15) / 16);
  // every context within three batches: each is one piece (no split merge)
  const bool unsplit = step_pages <= 3 * batch;
  REQUIRE(sl.piece_pages >= batch && sl.piece_pages % batch == 0, "piece %d batch %d",
          sl.piece_pages, batch);
  // the first batch's page ids beside each record: what the block table
  // holds for the pages the waves load first (the piece's last page past
  // its end)
  REQUIRE(sl.first_ids.size() == sl.recs.size() * (std::size_t)kStepFirstIds, "first ids");
  for (std::size_t r = 0; r < sl.recs.size(); ++r) {
    const StepRec& rec = sl.recs[r];
    for (int b = 0; b < batch / kStepWaves; ++b)
      for (int w = 0; w < kStepWaves; ++w) {
        const int pg = std::min(rec.page_begin + w + b * kStepWaves, rec.page_end - 1);
        REQUIRE(sl.first_ids[r * kStepFirstIds + (std::size_t)(b * kStepWaves + w)] ==
                    st.tables[(std::size_t)(rec.table_off + pg)],
                "first id of record %zu, batch page %d, wave %d", r, b, w);
      }
  }
  REQUIRE(sl.piece_pages == batch || sl.max_pieces > kStepMaxParts / 2, "pieces longer than needed");
  std::vector<int> slot_used((std::size_t)sl.parts, 0);
  std::size_t i = 0;
  int seg = 0, max_pieces = 0;
  for (int s = 0; s < (int)st.sessions.size(); ++s) {
    const SessionRec& sr = st.sessions[(std::size_t)s];
    const int pages = (sr.ctx + sr.n_new + 15) / 16;
    for (int h = 0; h < st.kv_heads; ++h, ++seg) {
      int at = 0, k = 0;
      const int n = sl.recs[i].seg_parts;
      REQUIRE(n >= 1 && n <= kStepMaxParts, "pieces %d", n);
      max_pieces = std::max(max_pieces, n);
      for (; k < n; ++k, ++i) {
        REQUIRE(i < sl.recs.size(), "records end early");
        const StepRec& r = sl.recs[i];
        REQUIRE(r.session == s && r.kv_head == h && r.seg == seg && r.seg_parts == n,
                "record %zu identity", i);
        REQUIRE(r.ctx == sr.ctx && r.n_new == sr.n_new && r.q_row == sr.q_row &&
                    r.table_off == sr.table_off, "record %zu session fields", i);
        REQUIRE(r.page_begin == at && r.page_end > r.page_begin, "record %zu pages", i);
        if (n > 1 && k == n - 1) {
          REQUIRE(r.page_begin == sr.ctx / 16 && r.page_end - r.page_begin <= 5,
                  "appending piece [%d, %d) of ctx %d", r.page_begin, r.page_end, sr.ctx);
        } else if (n > 1) {
          REQUIRE(r.page_end - r.page_begin == sl.piece_pages || k == 0, "piece length");
          REQUIRE(r.page_end - r.page_begin <= sl.piece_pages, "first piece length");
        } else {
          REQUIRE(pages <= sl.piece_pages || unsplit, "one piece of %d pages", pages);
        }
        REQUIRE(!unsplit || n == 1, "a split context in a step of short contexts");
        at = r.page_end;
        REQUIRE(r.append == (k == n - 1), "append flag");
        if (r.append) REQUIRE(16 * r.page_begin <= sr.ctx, "new positions before the last piece");
        if (n == 1) {
          REQUIRE(r.part == -1 && r.seg_first == -1, "single piece with a slot");
        } else {
          REQUIRE(r.part == r.seg_first + k && r.part >= 0 && r.part < sl.parts, "slot %d", r.part);
          REQUIRE(slot_used[(std::size_t)r.part]++ == 0, "slot %d twice", r.part);
        }
      }
      REQUIRE(at == pages, "segment covers %d of %d pages", at, pages);
    }
  }
  REQUIRE(i == sl.recs.size() && seg == sl.segments, "extra records");
  REQUIRE(max_pieces == sl.max_pieces, "max pieces");
  for (int u : slot_used) REQUIRE(u == 1, "unused slot");
}

// New-row records of a decode plan (build_decode_appends): each new row of
// every (session, KV head) once, in the list of the wave that reads its page
// ((page - page_begin + item) mod waves), with its page id and k/v row; no
// lists only when a wave would hold more than max_rows.
void check_appends(const Step& st, const AttnLists& l, int waves, int max_rows) {
  if (l.app_waves == 0) {
    REQUIRE(l.app_first.empty() && l.app_recs.empty(), "no lists: empty");
    // some wave holds more than max_rows
    bool over = false;
    for (int g = 0; g < l.groups && !over; ++g) {
      std::vector<int> n((std::size_t)waves, 0);
      for (int it = l.wg_first[(std::size_t)g]; it < l.wg_first[(std::size_t)g + 1]; ++it) {
        const WorkRec& u = l.work[(std::size_t)it];
        const SessionRec& sr = st.sessions[(std::size_t)u.session];
        for (int j = 0; j < sr.n_new; ++j) {
          const int pg = (sr.ctx + j) / 16;
          if (pg >= u.page_begin && pg < u.page_end) ++n[(std::size_t)((pg - u.page_begin + it) % waves)];
        }
      }
      for (int x : n) over = over || x > max_rows;
    }
    REQUIRE(over, "lists refused although every wave fits");
    return;
  }
  REQUIRE(l.app_waves == waves, "waves");
  REQUIRE(l.app_first.size() == (std::size_t)l.groups * waves + 1, "list bounds");
  const int total = l.app_first.back();
  REQUIRE(l.app_recs.size() == (std::size_t)(total + kAppPad) * kAppRecInts, "records and padding");
  for (std::size_t k = (std::size_t)total * kAppRecInts; k < l.app_recs.size(); ++k)
    REQUIRE(l.app_recs[k] == 0, "padding");
  std::map<std::tuple<int, int, int>, int> seen;  // (session, head, position)
  for (int g = 0; g < l.groups; ++g) {
    for (int w = 0; w < waves; ++w) {
      const int a = l.app_first[(std::size_t)(g * waves + w)], b = l.app_first[(std::size_t)(g * waves + w + 1)];
      REQUIRE(a <= b && b - a <= max_rows, "wave list %d..%d", a, b);
      for (int r = a; r < b; ++r) {
        const int* rec = &l.app_recs[(std::size_t)r * kAppRecInts];
        const int item = rec[3];
        REQUIRE(item >= l.wg_first[(std::size_t)g] && item < l.wg_first[(std::size_t)g + 1], "item of the share");
        const WorkRec& u = l.work[(std::size_t)item];
        const SessionRec& sr = st.sessions[(std::size_t)u.session];
        const int pos = rec[1], pg = pos / 16, j = pos - sr.ctx;
        REQUIRE(j >= 0 && j < sr.n_new, "a new position");
        REQUIRE(pg >= u.page_begin && pg < u.page_end, "a page of the item");
        REQUIRE((pg - u.page_begin + item) % waves == w, "the wave that reads the page");
        REQUIRE(rec[0] == st.tables[(std::size_t)(sr.table_off + pg)], "page id");
        REQUIRE(rec[2] == (sr.q_row + j) * st.kv_heads + u.kv_head, "k/v row");
        REQUIRE(seen.emplace(std::make_tuple(u.session, u.kv_head, pos), 1).second, "row listed twice");
      }
    }
  }
  std::size_t want = 0;
  for (const auto& sr : st.sessions) want += (std::size_t)sr.n_new * st.kv_heads;
  REQUIRE(seen.size() == want, "rows listed %zu of %zu", seen.size(), want);
}

void random_plans(int cases) {
  std::mt19937 rng(12345);
  int narrow_seen = 0, wide_seen = 0, appends_seen = 0;
  for (int i = 0; i < cases; ++i) {
    const int kvh = 1 << (rng() % 4);
    const int group = (i % 17 == 0) ? 1 + (int)(rng() % 128) : 1 + (int)(rng() % 8);
    const int ns = 1 + (int)(rng() % 70);
    const int pool = 64 + (int)(rng() % 100000);
    const bool decode_rows = rng() % 3 != 0;
    Desc d = random_desc(rng, ns, group, pool, decode_rows);
    Step st;
    const char* msg = nullptr;
    const int s = build_step(st, ns, d.ctx.data(), d.n_new.data(), d.offsets.data(), d.ids.data(),
                             kvh * group, kvh, 128, pool, &msg);
    REQUIRE(s == TGE_OK, "case %d rejected: %s", i, msg ? msg : "");
    REQUIRE((int)st.sessions.size() == ns, "sessions");
    int rows = 0;
    for (int k = 0; k < ns; ++k) rows += d.n_new[(std::size_t)k];
    REQUIRE((int)st.rows.size() == rows, "rows");
    const bool i8 = rng() % 2, sf32 = rng() % 2;
    check_step_lists(st, i8, sf32);
    {
      // the same sessions at head_dim 64, and a short slice of them (so
      // that many steps qualify for one launch)
      Step s64;
      REQUIRE(build_step(s64, ns, d.ctx.data(), d.n_new.data(), d.offsets.data(), d.ids.data(),
                         kvh * group, kvh, 64, pool, &msg) == TGE_OK, "head_dim 64");
      check_step_lists(s64, i8, sf32);
      const int few = std::min(ns, 1 + (int)(rng() % 4));
      Step sf;
      REQUIRE(build_step(sf, few, d.ctx.data(), d.n_new.data(), d.offsets.data(), d.ids.data(),
                         kvh * group, kvh, (i & 1) ? 64 : 128, pool, &msg) == TGE_OK, "slice");
      check_step_lists(sf, i8, sf32);
    }
    const int cus = (rng() % 2) ? 256 : 1 + (int)(rng() % 300);
    const Residency res{cus * (1 + (int)(rng() % 2)), cus};
    for (int only = 0; only < 3; ++only) {
      AttnLists dec, pf;
      if (only != 2 && st.max_rows <= max_unit_rows(st.block_dims)) {
        build_decode(st, res, dec, only);
        check_lists(st, dec, only, false);
        REQUIRE(dec.groups <= res.groups, "more workgroups than resident");
        if (only == 0) {
          const int waves = (rng() % 2) ? 4 : 8, max_rows = (rng() % 2) ? 8 : 16;
          build_decode_appends(st, dec, waves, max_rows);
          check_appends(st, dec, waves, max_rows);
          if (dec.app_waves) appends_seen++;
          std::size_t ofr = 0, off = 0, oapp = 0;
          const std::size_t bytes = image_layout(dec, &ofr, &off, &oapp);
          std::vector<char> img(bytes);
          write_image(dec, ofr, off, img.data(), oapp);
          if (!dec.app_recs.empty())
            REQUIRE(std::memcmp(img.data() + oapp + dec.app_first.size() * sizeof(int), dec.app_recs.data(),
                                dec.app_recs.size() * sizeof(int)) == 0, "records in the image");
        }
      }
      const int halves = 1 + (int)(rng() % 2);
      const bool pf_i8 = rng() % 2;
      build_prefill(st, cus, pf, only, halves, pf_i8);
      REQUIRE(pf.tile_rows == prefill_tile_rows(st.block_dims) ||
                  (pf.tile_rows == 64 && st.block_dims == 128 && halves == 2),
              "tile rows %d at %d dims", pf.tile_rows, st.block_dims);
      if (pf.tile_rows == 64 && st.block_dims == 128) narrow_seen++;
      if (pf.tile_rows == 128 && halves == 2) wide_seen++;
      check_lists(st, pf, only, true);
      std::size_t ofr = 0, off = 0;
      const std::size_t bytes = image_layout(pf, &ofr, &off);
      std::vector<char> img(std::max<std::size_t>(bytes, 1));
      write_image(pf, ofr, off, img.data());
      if (!pf.work.empty())
        REQUIRE(std::memcmp(img.data(), pf.work.data(), pf.work.size() * sizeof(WorkRec)) == 0,
                "image");
    }
  }
  REQUIRE(narrow_seen > 0 && wide_seen > 0, "tile widths: %d narrow, %d wide", narrow_seen,
          wide_seen);
  REQUIRE(appends_seen > 0, "no plan with new-row lists");
}

void invalid_descriptions() {
  const int ctx[2] = {20, 5}, nn[2] = {1, 2}, off[3] = {0, 2, 3}, ids[3] = {4, 5, 6};
  Step st;
  const char* msg = nullptr;
  REQUIRE(build_step(st, 2, ctx, nn, off, ids, 8, 2, 64, 10, &msg) == TGE_OK, "valid one");
  const std::size_t before = st.sessions.size();
  struct Bad {
    int ns;
    int ctx0, nn0, off1, id0, q_heads, kvh, pool;
  } bad[] = {
      {0, 20, 1, 2, 4, 8, 2, 10},    // no sessions
      {2, -1, 1, 2, 4, 8, 2, 10},    // negative ctx
      {2, 20, 0, 2, 4, 8, 2, 10},    // n_new 0
      {2, 40, 1, 2, 4, 8, 2, 10},    // table shorter than the context
      {2, 20, 1, 2, 10, 8, 2, 10},   // page id outside the pool
      {2, 20, 1, 2, 4, 7, 2, 10},    // q_heads not a multiple
      {2, 20, 1, 2, 4, 129, 1, 10},  // group above 128
      {2, 20, 1, 4, 4, 8, 2, 10},    // offsets decrease
  };
  for (const Bad& b : bad) {
    int c[2] = {b.ctx0, 5}, n[2] = {b.nn0, 2}, o[3] = {0, b.off1, 3}, p[3] = {b.id0, 5, 6};
    REQUIRE(build_step(st, b.ns, c, n, o, p, b.q_heads, b.kvh, 64, b.pool, &msg) ==
                TGE_ERR_INVALID,
            "accepted a bad description (ctx %d nn %d off %d id %d q %d kv %d)", b.ctx0, b.nn0,
            b.off1, b.id0, b.q_heads, b.kvh);
    REQUIRE(st.sessions.size() == before && st.sessions[0].ctx == 20, "step changed on failure");
  }
}

void allocation_failures() {
  // Staged: fail each allocation of a growing upload, then retry smaller.
  for (int fail_at = 0; fail_at < 2; ++fail_at) {
    FakeMem m;
    Staged s;
    auto fill = [](std::size_t n) {
      return [n](char* h) { std::memset(h, 7, n); };
    };
    REQUIRE(s.upload(m, 1000, nullptr, fill(1000)) == TGE_OK, "first upload");
    m.fail_at = m.allocs + fail_at;
    REQUIRE(s.upload(m, 5000, nullptr, fill(5000)) == TGE_ERR_CAPACITY, "injected failure");
    if (fail_at == 0) {
      REQUIRE(!s.host && s.host_bytes == 0, "failed host buffer left recorded");
    } else {
      REQUIRE(!s.dev && s.dev_bytes == 0, "failed device buffer left recorded");
    }
    // a smaller retry must allocate what was lost and succeed
    REQUIRE(s.upload(m, 600, nullptr, fill(600)) == TGE_OK, "retry after failure");
    REQUIRE(s.host && s.dev && s.host_bytes >= 600 && s.dev_bytes >= 600, "retry buffers");
    REQUIRE(s.dev[599] == 7, "copy");
    s.release(m);
    REQUIRE(m.live == 0 && m.events == 0, "leaked %d blocks %d events", m.live, m.events);
  }
  // Scratch: same rule.
  FakeMem m;
  Scratch a;
  REQUIRE(a.reserve(m, 100, nullptr) == TGE_OK && a.bytes == 100, "reserve");
  m.fail_at = m.allocs;
  REQUIRE(a.reserve(m, 1000, nullptr) == TGE_ERR_CAPACITY, "injected failure");
  REQUIRE(!a.dev && a.bytes == 0, "failed scratch left recorded");
  REQUIRE(a.reserve(m, 50, nullptr) == TGE_OK && a.dev && a.bytes == 50, "retry");
  std::memset(a.dev, 1, 50);
  a.release(m);
  REQUIRE(m.live == 0, "leaked");
}

int main() {
  invalid_descriptions();
  allocation_failures();
  random_plans(600);
  std::printf("plan_check ok\n");
  return 0;
}
