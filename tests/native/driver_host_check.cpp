// Host check of the Qwen2 KV driver's bookkeeping (aegean-tge_amd/host/
// qwen2_kv.cpp) over a stand-in for the device half of the C ABI, built
// with the address and undefined-behaviour sanitizers by
// tests/test_host_plan.py. No GPU is involved: the stand-in records plans
// and page copies and can be told to fail the next plan or copy.
//   - begin() is transactional: a failing plan or copy leaves every page
//     list, length, refcount and the free list exactly as they were;
//   - shared prefixes are matched token by token (partial pages included),
//     a page whose recorded rows are rewritten in place loses its record,
//     and records go with the last holder of a page;
//   - a random sequence of steps, rewinds, resets, remembers and attaches:
//     every attached page holds exactly the tokens the attach matched
//     (tracked per physical page from the writes the steps made).
// Prints "driver_host_check ok" or the first failure (exit 1).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../aegean-tge_amd/csrc/tge_error.h"
#include "tge_amd/qwen2_kv.hpp"
#include "tge_kv.h"

#define REQUIRE(c, ...)                                       \
  do {                                                        \
    if (!(c)) {                                               \
      std::printf("FAIL %s:%d: %s: ", __FILE__, __LINE__, #c); \
      std::printf(__VA_ARGS__);                               \
      std::printf("\n");                                      \
      std::exit(1);                                           \
    }                                                         \
  } while (0)

// ---------------------------------------------------------------------------
// Stand-in for the device entry points the driver calls.
// ---------------------------------------------------------------------------
namespace {
std::string g_err;
int g_fail_plan = 0;  // fail the next n plans
int g_fail_copy = 0;  // fail the next n page copies
int g_copies = 0;
std::vector<std::pair<int, int>> g_copy_log;
}  // namespace

struct tge_kv_pool {
  tge_kv_pool_desc d;
};
struct tge_batch {
  int planned = 0;
};

void tge::set_last_error(const std::string& m) { g_err = m; }

extern "C" {
const char* tge_last_error(void) { return g_err.c_str(); }
int tge_kv_pool_create(const tge_kv_pool_desc* d, tge_kv_pool** out) {
  *out = new tge_kv_pool{*d};
  return TGE_OK;
}
void tge_kv_pool_destroy(tge_kv_pool* p) { delete p; }
int tge_batch_create(tge_batch** out) {
  *out = new tge_batch;
  return TGE_OK;
}
void tge_batch_destroy(tge_batch* b) { delete b; }
int tge_batch_plan(tge_batch* b, const tge_kv_pool* p, const tge_batch_desc* d, void*) {
  if (g_fail_plan > 0) {
    --g_fail_plan;
    g_err = "injected plan failure";
    return TGE_ERR_CAPACITY;
  }
  for (int s = 0; s < d->n_sessions; ++s) {
    const int need = (d->ctx[s] + d->n_new[s] + 15) / 16;
    if (d->table_offsets[s + 1] - d->table_offsets[s] < need) return TGE_ERR_INVALID;
    for (int i = d->table_offsets[s]; i < d->table_offsets[s + 1]; ++i)
      if (d->page_ids[i] < 0 || d->page_ids[i] >= p->d.pages) return TGE_ERR_INVALID;
  }
  b->planned = 1;
  return TGE_OK;
}
int tge_kv_copy_page(tge_kv_pool*, int src, int dst, void*) {
  if (g_fail_copy > 0) {
    --g_fail_copy;
    g_err = "injected copy failure";
    return TGE_ERR_DEVICE;
  }
  ++g_copies;
  g_copy_log.emplace_back(src, dst);
  return TGE_OK;
}
int tge_kv_append(const tge_batch* b, tge_kv_pool*, int, const float*, const float*, void*) {
  return b->planned ? TGE_OK : TGE_ERR_INVALID;
}
int tge_kv_append_rope(const tge_batch* b, tge_kv_pool*, int, const tge_rope_append_args*,
                       void*) {
  return b->planned ? TGE_OK : TGE_ERR_INVALID;
}
int tge_batch_attention(const tge_batch* b, const tge_kv_pool*, int, const float*, float*,
                        void*) {
  return b->planned ? TGE_OK : TGE_ERR_INVALID;
}
int tge_decode_step(const tge_batch* b, tge_kv_pool*, int, const float*, const float*,
                    const float*, float*, void*) {
  return b->planned ? TGE_OK : TGE_ERR_INVALID;
}
int tge_batch_set_sparse(tge_batch*, int, int, int, int) { return TGE_OK; }
}

using tge::models::Qwen2KvConfig;
using tge::models::Qwen2KvPath;

namespace {

Qwen2KvConfig config(int sequences, int pages) {
  Qwen2KvConfig c;
  c.layers = 2;
  c.q_heads = 14;
  c.kv_heads = 2;
  c.head_dim = 64;
  c.context = 1024;
  c.sequences = sequences;
  c.pages = pages;
  return c;
}

// Everything observable about the driver's allocation state.
struct Snapshot {
  std::vector<std::vector<int>> pages;
  std::vector<int> lengths;
  std::vector<int> refs;
  int free_count;
  bool operator==(const Snapshot& o) const {
    return pages == o.pages && lengths == o.lengths && refs == o.refs &&
           free_count == o.free_count;
  }
};

Snapshot snap(const Qwen2KvPath& m) {
  Snapshot s;
  for (int q = 0; q < m.sequence_count(); ++q) {
    s.pages.push_back(m.pages(q));
    s.lengths.push_back(m.length(q));
  }
  for (int b = 0; b < m.table().capacity(); ++b)
    s.refs.push_back(m.table().live(b) ? m.table().refcount(b) : 0);
  s.free_count = m.table().free_count();
  return s;
}

template <class F>
bool throws(F&& f) {
  try {
    f();
  } catch (const std::exception&) {
    return true;
  }
  return false;
}

void transactional_begin() {
  Qwen2KvPath m(config(3, 32));
  m.begin_prefill(0, 0, 40);
  m.layer(0, nullptr, nullptr, nullptr, nullptr);
  const Snapshot before = snap(m);
  // a failing plan on a step that needs a new page
  g_fail_plan = 1;
  REQUIRE(throws([&] { m.begin_prefill(0, 40, 30); }), "plan failure not reported");
  REQUIRE(snap(m) == before, "a failed plan changed the model");
  REQUIRE(throws([&] { m.layer(0, nullptr, nullptr, nullptr, nullptr); }),
          "layer ran after a failed begin");
  // the same step succeeds afterwards and takes the same pages
  m.begin_prefill(0, 40, 30);
  REQUIRE(m.length(0) == 70 && m.pages(0).size() == 5, "retry");

  // copy-on-write whose copy fails: share pages with sequence 1, then write
  // into a shared page from sequence 1
  std::vector<int> toks(70);
  for (int i = 0; i < 70; ++i) toks[(std::size_t)i] = 100 + i;
  REQUIRE(m.remember_prefix(0, toks.data(), 70) == 70, "remember");
  REQUIRE(m.attach_prefix(1, toks.data(), 50) == 50, "attach");
  const Snapshot shared = snap(m);
  g_fail_copy = 1;
  REQUIRE(throws([&] { m.begin_verify_draft(1, 20, 3); }), "copy failure not reported");
  REQUIRE(snap(m) == shared, "a failed copy changed the model");
  g_fail_plan = 1;
  REQUIRE(throws([&] { m.begin_verify_draft(1, 20, 3); }), "plan failure not reported");
  REQUIRE(snap(m) == shared, "a failed plan (with copy-on-write) changed the model");
  const int copies = g_copies;
  m.begin_verify_draft(1, 20, 3);
  REQUIRE(g_copies == copies + 1, "one page copied");
  REQUIRE(m.pages(1)[1] != m.pages(0)[1] && m.pages(1)[0] == m.pages(0)[0], "copy-on-write");
  // a full table is reported before anything changes
  const Snapshot full_before = snap(m);
  REQUIRE(throws([&] { m.begin_prefill(2, 0, 1000); }), "table full not reported");
  REQUIRE(snap(m) == full_before, "a full table changed the model");
}

void exact_prefixes() {
  Qwen2KvPath m(config(4, 64));
  std::vector<int> a(50), b(40);
  for (int i = 0; i < 50; ++i) a[(std::size_t)i] = 7 + i;
  for (int i = 0; i < 40; ++i) b[(std::size_t)i] = i < 20 ? 7 + i : 900 + i;  // shares 20 with a
  m.begin_prefill(0, 0, 50);
  m.begin_prefill(1, 0, 40);
  REQUIRE(m.remember_prefix(0, a.data(), 50) == 50, "remember a");
  REQUIRE(m.remember_prefix(1, b.data(), 40) == 40, "remember b");
  auto len = [&](std::vector<int> t) { return m.shared_prefix_len(t.data(), (int)t.size()); };
  REQUIRE(len(a) == 50, "%d", len(a));
  REQUIRE(len(std::vector<int>(a.begin(), a.begin() + 47)) == 47, "partial page");
  std::vector<int> a2 = a;
  a2[33] = -5;
  REQUIRE(len(a2) == 33, "mismatch inside a page: %d", len(a2));
  REQUIRE(len(b) == 40, "second chain: %d", len(b));
  std::vector<int> c = b;
  c[25] = 1;  // follows b's first page, a's second? no: b's page 1 from 16..31
  REQUIRE(len(c) == 25, "%d", len(c));
  REQUIRE(len({8}) == 0 && len({}) == 0, "no match");
  // a sequence sharing nothing but the same hash bucket never matches:
  // only exact tokens count
  // attach the first 45 tokens of a: pages 0..2, the last one in part
  REQUIRE(m.attach_prefix(2, a.data(), 45) == 45, "attach 45");
  REQUIRE(m.pages(2) == std::vector<int>(m.pages(0).begin(), m.pages(0).begin() + 3), "pages");
  REQUIRE(m.table().refcount(m.pages(0)[2]) == 2, "shared partial page");
  // sequence 2 writes at 45: its third page is copied first; a's records stay
  m.begin_forward(2, 45);
  REQUIRE(m.pages(2)[2] != m.pages(0)[2], "partial page copied on write");
  REQUIRE(len(a) == 50, "a's chain intact after the copy");
  // a rewind of sequence 0 into pages sequence 2 still holds copies them:
  // the originals keep their records, so a's chain is still found
  m.begin_forward(0, 30);
  REQUIRE(m.pages(0)[1] != m.pages(2)[1], "rewind copied the shared page");
  REQUIRE(len(a) == 50, "originals keep their records: %d", len(a));
  m.reset_cache(2);
  // now sequence 0 alone holds its pages: a rewind to 20 rewrites page 1
  // in place, which loses its record (page 0 keeps its own)
  m.reset_cache(0);
  m.begin_prefill(0, 0, 50);
  REQUIRE(m.remember_prefix(0, a.data(), 50) == 50, "remember a again");
  REQUIRE(len(a) == 50, "%d", len(a));
  m.begin_forward(0, 20);
  // (tokens 16..19 of a are still in b's page 1, after b's identical page 0)
  REQUIRE(len(a) == 20, "after the rewind: %d", len(a));
  m.reset_cache(1);
  REQUIRE(len(a) == 16 && len(b) == 16, "after the rewind: %d %d", len(a), len(b));
  m.begin_prefill(1, 0, 40);
  REQUIRE(m.remember_prefix(1, b.data(), 40) == 40, "remember b again");
  a[20] = 4242;
  REQUIRE(m.remember_prefix(0, a.data(), 21) == 21, "remember again");
  REQUIRE(len(std::vector<int>(a.begin(), a.begin() + 21)) == 21, "new chain");
  // records go with the last holder
  REQUIRE(len(b) == 40, "b's own chain: %d", len(b));
  m.reset_cache(1);
  REQUIRE(len(b) == 20, "b's first 20 tokens are in a's pages: %d", len(b));
  m.reset_cache(0);
  REQUIRE(len(a) == 0 && len(b) == 0, "all released");
}

// Random operations; every attach is checked against the tokens each
// physical page holds.
void random_flow(int ops) {
  std::mt19937 rng(99);
  const int S = 5, P = 80;
  Qwen2KvPath m(config(S, P));
  std::vector<std::vector<int>> toks(S);         // tokens of each sequence, by position
  std::map<int, std::vector<int>> content;       // page -> token per slot (-1 unknown)
  auto write = [&](int s, int start, int count) {
    toks[(std::size_t)s].resize((std::size_t)start);
    for (int i = 0; i < count; ++i) toks[(std::size_t)s].push_back((int)(rng() % 6));
    const auto& pl = m.pages(s);
    for (int p = start; p < start + count; ++p) {
      auto& c = content[pl[(std::size_t)(p / 16)]];
      c.resize(16, -1);
      c[(std::size_t)(p % 16)] = toks[(std::size_t)s][(std::size_t)p];
    }
  };
  // page copies carry the contents over
  std::size_t seen_copies = g_copy_log.size();
  auto apply_copies = [&] {
    for (; seen_copies < g_copy_log.size(); ++seen_copies) {
      const auto cp = g_copy_log[seen_copies];
      content[cp.second] = content[cp.first];
    }
  };
  int n_attach = 0, n_attached_tokens = 0, n_steps = 0, n_full = 0;
  for (int op = 0; op < ops; ++op) {
    const int s = (int)(rng() % S);
    const int kind = (int)(rng() % 10);
    const int len = m.length(s);
    try {
      if (kind < 4) {  // extend or rewind
        const int start = (kind == 0 && len > 0) ? (int)(rng() % (len + 1)) : len;
        const int count = 1 + (int)(rng() % 40);
        if (start + count > 1024) continue;
        const Snapshot before = snap(m);
        if (rng() % 8 == 0) {
          g_fail_plan = 1;
          REQUIRE(throws([&] { m.begin_prefill(s, start, count); }), "injected");
          REQUIRE(snap(m) == before, "failed step changed the model");
          continue;
        }
        // a copy may be needed first; its source content is known
        m.begin_prefill(s, start, count);
        ++n_steps;
        apply_copies();
        write(s, start, count);
      } else if (kind < 6) {
        m.remember_prefix(s, toks[(std::size_t)s].data(), len);
      } else if (kind < 7) {
        m.reset_cache(s);
        toks[(std::size_t)s].clear();
      } else if (len == 0) {
        // attach from another sequence's tokens, possibly cut short
        const int o = (int)(rng() % S);
        std::vector<int> q = toks[(std::size_t)o];
        q.resize(std::min<std::size_t>(q.size(), rng() % 120));
        if (!q.empty() && rng() % 3 == 0) q.back() = 77;  // a late mismatch
        const int got = m.attach_prefix(s, q.data(), (int)q.size());
        REQUIRE(got <= (int)q.size(), "attached more than asked");
        const auto& pl = m.pages(s);
        REQUIRE((int)pl.size() == (got + 15) / 16, "page count %zu for %d", pl.size(), got);
        for (int p = 0; p < got; ++p) {
          const auto& c = content[pl[(std::size_t)(p / 16)]];
          REQUIRE((int)c.size() == 16 && c[(std::size_t)(p % 16)] == q[(std::size_t)p],
                  "op %d: attached page %d slot %d holds %d, the query has %d", op,
                  pl[(std::size_t)(p / 16)], p % 16, c.empty() ? -9 : c[(std::size_t)(p % 16)],
                  q[(std::size_t)p]);
        }
        toks[(std::size_t)s] = std::vector<int>(q.begin(), q.begin() + got);
        ++n_attach;
        n_attached_tokens += got;
        REQUIRE(m.shared_prefix_len(q.data(), (int)q.size()) >= got, "length shrank");
      }
    } catch (const std::runtime_error& e) {
      // a full table is the only expected refusal
      REQUIRE(std::string(e.what()).find("full") != std::string::npos, "op %d: %s", op, e.what());
      ++n_full;
    }
    // refcounts equal the number of sequences holding each page
    std::vector<int> holders((std::size_t)P, 0);
    for (int q = 0; q < S; ++q)
      for (int p : m.pages(q)) ++holders[(std::size_t)p];
    for (int p = 0; p < P; ++p) {
      const int rc = m.table().live(p) ? m.table().refcount(p) : 0;
      REQUIRE(rc == holders[(std::size_t)p], "op %d page %d refcount %d holders %d", op, p, rc,
              holders[(std::size_t)p]);
    }
  }
  std::printf("random flow: %d steps, %d attaches (%d tokens), %d copies, %d full-table refusals\n",
              n_steps, n_attach, n_attached_tokens, (int)g_copy_log.size(), n_full);
  REQUIRE(n_attach > 100 && n_attached_tokens > 1000 && g_copy_log.size() > 20, "too little coverage");
}

}  // namespace

int main() {
  transactional_begin();
  exact_prefixes();
  random_flow(4000);
  std::printf("driver_host_check ok\n");
  return 0;
}
