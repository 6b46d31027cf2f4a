// Qwen2-shaped paged KV driver and the C wrappers of the BlockTable and the
// driver. See include/tge_amd/qwen2_kv.hpp and include/tge_kv.h.
#include "tge_amd/qwen2_kv.hpp"

#include "../csrc/tge_error.h"

#include <algorithm>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>

namespace tge::models {
namespace {

// A HIP/ABI failure below the driver: carries the C status.
struct StatusError : std::runtime_error {
  int status;
  StatusError(int s, const std::string& what) : std::runtime_error(what), status(s) {}
};

void check(int status, const char* who) {
  if (status != TGE_OK) {
    throw StatusError(status, std::string(who) + ": " + tge_last_error());
  }
}

}  // namespace

Qwen2KvPath::Qwen2KvPath(const Qwen2KvConfig& config) : config_(config) {
  if (config_.layers <= 0 || config_.q_heads <= 0 || config_.kv_heads <= 0 ||
      config_.head_dim <= 0 || config_.sequences <= 0 || config_.context <= 0) {
    throw std::invalid_argument("Qwen2KvPath: non-positive shape");
  }
  if (config_.q_heads % config_.kv_heads != 0) {
    throw std::invalid_argument("Qwen2KvPath: q_heads must be a multiple of kv_heads");
  }
  if (config_.q_heads / config_.kv_heads > 128) {
    // a block-prefill tile holds one query's whole head group (128 rows)
    throw std::invalid_argument("Qwen2KvPath: more than 128 query heads per KV head");
  }
  if (config_.format == TGE_KV_I8 && (config_.kv_heads * config_.head_dim) % 32 != 0) {
    // qwen2.cpp:406-409: the i8 cache needs kv_dim to be a multiple of 32.
    throw std::invalid_argument("Qwen2KvPath: i8 KV needs kv_dim to be a multiple of 32");
  }
  config_.context = std::min(config_.context, kHardMaxContext);
  if (config_.pages <= 0) {
    config_.pages = config_.sequences * ((config_.context + kBlockTokens - 1) / kBlockTokens);
  }
  table_ = std::make_unique<BlockTable>(config_.pages, kBlockTokens);
  pages_.assign(static_cast<std::size_t>(config_.sequences), {});
  length_.assign(static_cast<std::size_t>(config_.sequences), 0);
  tge_kv_pool_desc d{};
  d.layers = config_.layers;
  d.pages = config_.pages;
  d.kv_heads = config_.kv_heads;
  d.head_dim = config_.head_dim;
  d.format = config_.format;
  d.scale_format = config_.scale_format;
  check(tge_kv_pool_create(&d, &pool_), "Qwen2KvPath");
  check(tge_batch_create(&batch_), "Qwen2KvPath");
}

Qwen2KvPath::~Qwen2KvPath() {
  tge_batch_destroy(batch_);
  tge_kv_pool_destroy(pool_);
}

void Qwen2KvPath::check_sequence(int sequence, const char* who) const {
  if (sequence < 0 || sequence >= config_.sequences) {
    throw std::runtime_error(std::string(who) + ": sequence outside the model");
  }
}

int Qwen2KvPath::length(int sequence) const {
  check_sequence(sequence, "length");
  return length_[static_cast<std::size_t>(sequence)];
}

const std::vector<int>& Qwen2KvPath::pages(int sequence) const {
  check_sequence(sequence, "pages");
  return pages_[static_cast<std::size_t>(sequence)];
}

// Pages [first, last] of `list` that the step writes and another sequence
// also holds (reference count above one): they are copied before the write.
static int shared_in(const BlockTable& table, const std::vector<int>& list, int first, int last) {
  int n = 0;
  for (int k = first; k <= last && k < static_cast<int>(list.size()); ++k) {
    if (table.refcount(list[static_cast<std::size_t>(k)]) > 1) ++n;
  }
  return n;
}

void Qwen2KvPath::begin(const std::vector<Group>& groups, void* stream) {
  begun_ = false;
  // Validate everything before touching the table.
  std::vector<int> need_pages(static_cast<std::size_t>(config_.sequences), 0);
  int extra = 0;
  for (const Group& g : groups) {
    const std::size_t s = static_cast<std::size_t>(g.sequence);
    if (g.start > length_[s]) {
      throw std::runtime_error("forward: position leaves a gap in the cache");
    }
    const int need = (g.start + g.count + kBlockTokens - 1) / kBlockTokens;
    const int have = std::max(static_cast<int>(pages_[s].size()), need_pages[s]);
    if (need > have) {
      extra += need - have;
      need_pages[s] = need;
    }
    extra += shared_in(*table_, pages_[s], g.start / kBlockTokens, need - 1);
  }
  if (extra > table_->free_count()) throw std::runtime_error("BlockTable: table full");

  // Tentative page lists: a written page still held by another sequence is
  // replaced by a private copy (copy-on-write), and new pages are appended.
  // Nothing is committed until the plan is uploaded and the copies are
  // queued; on any failure the allocations are returned in reverse order,
  // which restores the free list exactly, and the model is unchanged.
  std::vector<std::vector<int>> lists;
  std::vector<int> fresh;                 // allocated pages, in order
  std::vector<std::pair<int, int>> cow;   // (shared page, its private copy)
  std::vector<int> ctx, n_new, offsets{0}, ids;
  int max_count = 0;
  try {
    for (const Group& g : groups) {
      std::vector<int> list = pages_[static_cast<std::size_t>(g.sequence)];
      const int need = (g.start + g.count + kBlockTokens - 1) / kBlockTokens;
      for (int k = g.start / kBlockTokens; k < need && k < static_cast<int>(list.size()); ++k) {
        const int old = list[static_cast<std::size_t>(k)];
        if (table_->refcount(old) > 1) {
          const int copy = table_->allocate();
          fresh.push_back(copy);
          cow.emplace_back(old, copy);
          list[static_cast<std::size_t>(k)] = copy;
        }
      }
      while (static_cast<int>(list.size()) < need) {
        fresh.push_back(table_->allocate());
        list.push_back(fresh.back());
      }
      ctx.push_back(g.start);
      n_new.push_back(g.count);
      ids.insert(ids.end(), list.begin(), list.end());
      offsets.push_back(static_cast<int>(ids.size()));
      max_count = std::max(max_count, g.count);
      lists.push_back(std::move(list));
    }
    tge_batch_desc d{};
    d.n_sessions = static_cast<int>(groups.size());
    d.ctx = ctx.data();
    d.n_new = n_new.data();
    d.table_offsets = offsets.data();
    d.page_ids = ids.data();
    d.q_heads = config_.q_heads;
    check(tge_batch_plan(batch_, pool_, &d, stream), "begin");
    for (const auto& c : cow) check(tge_kv_copy_page(pool_, c.first, c.second, stream), "begin");
  } catch (...) {
    for (auto it = fresh.rbegin(); it != fresh.rend(); ++it) table_->release(*it);
    throw;
  }

  // Commit.
  for (const auto& c : cow) table_->release(c.first);  // still held elsewhere
  for (std::size_t i = 0; i < groups.size(); ++i) {
    const Group& g = groups[i];
    const std::size_t s = static_cast<std::size_t>(g.sequence);
    pages_[s] = std::move(lists[i]);
    length_[s] = g.start + g.count;
    // A recorded page whose recorded rows this step rewrites in place no
    // longer holds its recorded prefix.
    const int need = (g.start + g.count + kBlockTokens - 1) / kBlockTokens;
    for (int k = g.start / kBlockTokens; k < need; ++k) {
      const int page = pages_[s][static_cast<std::size_t>(k)];
      const auto it = prefix_.find(page);
      if (it != prefix_.end() && k * kBlockTokens + it->second.count > g.start) drop_prefix(page);
    }
  }
  const int group = config_.q_heads / config_.kv_heads;
  // some session's rows exceed a decode unit: its attention runs on the
  // block-prefill kernel (tge_batch_attention picks per session)
  prefill_ = max_count * group > 64;
  step_rows_ = 0;
  for (int c : n_new) step_rows_ += c;
  begun_ = true;
}

void Qwen2KvPath::begin_forward(int sequence, int position, void* stream) {
  // qwen2.cpp:2036-2044
  if (position < 0 || position >= config_.context) {
    throw std::runtime_error("forward: position outside the allocated context");
  }
  check_sequence(sequence, "forward");
  begin({Group{sequence, position, 1}}, stream);
}

void Qwen2KvPath::begin_forward_batch(const int* positions, int count, const int* sequences,
                                      void* stream) {
  // qwen2.cpp:1615-1639
  if (positions == nullptr || sequences == nullptr || count <= 0) {
    throw std::runtime_error("forward_batch: invalid batch");
  }
  std::vector<Group> groups;
  std::vector<int> seen(static_cast<std::size_t>(config_.sequences), 0);
  for (int i = 0; i < count; ++i) {
    if (positions[i] < 0 || positions[i] >= config_.context) {
      throw std::runtime_error("forward_batch: position outside the context");
    }
    if (sequences[i] < 0 || sequences[i] >= config_.sequences) {
      throw std::runtime_error("forward_batch: sequence outside the slots");
    }
    if (!groups.empty() && groups.back().sequence == sequences[i] &&
        groups.back().start + groups.back().count == positions[i]) {
      ++groups.back().count;
      continue;
    }
    if (seen[static_cast<std::size_t>(sequences[i])]++) {
      throw std::runtime_error(
          "forward_batch: a sequence's rows must be consecutive positions");
    }
    groups.push_back(Group{sequences[i], positions[i], 1});
  }
  begin(groups, stream);
}

void Qwen2KvPath::begin_prefill(int sequence, int start_position, int count, void* stream) {
  // qwen2.cpp:2132-2142
  check_sequence(sequence, "prefill");
  if (count <= 0 || start_position < 0 || start_position + count > config_.context) {
    throw std::runtime_error("prefill: tokens outside the allocated context");
  }
  begin({Group{sequence, start_position, count}}, stream);
}

void Qwen2KvPath::begin_verify_draft(int sequence, int start_position, int count,
                                     void* stream) {
  // qwen2.cpp:2518-2531 (the reference pins sequence 0; any slot here)
  if (count <= 0 || count > kSpeculativeBatch) {
    throw std::runtime_error("verify_draft_logits: invalid draft");
  }
  check_sequence(sequence, "verify_draft");
  if (start_position < 0 || start_position + count > config_.context) {
    throw std::runtime_error("verify_draft: tokens outside the allocated context");
  }
  begin({Group{sequence, start_position, count}}, stream);
}

void Qwen2KvPath::layer(int layer, const float* q, const float* k, const float* v,
                        float* out, void* stream) {
  if (!begun_) throw std::runtime_error("layer: no step begun");
  if (layer < 0 || layer >= config_.layers) {
    throw std::invalid_argument("layer: layer out of range");
  }
  if (!prefill_) {
    // every session's rows fit a decode unit: store and attend in one call
    // (one kernel for a small step)
    check(tge_decode_step(batch_, pool_, layer, q, k, v, out, stream), "layer");
    return;
  }
  check(tge_kv_append(batch_, pool_, layer, k, v, stream), "layer");
  check(tge_batch_attention(batch_, pool_, layer, q, out, stream), "layer");
}

void Qwen2KvPath::layer_rope(int layer, const tge_rope_append_args& args, float* out,
                             void* stream) {
  if (!begun_) throw std::runtime_error("layer: no step begun");
  if (layer < 0 || layer >= config_.layers) {
    throw std::invalid_argument("layer: layer out of range");
  }
  if (!args.q || !args.q_out) throw std::invalid_argument("layer: q and q_out are required");
  check(tge_kv_append_rope(batch_, pool_, layer, &args, stream), "layer");
  check(tge_batch_attention(batch_, pool_, layer, args.q_out, out, stream), "layer");
}

void Qwen2KvPath::store(int layer, const float* k, const float* v, void* stream) {
  if (!begun_) throw std::runtime_error("store: no step begun");
  if (layer < 0 || layer >= config_.layers) {
    throw std::invalid_argument("store: layer out of range");
  }
  check(tge_kv_append(batch_, pool_, layer, k, v, stream), "store");
}

void Qwen2KvPath::set_sparse_config(const SparseConfig& config) {
  if (config.enabled && config.stride < 2) throw std::runtime_error("sparse: stride must be >= 2");
  if (config.enabled && (config.sink < 0 || config.window < 1)) {
    throw std::runtime_error("sparse: sink must be >= 0 and window >= 1");
  }
  sparse_ = config;
  const bool on = config.enabled && config_.format == TGE_KV_F16;
  check(tge_batch_set_sparse(batch_, on ? 1 : 0, config.sink, config.window, config.stride),
        "set_sparse_config");
}

void Qwen2KvPath::record_prefix(int block, int prev, const int* tokens, int count) {
  auto it = prefix_.find(block);
  if (it != prefix_.end() && it->second.prev != prev) {
    auto& sib = children_[it->second.prev];
    sib.erase(std::remove(sib.begin(), sib.end(), block), sib.end());
    it = prefix_.end();
    prefix_.erase(block);
  }
  if (it == prefix_.end()) {
    it = prefix_.emplace(block, PrefixPage{}).first;
    it->second.prev = prev;
    children_[prev].push_back(block);
  }
  it->second.count = std::max(it->second.count, count);
  std::copy(tokens, tokens + count, it->second.tokens);
}

void Qwen2KvPath::drop_prefix(int block) {
  std::vector<int> todo{block};
  while (!todo.empty()) {
    const int b = todo.back();
    todo.pop_back();
    const auto it = prefix_.find(b);
    if (it == prefix_.end()) continue;
    auto& sib = children_[it->second.prev];
    sib.erase(std::remove(sib.begin(), sib.end(), b), sib.end());
    prefix_.erase(it);
    if (table_->live(b)) table_->forget_prefix(b);
    const auto ch = children_.find(b);
    if (ch != children_.end()) {
      todo.insert(todo.end(), ch->second.begin(), ch->second.end());
      children_.erase(ch);
    }
  }
}

int Qwen2KvPath::match_prefix(const int* tokens, int count, std::vector<int>* chain) const {
  // Longest chain of records spelling tokens[0, count). Several recorded
  // pages may hold the same tokens after the same page (sequences that
  // prefilled the same text separately) and continue differently, so every
  // matching page is followed; a page always sits at the same position of
  // the sequences holding it, so the best continuation after a page is
  // memoised per page.
  struct Best {
    int len;   // tokens matched from the page's children on
    int next;  // child taken (-1: none)
  };
  std::unordered_map<int, Best> memo;
  auto run_of = [&](int block, int pos) {
    const PrefixPage& r = prefix_.at(block);
    const int lim = std::min(std::min(kBlockTokens, count - pos), r.count);
    int run = 0;
    while (run < lim && r.tokens[run] == tokens[pos + run]) ++run;
    return run;
  };
  std::function<Best(int, int)> solve = [&](int prev, int pos) -> Best {
    const auto m = memo.find(prev);
    if (m != memo.end()) return m->second;
    Best best{0, -1};
    const auto ch = children_.find(prev);
    if (ch != children_.end() && pos < count) {
      for (int b : ch->second) {
        const int run = run_of(b, pos);
        if (run == 0) continue;
        int len = run;
        if (run == kBlockTokens && pos + kBlockTokens < count) len += solve(b, pos + run).len;
        if (len > best.len) best = Best{len, b};
      }
    }
    memo.emplace(prev, best);
    return best;
  };
  const int total = solve(-1, 0).len;
  if (chain) {
    int prev = -1, pos = 0;
    while (pos < total) {
      const int b = memo.at(prev).next;
      chain->push_back(b);
      pos += run_of(b, pos);
      prev = b;
    }
  }
  return total;
}

int Qwen2KvPath::remember_prefix(int sequence, const int* tokens, int count) {
  check_sequence(sequence, "remember_prefix");
  if (count < 0 || (count > 0 && tokens == nullptr)) {
    throw std::runtime_error("remember_prefix: invalid tokens");
  }
  const auto& list = pages_[static_cast<std::size_t>(sequence)];
  const int n = std::min(count, length_[static_cast<std::size_t>(sequence)]);
  std::uint64_t h = BlockTable::hash_tokens(nullptr, 0);
  int prev = -1;
  for (int k = 0; k * kBlockTokens < n; ++k) {
    const int m = std::min(kBlockTokens, n - k * kBlockTokens);
    const int block = list[static_cast<std::size_t>(k)];
    record_prefix(block, prev, tokens + k * kBlockTokens, m);
    if (m == kBlockTokens) {
      h = BlockTable::hash_extend(h, tokens + k * kBlockTokens, kBlockTokens);
      table_->remember_prefix(h, block);
    }
    prev = block;
  }
  return n;
}

int Qwen2KvPath::shared_prefix_len(const int* tokens, int count) const {
  if (count < 0 || (count > 0 && tokens == nullptr)) {
    throw std::runtime_error("shared_prefix_len: invalid tokens");
  }
  return match_prefix(tokens, count, nullptr);
}

int Qwen2KvPath::attach_prefix(int sequence, const int* tokens, int count) {
  check_sequence(sequence, "attach_prefix");
  if (count < 0 || (count > 0 && tokens == nullptr)) {
    throw std::runtime_error("attach_prefix: invalid tokens");
  }
  auto& list = pages_[static_cast<std::size_t>(sequence)];
  if (!list.empty() || length_[static_cast<std::size_t>(sequence)] != 0) {
    throw std::runtime_error("attach_prefix: the sequence is not empty");
  }
  std::vector<int> chain;
  const int matched = match_prefix(tokens, std::min(count, config_.context), &chain);
  for (int block : chain) table_->share(block);
  list = std::move(chain);
  length_[static_cast<std::size_t>(sequence)] = matched;
  begun_ = false;
  return matched;
}

void Qwen2KvPath::reset_cache(int sequence) {
  // qwen2.cpp:2540-2543; zero-fill becomes page release.
  if (sequence < 0 || sequence >= config_.sequences) {
    throw std::runtime_error("reset_cache: sequence outside the model");
  }
  auto& list = pages_[static_cast<std::size_t>(sequence)];
  for (int id : list) {
    table_->release(id);
    if (!table_->live(id)) drop_prefix(id);  // back on the free list
  }
  list.clear();
  length_[static_cast<std::size_t>(sequence)] = 0;
  begun_ = false;
}

void Qwen2KvPath::reset_cache() {
  for (int s = 0; s < config_.sequences; ++s) reset_cache(s);
}

}  // namespace tge::models

// ---------------------------------------------------------------------------
// C wrappers
// ---------------------------------------------------------------------------
namespace {

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return TGE_OK;
  } catch (const tge::models::StatusError& e) {
    tge::set_last_error(e.what());
    return e.status;
  } catch (const std::invalid_argument& e) {
    tge::set_last_error(e.what());
    return TGE_ERR_INVALID;
  } catch (const std::runtime_error& e) {
    tge::set_last_error(e.what());
    return TGE_ERR_RUNTIME;
  } catch (const std::bad_alloc&) {
    tge::set_last_error("out of host memory");
    return TGE_ERR_CAPACITY;
  }
}

}  // namespace

// A table handle either owns its BlockTable or views the one a driver owns.
struct tge_block_table {
  std::unique_ptr<tge::models::BlockTable> owned;
  tge::models::BlockTable* table;
  tge_block_table(int blocks, int tokens)
      : owned(std::make_unique<tge::models::BlockTable>(blocks, tokens)), table(owned.get()) {}
  explicit tge_block_table(tge::models::BlockTable* view) : table(view) {}
};

struct tge_qwen2_kv {
  tge::models::Qwen2KvPath impl;
  tge_block_table table_view;
  explicit tge_qwen2_kv(const tge::models::Qwen2KvConfig& c)
      : impl(c), table_view(&impl.mutable_table()) {}
};

extern "C" {

int tge_block_table_create(int blocks, int block_tokens, tge_block_table** out) {
  if (!out) return TGE_ERR_INVALID;
  return guarded([&] { *out = new tge_block_table(blocks, block_tokens); });
}
void tge_block_table_destroy(tge_block_table* t) { delete t; }
int tge_block_table_allocate(tge_block_table* t, int* block) {
  if (!t || !block) return TGE_ERR_INVALID;
  return guarded([&] { *block = t->table->allocate(); });
}
int tge_block_table_share(tge_block_table* t, int block) {
  if (!t) return TGE_ERR_INVALID;
  return guarded([&] { t->table->share(block); });
}
int tge_block_table_release(tge_block_table* t, int block) {
  if (!t) return TGE_ERR_INVALID;
  return guarded([&] { t->table->release(block); });
}
int tge_block_table_refcount(const tge_block_table* t, int block, int* out) {
  if (!t || !out) return TGE_ERR_INVALID;
  return guarded([&] { *out = t->table->refcount(block); });
}
int tge_block_table_free_count(const tge_block_table* t) {
  return t ? t->table->free_count() : TGE_ERR_INVALID;
}
int tge_block_table_capacity(const tge_block_table* t) {
  return t ? t->table->capacity() : TGE_ERR_INVALID;
}
int tge_block_table_remember_prefix(tge_block_table* t, uint64_t hash, int block) {
  if (!t) return TGE_ERR_INVALID;
  return guarded([&] { t->table->remember_prefix(hash, block); });
}
int tge_block_table_find_prefix(const tge_block_table* t, uint64_t hash) {
  return t ? t->table->find_prefix(hash) : TGE_ERR_INVALID;
}
int tge_slot_for(int logical_pos, int block_tokens, int* block, int* offset) {
  if (!block || !offset) return TGE_ERR_INVALID;
  return guarded([&] {
    const auto s = tge::models::BlockTable::slot_for(logical_pos, block_tokens);
    *block = s.first;
    *offset = s.second;
  });
}
int tge_hash_tokens(const int* tokens, int count, uint64_t* out) {
  if (!out) return TGE_ERR_INVALID;
  return guarded([&] { *out = tge::models::BlockTable::hash_tokens(tokens, count); });
}

int tge_qwen2_kv_create(const tge_qwen2_kv_config* c, tge_qwen2_kv** out) {
  if (!c || !out) return TGE_ERR_INVALID;
  tge::models::Qwen2KvConfig cfg;
  cfg.layers = c->layers;
  cfg.q_heads = c->q_heads;
  cfg.kv_heads = c->kv_heads;
  cfg.head_dim = c->head_dim;
  cfg.context = c->context;
  cfg.sequences = c->sequences;
  cfg.pages = c->pages;
  cfg.format = c->format;
  cfg.scale_format = c->scale_format;
  return guarded([&] { *out = new tge_qwen2_kv(cfg); });
}
void tge_qwen2_kv_destroy(tge_qwen2_kv* m) { delete m; }
int tge_qwen2_kv_begin_forward(tge_qwen2_kv* m, int sequence, int position, void* stream) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.begin_forward(sequence, position, stream); });
}
int tge_qwen2_kv_begin_forward_batch(tge_qwen2_kv* m, const int* positions, int count,
                                     const int* sequences, void* stream) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.begin_forward_batch(positions, count, sequences, stream); });
}
int tge_qwen2_kv_begin_prefill(tge_qwen2_kv* m, int sequence, int start, int count,
                               void* stream) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.begin_prefill(sequence, start, count, stream); });
}
int tge_qwen2_kv_begin_verify(tge_qwen2_kv* m, int sequence, int start, int count,
                              void* stream) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.begin_verify_draft(sequence, start, count, stream); });
}
int tge_qwen2_kv_layer(tge_qwen2_kv* m, int layer, const float* q, const float* k,
                       const float* v, float* out, void* stream) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.layer(layer, q, k, v, out, stream); });
}
int tge_qwen2_kv_layer_rope(tge_qwen2_kv* m, int layer, const tge_rope_append_args* args,
                            float* out, void* stream) {
  if (!m || !args) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.layer_rope(layer, *args, out, stream); });
}
int tge_qwen2_kv_store(tge_qwen2_kv* m, int layer, const float* k, const float* v,
                       void* stream) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.store(layer, k, v, stream); });
}
int tge_qwen2_kv_reset(tge_qwen2_kv* m, int sequence) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] { m->impl.reset_cache(sequence); });
}
int tge_qwen2_kv_length(const tge_qwen2_kv* m, int sequence) {
  if (!m) return TGE_ERR_INVALID;
  int n = 0;
  const int s = guarded([&] { n = m->impl.length(sequence); });
  return s == TGE_OK ? n : s;
}
int tge_qwen2_kv_pages(const tge_qwen2_kv* m, int sequence, int* ids, int cap) {
  if (!m) return TGE_ERR_INVALID;
  int n = 0;
  const int s = guarded([&] {
    const auto& list = m->impl.pages(sequence);
    n = static_cast<int>(list.size());
    for (int i = 0; i < std::min(n, cap); ++i) ids[i] = list[static_cast<std::size_t>(i)];
  });
  return s == TGE_OK ? n : s;
}
int tge_qwen2_kv_set_sparse(tge_qwen2_kv* m, int enabled, int sink, int window, int stride) {
  if (!m) return TGE_ERR_INVALID;
  return guarded([&] {
    m->impl.set_sparse_config(tge::models::SparseConfig{enabled != 0, sink, window, stride});
  });
}
int tge_qwen2_kv_remember_prefix(tge_qwen2_kv* m, int sequence, const int* tokens, int count) {
  if (!m) return TGE_ERR_INVALID;
  int n = 0;
  const int s = guarded([&] { n = m->impl.remember_prefix(sequence, tokens, count); });
  return s == TGE_OK ? n : s;
}
int tge_qwen2_kv_shared_prefix_len(const tge_qwen2_kv* m, const int* tokens, int count) {
  if (!m) return TGE_ERR_INVALID;
  int n = 0;
  const int s = guarded([&] { n = m->impl.shared_prefix_len(tokens, count); });
  return s == TGE_OK ? n : s;
}
int tge_qwen2_kv_attach_prefix(tge_qwen2_kv* m, int sequence, const int* tokens, int count) {
  if (!m) return TGE_ERR_INVALID;
  int n = 0;
  const int s = guarded([&] { n = m->impl.attach_prefix(sequence, tokens, count); });
  return s == TGE_OK ? n : s;
}
const tge_kv_pool* tge_qwen2_kv_pool(const tge_qwen2_kv* m) { return m ? m->impl.pool() : nullptr; }
const tge_batch* tge_qwen2_kv_batch(const tge_qwen2_kv* m) { return m ? m->impl.batch() : nullptr; }
tge_block_table* tge_qwen2_kv_table(tge_qwen2_kv* m) { return m ? &m->table_view : nullptr; }
int tge_qwen2_kv_free_pages(const tge_qwen2_kv* m) {
  return m ? m->impl.table().free_count() : TGE_ERR_INVALID;
}

}  // extern "C"
