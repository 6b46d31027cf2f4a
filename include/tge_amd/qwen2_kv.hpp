// tge::models::Qwen2KvPath — the Qwen2 decoder's KV-cache path over paged
// gfx950 memory.
//
// Mirrors the cache-facing half of the reference's Qwen2 class
// (include/tge/models/qwen2.hpp:107-305 in AegeanWorks/Aegean-TGE):
// forward / forward_batch / prefill / verify_draft / reset_cache keep their
// validation rules and their store-then-attend order per layer
// (qwen2.cpp:2032-2095, 1613-1747, 2130-2335, 2502-2577), with the flat
// [sequence][layer][position][kv_dim] cache replaced by BlockTable pages.
// Weights are not on this path: the caller supplies each layer's post-RoPE
// q, k, v rows (device memory) and receives the attention rows.
//
// A step is begun once (pages allocated from the BlockTable, plan uploaded)
// and then run layer by layer, so every layer reuses one host->device copy.
// Misuse throws std::runtime_error (model contract) or std::invalid_argument
// (shape contract); device failures throw std::runtime_error with the HIP
// message.
#pragma once

#include <memory>
#include <unordered_map>
#include <vector>

#include "tge_amd/block_table.hpp"
#include "tge_kv.h"

namespace tge::models {

// Static sparse attention (qwen2.hpp:30-35).
struct SparseConfig {
  bool enabled = false;
  int sink = 4;
  int window = 512;
  int stride = 4;
};

struct Qwen2KvConfig {
  int layers = 0;
  int q_heads = 0;
  int kv_heads = 0;
  int head_dim = 0;
  int context = 4096;  // kDefaultContext, qwen2.cpp:25
  int sequences = 1;
  int pages = 0;       // 0: sequences * ceil(context / 16)
  int format = TGE_KV_F16;
  int scale_format = TGE_SCALE_F16;
};

class Qwen2KvPath {
 public:
  static constexpr int kSpeculativeBatch = 6;  // qwen2.hpp:140
  static constexpr int kHardMaxContext = 32768;  // qwen2.cpp:26

  explicit Qwen2KvPath(const Qwen2KvConfig& config);
  ~Qwen2KvPath();
  Qwen2KvPath(const Qwen2KvPath&) = delete;
  Qwen2KvPath& operator=(const Qwen2KvPath&) = delete;

  const Qwen2KvConfig& config() const { return config_; }
  int sequence_count() const { return config_.sequences; }
  int max_context() const { return config_.context; }

  // Step set-up. `stream` is a hipStream_t (nullptr = default stream).
  void begin_forward(int sequence, int position, void* stream = nullptr);
  void begin_forward_batch(const int* positions, int count, const int* sequences,
                           void* stream = nullptr);
  void begin_prefill(int sequence, int start_position, int count, void* stream = nullptr);
  void begin_verify_draft(int sequence, int start_position, int count,
                          void* stream = nullptr);

  // Store this step's K/V rows for `layer`, then attend: per session, the
  // decode kernel when its rows fit a decode unit (n_new * group <= 64),
  // else the MFMA block-prefill kernel (tge_batch_attention), so one
  // forward_batch step may mix decoding and prefilling sessions.
  void layer(int layer, const float* q, const float* k, const float* v, float* out,
             void* stream = nullptr);

  // layer() with bias + RoPE fused into the append (tge_kv_append_rope):
  // args.k/v/q are the rows before bias and RoPE; attention reads
  // args.q_out.
  void layer_rope(int layer, const tge_rope_append_args& args, float* out,
                  void* stream = nullptr);

  // Store this step's K/V rows for `layer` without attending: the cache-
  // priming path (prime_cache_from_table, qwen2.hpp:283-288 and
  // qwen2.cpp:1973-2026, copies rows into a slot with no recompute).
  void store(int layer, const float* k, const float* v, void* stream = nullptr);

  // set_sparse_config (qwen2.cpp:182-189): stride >= 2, sink >= 0 and
  // window >= 1 or runtime_error. Like the reference (uses_sparse,
  // qwen2.cpp:1313-1317) it applies to f16 caches only; i8 stays dense.
  void set_sparse_config(const SparseConfig& config);
  const SparseConfig& sparse_config() const { return sparse_; }

  // Shared prefixes over pages, matched token by token. remember_prefix
  // records, for each cached page among the sequence's first `count`
  // tokens, the tokens it holds (up to 16; the last page may be partial)
  // and the page before it, so a chain of records spells out a prefix
  // exactly (the populate step, qwen2.cpp:2388-2465); full pages are also
  // keyed in the BlockTable under the hash of tokens [0, 16(k+1)). Returns
  // the tokens recorded. shared_prefix_len is the longest run of tokens,
  // from the first, that some recorded chain holds (qwen2.cpp:1948-1971):
  // every token is compared, never a hash alone. attach_prefix gives an
  // empty sequence that run by reference count (BlockTable::share;
  // qwen2.cpp:1973-2026 copies rows instead), the last page possibly only
  // in part, and returns its cached length. A step that writes into a page
  // another sequence also holds copies the page first (copy-on-write); a
  // step that rewrites recorded rows of a page in place drops its record.
  int remember_prefix(int sequence, const int* tokens, int count);
  int shared_prefix_len(const int* tokens, int count) const;
  int attach_prefix(int sequence, const int* tokens, int count);

  // reset_cache(sequence): the sequence's pages go back to the table in
  // logical order; reset_cache() does every sequence.
  void reset_cache(int sequence);
  void reset_cache();

  int length(int sequence) const;
  const std::vector<int>& pages(int sequence) const;
  const BlockTable& table() const { return *table_; }
  // The page allocator itself, e.g. to pre-shape its free list before the
  // first step (fragmented pools). Pages a sequence holds must not be
  // released through it.
  BlockTable& mutable_table() { return *table_; }
  const tge_kv_pool* pool() const { return pool_; }
  const tge_batch* batch() const { return batch_; }
  int step_rows() const { return step_rows_; }
  bool step_is_prefill() const { return prefill_; }

 private:
  struct Group {
    int sequence;
    int start;
    int count;
  };
  // One recorded page of a shared prefix: the tokens its first `count`
  // rows hold and the recorded page before it (-1 for a chain's first).
  struct PrefixPage {
    int prev = -1;
    int count = 0;
    int tokens[kBlockTokens] = {};
  };
  void check_sequence(int sequence, const char* who) const;
  void begin(const std::vector<Group>& groups, void* stream);
  // Pages of the longest recorded chain matching `tokens`; returns the
  // matched token count.
  int match_prefix(const int* tokens, int count, std::vector<int>* chain) const;
  void record_prefix(int block, int prev, const int* tokens, int count);
  // Drops a page's record and, since their chains pass through it, the
  // records of every page recorded after it.
  void drop_prefix(int block);

  Qwen2KvConfig config_;
  std::unique_ptr<BlockTable> table_;
  std::vector<std::vector<int>> pages_;
  std::vector<int> length_;
  tge_kv_pool* pool_ = nullptr;
  tge_batch* batch_ = nullptr;
  int step_rows_ = 0;
  bool prefill_ = false;
  bool begun_ = false;
  SparseConfig sparse_;
  std::unordered_map<int, PrefixPage> prefix_;          // page -> record
  std::unordered_map<int, std::vector<int>> children_;  // record's prev -> pages
};

}  // namespace tge::models
