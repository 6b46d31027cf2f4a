// tge::models::BlockTable — the page-id allocator of the paged KV path.
//
// Same interface and behaviour as the reference's design-only table
// (include/tge/models/block_table.hpp:21-130 in AegeanWorks/Aegean-TGE):
//   - a fresh table hands out ids 0, 1, 2, ... (free list kept as a stack
//     whose top is the lowest id), and released pages are reused LIFO;
//   - share/release keep a refcount; a page returns to the free list when
//     its count reaches zero;
//   - slot_for maps a logical position to (page index, offset);
//   - hash_tokens is FNV-1a 64 over the little-endian bytes of int32 tokens;
//   - remember_prefix/find_prefix map a prefix hash to a page. Releasing a
//     page drops the hash it was remembered under from the lookup (the
//     page -> hash record itself is kept, as in the reference, :64-67);
//   - every misuse throws std::runtime_error.
// Two additions of this build (live, forget_prefix) serve the KV driver.
// Single-threaded, like the reference.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <unordered_map>
#include <utility>
#include <vector>

namespace tge::models {

inline constexpr int kBlockTokens = 16;

class BlockTable {
 public:
  explicit BlockTable(int blocks, int block_tokens = kBlockTokens)
      : block_tokens_(block_tokens) {
    if (blocks <= 0) throw std::runtime_error("BlockTable: blocks must be positive");
    if (block_tokens <= 0) {
      throw std::runtime_error("BlockTable: block_tokens must be positive");
    }
    refs_.assign(static_cast<std::size_t>(blocks), 0);
    stack_.reserve(static_cast<std::size_t>(blocks));
    for (int id = blocks; id-- > 0;) stack_.push_back(id);
  }

  int block_tokens() const { return block_tokens_; }
  int capacity() const { return static_cast<int>(refs_.size()); }
  int free_count() const { return static_cast<int>(stack_.size()); }

  int allocate() {
    if (stack_.empty()) throw std::runtime_error("BlockTable: table full");
    const int id = stack_.back();
    stack_.pop_back();
    refs_[static_cast<std::size_t>(id)] = 1;
    return id;
  }

  void share(int block) {
    check_live(block);
    ++refs_[static_cast<std::size_t>(block)];
  }

  void release(int block) {
    check_live(block);
    int& count = refs_[static_cast<std::size_t>(block)];
    if (--count > 0) return;
    stack_.push_back(block);
    const auto it = hash_of_.find(block);
    owner_.erase(it != hash_of_.end() ? it->second : kNoHash);
  }

  int refcount(int block) const {
    check_live(block);
    return refs_[static_cast<std::size_t>(block)];
  }

  static std::pair<int, int> slot_for(int logical_pos, int block_tokens) {
    if (logical_pos < 0 || block_tokens <= 0) {
      throw std::runtime_error("BlockTable: bad slot_for arguments");
    }
    return {logical_pos / block_tokens, logical_pos % block_tokens};
  }

  static std::uint64_t hash_tokens(const int* tokens, int count) {
    return hash_extend(kFnvBasis, tokens, count);
  }

  // The hash of a token run continued by `count` more tokens: hash_tokens of
  // a longer run is hash_extend of its head's hash over the tail.
  static std::uint64_t hash_extend(std::uint64_t h, const int* tokens, int count) {
    if (count < 0 || (count > 0 && tokens == nullptr)) {
      throw std::runtime_error("BlockTable: bad hash arguments");
    }
    for (int i = 0; i < count; ++i) {
      const auto word = static_cast<std::uint32_t>(tokens[i]);
      for (int shift = 0; shift < 32; shift += 8) {
        h = (h ^ ((word >> shift) & 0xFFu)) * kFnvPrime;
      }
    }
    return h;
  }

  void remember_prefix(std::uint64_t hash, int block) {
    check_live(block);
    owner_[hash] = block;
    hash_of_[block] = hash;
  }

  int find_prefix(std::uint64_t hash) const {
    const auto it = owner_.find(hash);
    return it == owner_.end() ? -1 : it->second;
  }

  // Not in the reference table: whether a block is allocated, and dropping
  // the prefix hash a block was remembered under (for a page whose rows are
  // rewritten in place, so the hash no longer describes its contents).
  bool live(int block) const {
    return block >= 0 && block < capacity() && refs_[static_cast<std::size_t>(block)] > 0;
  }
  void forget_prefix(int block) {
    const auto it = hash_of_.find(block);
    if (it == hash_of_.end()) return;
    const auto own = owner_.find(it->second);
    if (own != owner_.end() && own->second == block) owner_.erase(own);
    hash_of_.erase(it);
  }

 private:
  static constexpr std::uint64_t kNoHash = ~std::uint64_t{0};
  static constexpr std::uint64_t kFnvBasis = 1469598103934665603ULL;
  static constexpr std::uint64_t kFnvPrime = 1099511628211ULL;

  void check_live(int block) const {
    if (block < 0 || block >= capacity()) {
      throw std::runtime_error("BlockTable: block id out of range");
    }
    if (refs_[static_cast<std::size_t>(block)] <= 0) {
      throw std::runtime_error("BlockTable: block is not live");
    }
  }

  int block_tokens_;
  std::vector<int> refs_;
  std::vector<int> stack_;
  std::unordered_map<std::uint64_t, int> owner_;
  std::unordered_map<int, std::uint64_t> hash_of_;
};

}  // namespace tge::models
