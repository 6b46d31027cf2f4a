// CPU baseline for bench.py — TEST/MEASUREMENT INFRASTRUCTURE ONLY.
//
// Restates the reference engine's attention *schedule* (which kernel runs
// for which span, how positions split into chunks, how tasks spread over the
// worker pool) and calls the reference's own AVX2 kernels, linked from
// /root/reference/src/cpu/avx2/attention_avx2.cpp. The reference's
// ThreadPool does not build on Linux (thread_pool.cpp:145,149 use a Windows
// topology call), so a fork-join team with dynamic claiming stands in for
// it: same task granularity, caller participates.
//
// Schedules restated:
//   decode_gqa    qwen2.cpp:1319-1380 (attention), 1382-1467 (attention_gqa),
//                 1469-1522 (merge_gqa_chunks)
//   batch_heads   qwen2.cpp:1705-1747 (forward_batch attention, per head)
//   block_prefill qwen2.cpp:1524-1571 (attention_batch, query-block kernel)
//   append        qwen2.cpp:2073-2093 (f16 store), 88-120 (i8 store)
#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "tge/cpu/kernels.hpp"

namespace {

class Team {
 public:
  explicit Team(int threads) : threads_(std::max(1, threads)) {
    for (int i = 1; i < threads_; ++i) workers_.emplace_back([this] { loop(); });
  }
  ~Team() {
    {
      std::lock_guard<std::mutex> lock(mutex_);
      stop_ = true;
      ++generation_;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  int threads() const { return threads_; }

  void parallel_for(int count, const std::function<void(int)>& fn) {
    if (threads_ == 1 || count <= 1) {
      for (int i = 0; i < count; ++i) fn(i);
      return;
    }
    {
      std::lock_guard<std::mutex> lock(mutex_);
      fn_ = &fn;
      count_ = count;
      next_.store(0);
      pending_ = static_cast<int>(workers_.size());
      ++generation_;
    }
    cv_.notify_all();
    drain();
    std::unique_lock<std::mutex> lock(mutex_);
    done_cv_.wait(lock, [this] { return pending_ == 0; });
    fn_ = nullptr;
  }

 private:
  void drain() {
    for (;;) {
      const int i = next_.fetch_add(1);
      if (i >= count_) break;
      (*fn_)(i);
    }
  }
  void loop() {
    std::uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lock(mutex_);
        cv_.wait(lock, [&] { return generation_ != seen; });
        seen = generation_;
        if (stop_) return;
      }
      drain();
      std::lock_guard<std::mutex> lock(mutex_);
      if (--pending_ == 0) done_cv_.notify_all();
    }
  }

  int threads_;
  std::vector<std::thread> workers_;
  std::mutex mutex_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int)>* fn_ = nullptr;
  int count_ = 0;
  std::atomic<int> next_{0};
  int pending_ = 0;
  std::uint64_t generation_ = 0;
  bool stop_ = false;
};

enum { kF32 = 0, kF16 = 1, kI8 = 2 };

template <typename Args>
void set_kv(Args& a, int format, const void* k, const void* v,
            const float* ks, const float* vs, std::size_t off) {
  if (format == kF16) {
    a.half = true;
    a.keys_half = static_cast<const std::uint16_t*>(k) + off;
    a.values_half = static_cast<const std::uint16_t*>(v) + off;
  } else if (format == kI8) {
    a.q8 = true;
    a.keys_q8 = static_cast<const std::int8_t*>(k) + off;
    a.values_q8 = static_cast<const std::int8_t*>(v) + off;
    a.keys_q8_scales = ks + off / 32;
    a.values_q8_scales = vs + off / 32;
  } else {
    a.keys = static_cast<const float*>(k) + off;
    a.values = static_cast<const float*>(v) + off;
  }
}

void merge_chunks(const float* maxima, const float* sums, const float* acc,
                  std::size_t base, int chunks, int group, int gh, int d,
                  float* red, float* out) {
  bool have = false;
  float m = -INFINITY, s = 0.0F;
  std::fill(red, red + d, 0.0F);
  for (int c = 0; c < chunks; ++c) {
    const std::size_t st = base + static_cast<std::size_t>(c) * group + gh;
    if (!(sums[st] > 0.0F)) continue;
    const float* a = acc + st * d;
    if (!have) {
      m = maxima[st];
      s = sums[st];
      std::copy(a, a + d, red);
      have = true;
      continue;
    }
    const float mm = std::max(m, maxima[st]);
    const float al = std::exp(m - mm), be = std::exp(maxima[st] - mm);
    s = s * al + sums[st] * be;
    for (int i = 0; i < d; ++i) red[i] = red[i] * al + a[i] * be;
    m = mm;
  }
  const float inv = (have && s > 0.0F) ? 1.0F / s : 0.0F;
  for (int i = 0; i < d; ++i) out[i] = have ? red[i] * inv : 0.0F;
}

}  // namespace

extern "C" {

void* ref_team_create(int threads) { return new Team(threads); }
void ref_team_destroy(void* t) { delete static_cast<Team*>(t); }
int ref_hw_threads() { return static_cast<int>(std::thread::hardware_concurrency()); }

// One decode step of one sequence at `span` positions (all heads).
// cache_k/cache_v/k_scales/v_scales point at the (sequence, layer) slot base
// of a flat [position][kv_dim] cache. scratch must hold
// kv_heads*16*group*(head_dim+2) + heads*span + head_dim floats.
void ref_baseline_decode(void* team, int format, const float* queries,
                         const void* cache_k, const void* cache_v,
                         const float* k_scales, const float* v_scales,
                         int heads, int kv_heads, int head_dim, int span,
                         float* scratch, float* out) {
  Team& pool = *static_cast<Team*>(team);
  const int group = heads / kv_heads;
  const int kv_dim = kv_heads * head_dim;
  const float scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
  const int threads = pool.threads();
  if (threads > 1 && span >= 256) {  // uses_gqa, qwen2.cpp:1306-1311
    const int base_chunks =
        std::min(16, std::max(1, (threads * 2 + kv_heads - 1) / kv_heads));
    const int chunks =
        span >= 1024 ? std::min(16, std::max(4, base_chunks)) : base_chunks;
    const int chunk_size = (span + chunks - 1) / chunks;
    const int actual = (span + chunk_size - 1) / chunk_size;
    float* maxima = scratch;
    float* sums = maxima + static_cast<std::size_t>(kv_heads) * 16 * group;
    float* acc = sums + static_cast<std::size_t>(kv_heads) * 16 * group;
    pool.parallel_for(kv_heads * actual, [&](int task) {
      const int h = task / actual, c = task % actual;
      const int start = c * chunk_size;
      const int count = std::min(chunk_size, span - start);
      const std::size_t st = (static_cast<std::size_t>(h) * actual + c) * group;
      tge::cpu::AttentionGroupArgs a;
      a.queries = queries + static_cast<std::size_t>(h) * group * head_dim;
      set_kv(a, format, cache_k, cache_v, k_scales, v_scales,
             static_cast<std::size_t>(h) * head_dim +
                 static_cast<std::size_t>(start) * kv_dim);
      a.kv_stride = kv_dim;
      a.count = count;
      a.head_dim = head_dim;
      a.group_heads = group;
      a.scale = scale;
      a.maxima = maxima + st;
      a.sums = sums + st;
      a.accumulators = acc + st * head_dim;
      tge::cpu::attention_group_avx2(a);
    });
    float* red = acc + static_cast<std::size_t>(kv_heads) * 16 * group * head_dim;
    for (int head = 0; head < heads; ++head) {
      const int h = head / group;
      merge_chunks(maxima, sums, acc,
                   static_cast<std::size_t>(h) * actual * group, actual, group,
                   head % group, head_dim, red,
                   out + static_cast<std::size_t>(head) * head_dim);
    }
    return;
  }
  auto one = [&](int head, float* scores) {
    tge::cpu::AttentionArgs a;
    a.query = queries + static_cast<std::size_t>(head) * head_dim;
    set_kv(a, format, cache_k, cache_v, k_scales, v_scales,
           static_cast<std::size_t>(head / group) * head_dim);
    a.kv_stride = kv_dim;
    a.span = span;
    a.head_dim = head_dim;
    a.scale = scale;
    a.scores = scores;
    a.out = out + static_cast<std::size_t>(head) * head_dim;
    tge::cpu::attention_head_avx2(a);
  };
  if (threads <= 1 || span - 1 < 64) {
    for (int head = 0; head < heads; ++head) one(head, scratch);
    return;
  }
  pool.parallel_for(heads, [&](int head) {
    one(head, scratch + static_cast<std::size_t>(head) * span);
  });
}

// forward_batch attention (qwen2.cpp:1705-1747): `count` query rows, row i
// belongs to the flat slot at slot_bases[i] (element offset into the caches)
// and attends spans[i] positions; every head runs attention_head_avx2.
// scores must hold count*heads*max_span floats.
void ref_baseline_batch_heads(void* team, int format, const float* queries,
                              const void* cache_k, const void* cache_v,
                              const float* k_scales, const float* v_scales,
                              const std::int64_t* slot_bases, const int* spans,
                              int count, int heads, int kv_heads, int head_dim,
                              int max_span, float* scores, float* out) {
  Team& pool = *static_cast<Team*>(team);
  const int group = heads / kv_heads;
  const int kv_dim = kv_heads * head_dim;
  const int dim = heads * head_dim;
  const float scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
  auto one = [&](int row, int head) {
    tge::cpu::AttentionArgs a;
    a.query = queries + static_cast<std::size_t>(row) * dim +
              static_cast<std::size_t>(head) * head_dim;
    set_kv(a, format, cache_k, cache_v, k_scales, v_scales,
           static_cast<std::size_t>(slot_bases[row]) +
               static_cast<std::size_t>(head / group) * head_dim);
    a.kv_stride = kv_dim;
    a.span = spans[row];
    a.head_dim = head_dim;
    a.scale = scale;
    a.scores = scores + (static_cast<std::size_t>(row) * heads + head) * max_span;
    a.out = out + static_cast<std::size_t>(row) * dim +
            static_cast<std::size_t>(head) * head_dim;
    tge::cpu::attention_head_avx2(a);
  };
  if (count >= pool.threads()) {
    pool.parallel_for(count, [&](int row) {
      for (int head = 0; head < heads; ++head) one(row, head);
    });
  } else {
    pool.parallel_for(count * heads, [&](int task) { one(task / heads, task % heads); });
  }
}

// attention_batch's query-block path (qwen2.cpp:1540-1571): one task per
// query head. scores must hold heads*tokens*context floats.
void ref_baseline_block_prefill(void* team, int format, const float* queries,
                                const void* cache_k, const void* cache_v,
                                int tokens, int start_position, int heads,
                                int kv_heads, int head_dim, int context,
                                float* scores, float* out) {
  Team& pool = *static_cast<Team*>(team);
  const int group = heads / kv_heads;
  tge::cpu::AttentionBlockArgs b;
  b.queries = queries;
  if (format == kF16) {
    b.half = true;
    b.keys_half = static_cast<const std::uint16_t*>(cache_k);
    b.values_half = static_cast<const std::uint16_t*>(cache_v);
  } else {
    b.keys = static_cast<const float*>(cache_k);
    b.values = static_cast<const float*>(cache_v);
  }
  b.tokens = tokens;
  b.start_position = start_position;
  b.head_dim = head_dim;
  b.kv_stride = kv_heads * head_dim;
  b.query_stride = heads * head_dim;
  b.score_stride = heads * context;
  b.context = context;
  b.scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
  b.out = out;
  pool.parallel_for(heads, [&](int head) {
    tge::cpu::AttentionBlockArgs h = b;
    h.kv_head_offset = (head / group) * head_dim;
    h.scores = scores + static_cast<std::size_t>(head) * context;
    tge::cpu::attention_block_head_avx2(h, head);
  });
}

// f16 store of `rows` K and V rows (qwen2.cpp:2073-2082), sequential.
void ref_baseline_append_f16(const float* k, const float* v, int rows,
                             int kv_dim, std::uint16_t* k_out,
                             std::uint16_t* v_out) {
  const std::size_t n = static_cast<std::size_t>(rows) * kv_dim;
  for (std::size_t i = 0; i < n; ++i) {
    k_out[i] = tge::cpu::float_to_half(k[i]);
    v_out[i] = tge::cpu::float_to_half(v[i]);
  }
}

}  // extern "C"
