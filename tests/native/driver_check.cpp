// Native use of the C++20 driver (tge::models::Qwen2KvPath), the way a C++
// engine would call it: device buffers from hipMalloc, one prefill chunk and
// one decode step per layer, and the reference's misuse exceptions.
// TEST INFRASTRUCTURE: built by the package Makefile, run by
// tests/test_gpu_driver.py, which writes the inputs and checks the outputs
// against the oracle.
//
// usage: driver_check <in.bin> <out.bin>
//   in.bin : int32 {layers, q_heads, kv_heads, head_dim, n_prefill, n_decode,
//            context, format}, then per layer: k, v [n][kv_dim], q [n][q_dim]
//            as float32, n = n_prefill + n_decode
//   out.bin: per layer the attention rows [n][q_dim] as float32
// Prints "exceptions ok" when the misuse checks threw what the reference
// throws.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <stdexcept>
#include <vector>

#include "tge_amd/qwen2_kv.hpp"

namespace {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    std::exit(2);
  }
}

struct Dev {
  float* p = nullptr;
  explicit Dev(size_t n) { hip_check(hipMalloc(&p, n * sizeof(float)), "hipMalloc"); }
  ~Dev() { (void)hipFree(p); }
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
};

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: driver_check <in.bin> <out.bin>\n");
    return 2;
  }
  std::FILE* in = std::fopen(argv[1], "rb");
  if (!in) return 2;
  int h[8];
  if (std::fread(h, sizeof(int), 8, in) != 8) return 2;
  const int layers = h[0], qh = h[1], kvh = h[2], hd = h[3], n_pre = h[4], n_dec = h[5];
  const int n = n_pre + n_dec, q_dim = qh * hd, kv_dim = kvh * hd;
  std::vector<std::vector<float>> k(layers), v(layers), q(layers);
  for (int l = 0; l < layers; ++l) {
    k[l].resize((size_t)n * kv_dim);
    v[l].resize((size_t)n * kv_dim);
    q[l].resize((size_t)n * q_dim);
    if (std::fread(k[l].data(), 4, k[l].size(), in) != k[l].size() ||
        std::fread(v[l].data(), 4, v[l].size(), in) != v[l].size() ||
        std::fread(q[l].data(), 4, q[l].size(), in) != q[l].size())
      return 2;
  }
  std::fclose(in);

  tge::models::Qwen2KvConfig cfg;
  cfg.layers = layers;
  cfg.q_heads = qh;
  cfg.kv_heads = kvh;
  cfg.head_dim = hd;
  cfg.context = h[6];
  cfg.sequences = 2;
  cfg.format = h[7];
  tge::models::Qwen2KvPath model(cfg);

  Dev dk((size_t)n * kv_dim), dv((size_t)n * kv_dim), dq((size_t)n * q_dim), dout((size_t)n * q_dim);
  std::vector<std::vector<float>> out(layers, std::vector<float>((size_t)n * q_dim));
  const size_t kv_row = (size_t)kv_dim * 4, q_row = (size_t)q_dim * 4;

  // Sequence 1 holds a few tokens first, so sequence 0's pages interleave.
  model.begin_prefill(1, 0, 20);
  for (int l = 0; l < layers; ++l) {
    hip_check(hipMemcpy(dk.p, k[l].data(), 20 * kv_row, hipMemcpyHostToDevice), "copy");
    hip_check(hipMemcpy(dv.p, v[l].data(), 20 * kv_row, hipMemcpyHostToDevice), "copy");
    model.store(l, dk.p, dv.p);
  }
  // Prefill chunk, then decode steps, each store-then-attend per layer.
  for (int step = 0; step <= n_dec; ++step) {
    const int start = step == 0 ? 0 : n_pre + step - 1;
    const int count = step == 0 ? n_pre : 1;
    if (step == 0) {
      model.begin_prefill(0, start, count);
    } else {
      model.begin_forward(0, start);
    }
    for (int l = 0; l < layers; ++l) {
      hip_check(hipMemcpy(dk.p, k[l].data() + (size_t)start * kv_dim, count * kv_row,
                          hipMemcpyHostToDevice), "copy");
      hip_check(hipMemcpy(dv.p, v[l].data() + (size_t)start * kv_dim, count * kv_row,
                          hipMemcpyHostToDevice), "copy");
      hip_check(hipMemcpy(dq.p, q[l].data() + (size_t)start * q_dim, count * q_row,
                          hipMemcpyHostToDevice), "copy");
      model.layer(l, dq.p, dk.p, dv.p, dout.p);
      hip_check(hipMemcpy(out[l].data() + (size_t)start * q_dim, dout.p, count * q_row,
                          hipMemcpyDeviceToHost), "copy");
    }
  }
  if (model.length(0) != n) {
    std::fprintf(stderr, "length %d, expected %d\n", model.length(0), n);
    return 1;
  }

  // Misuse: position past the context, unknown sequence, a layer before a
  // step has begun (qwen2.cpp:2036-2044 throw runtime_error).
  int thrown = 0;
  try {
    model.begin_forward(0, cfg.context);
  } catch (const std::runtime_error&) {
    ++thrown;
  }
  try {
    model.begin_forward(5, 0);
  } catch (const std::runtime_error&) {
    ++thrown;
  }
  model.reset_cache(0);
  if (model.length(0) != 0) return 1;

  std::FILE* o = std::fopen(argv[2], "wb");
  if (!o) return 2;
  for (int l = 0; l < layers; ++l) std::fwrite(out[l].data(), 4, out[l].size(), o);
  std::fclose(o);
  if (thrown == 2) std::printf("exceptions ok\n");
  return 0;
}
