// Fused quantize-and-scatter KV append, and the page -> flat-row gather.
//
// Append replaces the reference's per-token store loops (qwen2.cpp:2073-2093
// forward, 1681-1702 forward_batch, 2308-2329 prefill_run; i8 via
// store_kv_q8/quantize_kv_block, qwen2.cpp:88-120). One thread owns one
// 32-value block of one K or V row of one KV head: it reads the 128 input
// bytes, converts or quantizes them with the reference's bit recipe, and
// writes them straight into the page block at the token's slot. This TU is
// built with -ffp-contract=off in addition to the explicit _rn intrinsics.
#include "tge_common.h"
#include "tge_kernels.h"

namespace tge {
namespace {

template <int FMT>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
  const int nb = p.head_dim >> 5;
  const long total = (long)p.n_rows * 2 * p.kv_heads * nb;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  // idx -> (row, which, head, block), block fastest so neighbouring threads
  // read neighbouring 128-byte slices of the same input row.
  const int b = (int)(idx % nb);
  long rest = idx / nb;
  const int h = (int)(rest % p.kv_heads);
  rest /= p.kv_heads;
  const int which = (int)(rest & 1);
  const int row = (int)(rest >> 1);

  const RowRec rr = p.rows[row];
  const int kv_dim = p.kv_heads * p.head_dim;
  const float* src = (which ? p.v : p.k) + (size_t)row * kv_dim + h * p.head_dim + b * 32;
  float x[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 f = reinterpret_cast<const float4*>(src)[i];
    x[4 * i + 0] = f.x;
    x[4 * i + 1] = f.y;
    x[4 * i + 2] = f.z;
    x[4 * i + 3] = f.w;
  }
  char* const blk = static_cast<char*>(p.pool) + ((size_t)rr.page * p.kv_heads + h) * p.geom.block_bytes;
  const int t = rr.slot;

  if (FMT == kF16) {
    uint16_t hx[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) hx[i] = float_to_half_ref(x[i]);
    if (which == 0) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(blk);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint4 w;
        w.x = hx[4 * g + 0] | ((uint32_t)hx[4 * g + 1] << 16);
        w.y = hx[4 * g + 2] | ((uint32_t)hx[4 * g + 3] << 16);
        w.z = hx[16 + 4 * g + 0] | ((uint32_t)hx[16 + 4 * g + 1] << 16);
        w.w = hx[16 + 4 * g + 2] | ((uint32_t)hx[16 + 4 * g + 3] << 16);
        *reinterpret_cast<uint4*>(dst + k_index_np(t, 32 * b + 4 * g, nb)) = w;
      }
    } else {
      uint16_t* dst = reinterpret_cast<uint16_t*>(blk + p.geom.v_off());
#pragma unroll
      for (int d = 0; d < 32; ++d) dst[v_index_np(t, 32 * b + d, nb)] = hx[d];
    }
  } else {
    int8_t c[32];
    const float scale = quantize_block_ref(x, c);
    if (which == 0) {
      int8_t* dst = reinterpret_cast<int8_t*>(blk);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 w;
        w.x = (uint8_t)c[4 * g] | ((uint32_t)(uint8_t)c[4 * g + 1] << 8) |
              ((uint32_t)(uint8_t)c[4 * g + 2] << 16) | ((uint32_t)(uint8_t)c[4 * g + 3] << 24);
        w.y = (uint8_t)c[16 + 4 * g] | ((uint32_t)(uint8_t)c[16 + 4 * g + 1] << 8) |
              ((uint32_t)(uint8_t)c[16 + 4 * g + 2] << 16) |
              ((uint32_t)(uint8_t)c[16 + 4 * g + 3] << 24);
        *reinterpret_cast<uint2*>(dst + k_index_np(t, 32 * b + 4 * g, nb)) = w;
      }
    } else {
      int8_t* dst = reinterpret_cast<int8_t*>(blk + p.geom.v_off());
#pragma unroll
      for (int d = 0; d < 32; ++d) dst[v_index_np(t, 32 * b + d, nb)] = c[d];
    }
    char* sp = blk + (which ? p.geom.vs_off() : p.geom.ks_off());
    if (p.scale_f32) {
      reinterpret_cast<float*>(sp)[scale_index_np(t, b, nb)] = scale;
    } else {
      reinterpret_cast<uint16_t*>(sp)[scale_index_np(t, b, nb)] = float_to_half_ref(scale);
    }
  }
}

// One thread per (position, kv head, element) of the gathered rows.
template <typename T>
__global__ __launch_bounds__(256) void kv_gather_kernel(GatherParams p) {
  const int kv_dim = p.kv_heads * p.head_dim;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)p.count * kv_dim;
  if (idx >= total) return;
  const int pos = (int)(idx / kv_dim);
  const int c = (int)(idx % kv_dim);
  const int h = c / p.head_dim, d = c % p.head_dim;
  const int page = p.table[pos >> 4], t = pos & 15;
  const int np = p.head_dim >> 5;
  const char* blk = static_cast<const char*>(p.pool) + ((size_t)page * p.kv_heads + h) * p.geom.block_bytes;
  static_cast<T*>(p.k_rows)[idx] = reinterpret_cast<const T*>(blk)[k_index_np(t, d, np)];
  static_cast<T*>(p.v_rows)[idx] = reinterpret_cast<const T*>(blk + p.geom.v_off())[v_index_np(t, d, np)];
  if (p.k_scales && (d & 31) == 0) {
    const size_t o = (size_t)pos * (kv_dim >> 5) + (c >> 5);
    const int si = scale_index_np(t, d >> 5, np);
    const char* ks = blk + p.geom.ks_off();
    const char* vs = blk + p.geom.vs_off();
    if (p.scale_bytes == 4) {
      static_cast<float*>(p.k_scales)[o] = reinterpret_cast<const float*>(ks)[si];
      static_cast<float*>(p.v_scales)[o] = reinterpret_cast<const float*>(vs)[si];
    } else {
      static_cast<uint16_t*>(p.k_scales)[o] = reinterpret_cast<const uint16_t*>(ks)[si];
      static_cast<uint16_t*>(p.v_scales)[o] = reinterpret_cast<const uint16_t*>(vs)[si];
    }
  }
}

}  // namespace

hipError_t launch_kv_append(int format, const AppendParams& p, hipStream_t stream) {
  const long total = (long)p.n_rows * 2 * p.kv_heads * (p.head_dim >> 5);
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (format == kF16) {
    hipLaunchKernelGGL(kv_append_kernel<kF16>, grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(kv_append_kernel<kI8>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_kv_gather(int format, const GatherParams& p, hipStream_t stream) {
  const long total = (long)p.count * p.kv_heads * p.head_dim;
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (format == kF16) {
    hipLaunchKernelGGL(kv_gather_kernel<uint16_t>, grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(kv_gather_kernel<int8_t>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace tge
