// Fused quantize-and-scatter KV append, and the page -> flat-row gather.
//
// Append replaces the reference's per-token store loops (qwen2.cpp:2073-2093
// forward, 1681-1702 forward_batch, 2308-2329 prefill_run; i8 via
// store_kv_q8/quantize_kv_block, qwen2.cpp:88-120). Four lanes own one
// 32-value block of one K or V row of one KV head: they read its 128 input
// bytes, convert or quantize them with the reference's bit recipe, and
// write them straight into the page block at the token's slot. This TU is
// built with -ffp-contract=off in addition to the explicit _rn intrinsics.
#include "tge_common.h"
#include "tge_kernels.h"

namespace tge {
namespace {

// Append: four lanes per (row, K|V, kv head, 32-value block), each owning 8
// consecutive values (two 16-byte loads). f16: each lane converts its 8
// values with the reference's float_to_half recipe. int8: the four lanes
// combine their absmax runs in order (see FoldRun), then each computes the
// block's scale and inverse exactly as quantize_kv_block does (correctly
// rounded fp32 division) and quantizes its 8 values.
template <int FMT>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
  const int nb = p.head_dim >> 5;
  const long total = (long)p.n_rows * 2 * p.kv_heads * nb * 4;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = idx < total;  // dead lanes still take part in the shuffles
  const long id = live ? idx : total - 1;
  // id -> (row, which, head, block, quarter), quarter fastest so the four
  // lanes of a block are adjacent and neighbouring blocks read neighbouring
  // 128-byte slices of the same input row.
  const int quarter = (int)(id & 3);
  long rest = id >> 2;
  const int b = (int)(rest % nb);
  rest /= nb;
  const int h = (int)(rest % p.kv_heads);
  rest /= p.kv_heads;
  const int which = (int)(rest & 1);
  const int row = (int)(rest >> 1);

  const RowRec rr = p.rows[row];
  const int kv_dim = p.kv_heads * p.head_dim;
  const float* src = (which ? p.v : p.k) + (size_t)row * kv_dim + h * p.head_dim + b * 32 + quarter * 8;
  float x[8];
  {
    const float4 f0 = reinterpret_cast<const float4*>(src)[0];
    const float4 f1 = reinterpret_cast<const float4*>(src)[1];
    x[0] = f0.x; x[1] = f0.y; x[2] = f0.z; x[3] = f0.w;
    x[4] = f1.x; x[5] = f1.y; x[6] = f1.z; x[7] = f1.w;
  }
  char* const blk = static_cast<char*>(p.pool) + ((size_t)rr.page * p.kv_heads + h) * p.geom.block_bytes;
  const int t = rr.slot;
  const int d0 = 32 * b + 8 * quarter;  // first dim of this lane
  // K chunk of (token t, dims d0..d0+3) and (d0+4..d0+7): 4 contiguous
  // elements each (k_index_np is contiguous in d&3).
  const int k0 = k_index_np(t, d0, nb);
  const int k1 = k_index_np(t, d0 + 4, nb);

  if (FMT == kF16) {
    uint16_t hx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) hx[i] = float_to_half_ref(x[i]);
    if (!live) return;
    if (which == 0) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(blk);
      *reinterpret_cast<uint2*>(dst + k0) = make_uint2(hx[0] | ((uint32_t)hx[1] << 16), hx[2] | ((uint32_t)hx[3] << 16));
      *reinterpret_cast<uint2*>(dst + k1) = make_uint2(hx[4] | ((uint32_t)hx[5] << 16), hx[6] | ((uint32_t)hx[7] << 16));
    } else {
      uint16_t* dst = reinterpret_cast<uint16_t*>(blk + p.geom.v_off());
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[v_index_np(t, d0 + i, nb)] = hx[i];
    }
  } else {
    // the block's absmax: lane runs joined in lane order
    const FoldRun mine = fold_run(x);
    const int base = (threadIdx.x & 63) & ~3;
    FoldRun all{false, -INFINITY};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const FoldRun o{__shfl(mine.nan ? 1 : 0, base + j) != 0, __shfl(mine.v, base + j)};
      all = j == 0 ? o : fold_join(all, o);
    }
    const float maximum = all.v;
    const float scale = __fdiv_rn(maximum, 127.0f);
    const float inverse = scale != 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
    uint32_t packed[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float scaled = __fmul_rn(x[i], inverse);
      const float rounded = scaled >= 0.0f ? __fadd_rn(scaled, 0.5f) : __fadd_rn(scaled, -0.5f);
      int c = trunc_to_int_x86(rounded);
      c = c > 127 ? 127 : (c < -127 ? -127 : c);
      packed[i >> 2] |= (uint32_t)(uint8_t)(int8_t)c << (8 * (i & 3));
    }
    if (!live) return;
    if (which == 0) {
      int8_t* dst = reinterpret_cast<int8_t*>(blk);
      *reinterpret_cast<uint32_t*>(dst + k0) = packed[0];
      *reinterpret_cast<uint32_t*>(dst + k1) = packed[1];
    } else {
      int8_t* dst = reinterpret_cast<int8_t*>(blk + p.geom.v_off());
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[v_index_np(t, d0 + i, nb)] = (int8_t)(packed[i >> 2] >> (8 * (i & 3)));
    }
    if (quarter == 0) {
      char* sp = blk + (which ? p.geom.vs_off() : p.geom.ks_off());
      if (p.scale_f32) {
        reinterpret_cast<float*>(sp)[scale_index_np(t, b, nb)] = scale;
      } else {
        reinterpret_cast<uint16_t*>(sp)[scale_index_np(t, b, nb)] = float_to_half_ref(scale);
      }
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
  const long total = (long)p.n_rows * 2 * p.kv_heads * (p.head_dim >> 5) * 4;
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
