// Fused quantize-and-scatter KV append, and the page -> flat-row gather.
//
// Append replaces the reference's per-token store loops (qwen2.cpp:2073-2093
// forward, 1681-1702 forward_batch, 2308-2329 prefill_run; i8 via
// store_kv_q8/quantize_kv_block, qwen2.cpp:88-120). Four lanes own one
// 32-value block of one K or V row of one KV head: they read its 128 input
// bytes, convert or quantize them with the reference's bit recipe, and
// write them straight into the page block at the token's slot. A second
// entry fuses the step before the store (bias add and NeoX RoPE of q and k).
// This TU is built with -ffp-contract=off in addition to the explicit _rn
// intrinsics.
#include "append_common.h"

namespace tge {
namespace {

// Append: four lanes per (row, K|V, kv head, 32-value block), each owning 8
// consecutive values (two 16-byte loads).
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

  // (dims past the head's own are stored as zeros)
  const int d0 = b * 32 + quarter * 8;
  float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const float* head_row = (which ? p.v : p.k) + (size_t)row * p.kv_heads * p.dims + h * p.dims;
  if ((p.dims & 7) == 0) {
    if (d0 < p.dims) load8(x, head_row + d0);
  } else {
    load8_head(x, head_row, d0, p.dims);
  }
  store_lane<FMT>(p, x, p.rows[row], which, h, b, quarter, live);
}

// NeoX rotation of one (low, high) pair by (c, s), in the rounding of
// apply_rope_avx2 (attention's default CPU path: l*c - (h*s) and
// l*s + (h*c) with one rounding each, norm_rope_avx2.cpp:97-131) or of
// apply_rope_scalar (every product and the sum rounded,
// norm_rope_scalar.cpp:23-40).
__device__ __forceinline__ void rope_pair(float l, float h, float c, float s, bool fma, float& lo,
                                          float& hi) {
  if (fma) {
    lo = __fmaf_rn(l, c, -__fmul_rn(h, s));
    hi = __fmaf_rn(l, s, __fmul_rn(h, c));
  } else {
    lo = __fsub_rn(__fmul_rn(l, c), __fmul_rn(h, s));
    hi = __fadd_rn(__fmul_rn(l, s), __fmul_rn(h, c));
  }
}

// Bias + RoPE + append in one launch: the reference's per-token sequence
// q += q_bias, k += k_bias, v += v_bias, apply_rope(q), apply_rope(k), store
// (qwen2.cpp:2062-2093, 1665-1702, 2286-2329). Per row, the lanes are
// [K lanes | V lanes | Q lanes]:
//   - K/V: four lanes per (K|V, kv head, 32-value block), as in the plain
//     append; a K lane also reads the 8 partner values half a head away
//     (NeoX halves) and rotates its own 8;
//   - Q: one lane per (q head, 8 low dims): it rotates those 8 and their 8
//     high partners together and writes both, so q_out may alias q.
template <int FMT>
__global__ __launch_bounds__(256) void kv_append_rope_kernel(AppendParams p) {
  const int D = p.dims, half = D >> 1, nb = p.head_dim >> 5;  // pairs of the head's own dims
  const int kv_lanes = 2 * p.kv_heads * nb * 4;
  const int q_used = p.q ? p.q_heads * (half >> 3) : 0;
  // rounded up to a multiple of 4 so every row starts on a quad and the
  // int8 blocks' four lanes stay in one aligned quad of the wave
  const int per_row = kv_lanes + ((q_used + 3) & ~3);
  const long total = (long)p.n_rows * per_row;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = idx < total;
  const long id = live ? idx : total - 1;
  const int row = (int)(id / per_row);
  const int r = (int)(id % per_row);
  const RowRec rr = p.rows[row];
  const float* cs = p.rope_cos + (size_t)rr.pos * half;
  const float* sn = p.rope_sin + (size_t)rr.pos * half;
  const bool fma = p.rope_fma != 0;

  if (r >= kv_lanes) {  // Q lane (whole quads of lanes: no block shares a quad with it)
    const int qi = r - kv_lanes;
    if (!live || qi >= q_used) return;  // past the grid, or a padding lane of the row
    const int hq = qi / (half >> 3);
    const int j = 8 * (qi % (half >> 3));
    const size_t o = (size_t)row * p.q_heads * D + (size_t)hq * D;
    float lo[8], hi[8];
    load8(lo, p.q + o + j);
    load8(hi, p.q + o + half + j);
    if (p.q_bias) {
      float bl[8], bh[8];
      load8(bl, p.q_bias + hq * D + j);
      load8(bh, p.q_bias + hq * D + half + j);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        lo[i] = __fadd_rn(lo[i], bl[i]);
        hi[i] = __fadd_rn(hi[i], bh[i]);
      }
    }
    float c[8], s[8], ol[8], oh[8];
    load8(c, cs + j);
    load8(s, sn + j);
#pragma unroll
    for (int i = 0; i < 8; ++i) rope_pair(lo[i], hi[i], c[i], s[i], fma, ol[i], oh[i]);
    float* dst = p.q_out + o;
    reinterpret_cast<float4*>(dst + j)[0] = make_float4(ol[0], ol[1], ol[2], ol[3]);
    reinterpret_cast<float4*>(dst + j)[1] = make_float4(ol[4], ol[5], ol[6], ol[7]);
    reinterpret_cast<float4*>(dst + half + j)[0] = make_float4(oh[0], oh[1], oh[2], oh[3]);
    reinterpret_cast<float4*>(dst + half + j)[1] = make_float4(oh[4], oh[5], oh[6], oh[7]);
    return;
  }
  const int quarter = r & 3;
  int rest = r >> 2;
  const int b = rest % nb;
  rest /= nb;
  const int h = rest % p.kv_heads;
  const int which = rest / p.kv_heads;
  const int kv_dim = p.kv_heads * D;
  const int d0 = 32 * b + 8 * quarter;
  if (d0 >= D) {  // a dim past the head's own: stored as zero
    const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    store_lane<FMT>(p, z, rr, which, h, b, quarter, live);
    return;
  }
  const float* src = (which ? p.v : p.k) + (size_t)row * kv_dim + h * D;
  const float* bias = which ? p.v_bias : p.k_bias;
  float x[8];
  load8(x, src + d0);
  if (bias) {
    float bx[8];
    load8(bx, bias + h * D + d0);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = __fadd_rn(x[i], bx[i]);
  }
  if (which == 0) {
    // the partner half: dims d0 +- half (a lane's 8 dims lie in one half:
    // half is a multiple of 8)
    const bool low = d0 < half;
    const int dp = low ? d0 + half : d0 - half;
    float y[8];
    load8(y, src + dp);
    if (bias) {
      float by[8];
      load8(by, bias + h * D + dp);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = __fadd_rn(y[i], by[i]);
    }
    const int j = low ? d0 : dp;  // table index of the pair
    float c[8], s[8];
    load8(c, cs + j);
    load8(s, sn + j);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float ol, oh;
      rope_pair(low ? x[i] : y[i], low ? y[i] : x[i], c[i], s[i], fma, ol, oh);
      x[i] = low ? ol : oh;
    }
  }
  store_lane<FMT>(p, x, rr, which, h, b, quarter, live);
}

// One thread per (position, kv head, element) of the gathered rows.
template <typename T>
__global__ __launch_bounds__(256) void kv_gather_kernel(GatherParams p) {
  const int kv_dim = p.kv_heads * p.dims;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)p.count * kv_dim;
  if (idx >= total) return;
  const int pos = (int)(idx / kv_dim);
  const int c = (int)(idx % kv_dim);
  const int h = c / p.dims, d = c % p.dims;
  const int page = p.table[pos >> 4], t = pos & 15;
  const int np = p.head_dim >> 5;
  const char* blk = static_cast<const char*>(p.pool) + ((size_t)page * p.kv_heads + h) * p.geom.block_bytes;
  static_cast<T*>(p.k_rows)[idx] = reinterpret_cast<const T*>(blk)[k_index(t, d, (int)sizeof(T))];
  static_cast<T*>(p.v_rows)[idx] = reinterpret_cast<const T*>(blk + p.geom.v_off())[v_index(t, d, (int)sizeof(T))];
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

hipError_t launch_kv_append_rope(int format, const AppendParams& p, hipStream_t stream) {
  const int nb = p.head_dim >> 5;
  const long q_used = p.q ? (long)p.q_heads * (p.dims >> 4) : 0;
  const long per_row = 2L * p.kv_heads * nb * 4 + ((q_used + 3) & ~3L);
  const long total = (long)p.n_rows * per_row;
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (format == kF16) {
    hipLaunchKernelGGL(kv_append_rope_kernel<kF16>, grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(kv_append_rope_kernel<kI8>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_kv_gather(int format, const GatherParams& p, hipStream_t stream) {
  const long total = (long)p.count * p.kv_heads * p.dims;
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
