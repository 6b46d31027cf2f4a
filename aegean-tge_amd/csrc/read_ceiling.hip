// Read-only streaming kernels that measure the HBM read ceiling of the GPU
// the library runs on: the figure the decode kernel's bandwidth is judged
// against beside the 8 TB/s specification. Measurement helper only; nothing
// on the attention path calls it.
//
// Patterns (every byte of the buffer is read exactly once per launch):
//   TGE_READ_STREAM  16 bytes per lane, a workgroup's 4 KiB chunks spread
//                    over the grid (chunk c of the buffer goes to workgroup
//                    c mod grid), UNROLL chunks in flight per lane;
//   TGE_READ_BLOCKS  whole blocks of `block_bytes` (the page-block size of a
//                    pool, e.g. 4352 for int8 at head_dim 128), one wave per
//                    block, each load a contiguous KiB with the non-temporal
//                    policy, blocks taken in a scattered order (block
//                    i*stride mod n, stride coprime to n), two blocks in
//                    flight per wave: the access shape of the decode kernel.
// The loaded words are folded into one value that is stored only when it
// equals an impossible key, so the loads cannot be dropped and nothing is
// written.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tge_kernels.h"

namespace tge {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kChunk = 256 * 16;  // bytes one workgroup reads per load round

// the word the kernels would store to (never, in practice)
__device__ uint32_t g_read_sink;

template <int UNROLL>
__global__ __launch_bounds__(256) void read_stream_kernel(const char* buf, size_t chunks,
                                                          uint32_t key, uint32_t* sink) {
  const size_t grid = gridDim.x;
  uint32_t acc = 0;
  size_t c = blockIdx.x;
  // full rounds: UNROLL chunks of this workgroup in flight at once
  for (; c + (UNROLL - 1) * grid < chunks; c += UNROLL * grid) {
    u32x4_t v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const char* p = buf + (c + u * grid) * kChunk + threadIdx.x * 16;
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; c < chunks; c += grid) {
    const u32x4_t v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(buf + c * kChunk + threadIdx.x * 16));
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == key) sink[0] = acc;
}

// One wave per block; PIECES 16-byte loads per lane cover 1 KiB each, the
// buffer resource bounds the block (lanes past its end read zeros).
template <int PIECES>
__device__ __forceinline__ uint32_t load_block(const char* buf, size_t blk, uint32_t block_bytes,
                                               int lane, u32x4_t (&r)[PIECES]) {
  const auto rs = rsrc(buf + blk * block_bytes, block_bytes);
#pragma unroll
  for (int i = 0; i < PIECES; ++i)
    r[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, i * 1024 + lane * 16, 0, 2));
  return 0;
}

template <int PIECES>
__global__ __launch_bounds__(256) void read_blocks_kernel(const char* buf, uint32_t nblocks,
                                                          uint32_t block_bytes, uint32_t stride,
                                                          uint32_t key, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const uint32_t waves = gridDim.x * 4;
  const uint32_t w = blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t acc = 0;
  auto block_of = [&](uint32_t i) { return (size_t)(((uint64_t)i * stride) % nblocks); };
  u32x4_t a[PIECES], b[PIECES];
  uint32_t i = w;
  if (i < nblocks) load_block<PIECES>(buf, block_of(i), block_bytes, lane, a);
  for (; i < nblocks; i += 2 * waves) {
    const uint32_t j = i + waves;
    if (j < nblocks) load_block<PIECES>(buf, block_of(j), block_bytes, lane, b);
#pragma unroll
    for (int k = 0; k < PIECES; ++k) acc ^= a[k].x ^ a[k].w;
    if (j >= nblocks) break;
    const uint32_t n = j + waves;
    if (n < nblocks) load_block<PIECES>(buf, block_of(n), block_bytes, lane, a);
#pragma unroll
    for (int k = 0; k < PIECES; ++k) acc ^= b[k].y ^ b[k].z;
  }
  if (acc == key) sink[0] = acc;
}

}  // namespace

hipError_t launch_read_ceiling(const void* buf, size_t bytes, int pattern, int workgroups,
                               int block_bytes, hipStream_t stream) {
  const char* b = static_cast<const char*>(buf);
  uint32_t* sink = nullptr;
  const hipError_t e = hipGetSymbolAddress(reinterpret_cast<void**>(&sink), HIP_SYMBOL(g_read_sink));
  if (e != hipSuccess) return e;
  if (pattern == 0) {
    const size_t chunks = bytes / kChunk;
    hipLaunchKernelGGL(read_stream_kernel<8>, dim3(workgroups), dim3(256), 0, stream, b, chunks,
                       0x9e3779b9u, sink);
  } else {
    const uint32_t n = (uint32_t)(bytes / (size_t)block_bytes);
    // a stride near n / golden ratio, made coprime to n
    uint32_t s = (uint32_t)((double)n * 0.6180339887) | 1u;
    auto gcd = [](uint32_t x, uint32_t y) {
      while (y) {
        const uint32_t t = x % y;
        x = y;
        y = t;
      }
      return x;
    };
    while (gcd(s, n) != 1) s += 2;
    const int pieces = (block_bytes + 1023) / 1024;
    if (pieces <= 5) {
      hipLaunchKernelGGL(read_blocks_kernel<5>, dim3(workgroups), dim3(256), 0, stream, b, n,
                         (uint32_t)block_bytes, s, 0x9e3779b9u, sink);
    } else {
      hipLaunchKernelGGL(read_blocks_kernel<17>, dim3(workgroups), dim3(256), 0, stream, b, n,
                         (uint32_t)block_bytes, s, 0x9e3779b9u, sink);
    }
  }
  return hipGetLastError();
}

}  // namespace tge
