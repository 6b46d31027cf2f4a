// Upload of a step's plan: a kernel copies the pinned host staging buffer
// into device memory. On the launch stream a DMA-engine copy between two
// kernels costs a queue hand-off on each side (about 25 us each way on an
// MI355X, against a few microseconds for this kernel), once per step.
//
// The loads read host memory over the bus with the system-coherent cache
// policy (sc0 sc1): the staging buffer is rewritten for every step, so no
// line of it may be served from a GPU cache. The stores are plain; the
// kernels that read the plan run after this one on the same stream.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tge_kernels.h"

namespace tge {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSysPolicy = 1 | 16;  // buffer cache-policy operand: sc0 | sc1 (system scope)

__global__ __launch_bounds__(256) void upload_kernel(char* dst, const char* src, uint32_t n) {
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(src), (short)0, (int)n, 0x00020000);
  const uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 16u;
  if (i + 16 <= n) {
    const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, i, 0, kSysPolicy));
    *reinterpret_cast<u32x4_t*>(dst + i) = v;
  } else if (i < n) {
    for (uint32_t j = i; j < n; ++j) dst[j] = (char)__builtin_amdgcn_raw_buffer_load_b8(rs, j, 0, kSysPolicy);
  }
}

}  // namespace

hipError_t launch_upload(char* dst, const char* src_dev, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if (n > 0x7fffffffu) return hipErrorInvalidValue;  // (plans are far smaller)
  const unsigned chunks = (unsigned)((n + 15) / 16);
  hipLaunchKernelGGL(upload_kernel, dim3((chunks + 255) / 256), dim3(256), 0, stream, dst, src_dev,
                     (uint32_t)n);
  return hipGetLastError();
}

}  // namespace tge
