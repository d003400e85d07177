// Measurement probe: a plain streaming read, the floor any single kernel
// that reads a buffer of this size once can reach on this part (launch,
// first-data latency and drain included).  Used beside the decode kernels
// at the same byte count; it computes nothing the attention stage needs.
#include "common.h"

namespace hl {
namespace {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Grid-stride 16-byte loads, four in flight per thread per iteration,
// XOR-folded; the fold reaches memory only for one 2^-32-likely value, so
// the loads cannot be dropped and nothing is written.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4v* __restrict__ p, size_t n16,
                                                          unsigned* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  u32x4v acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4v a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const unsigned v = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (v == 0x9E3779B9u) sink[0] = v;
}

}  // namespace
}  // namespace hl

extern "C" int hl_probe_stream_read(const void* buf, size_t bytes, int blocks, unsigned* sink, void* stream) {
  if (!buf || !sink || bytes < 16 || (bytes & 15) || ((uintptr_t)buf & 15)) return HL_EINVAL;
  if (blocks <= 0) blocks = 1024;
  hipLaunchKernelGGL(hl::stream_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     (const hl::u32x4v*)buf, bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? HL_OK : HL_EHIP;
}
