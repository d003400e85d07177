// Measurement probe: a plain streaming read, the floor any single kernel
// that reads a buffer of this size once can reach on this part (launch,
// first-data latency and drain included).  Used beside the decode kernels
// at the same byte count; it computes nothing the attention stage needs.
#include "common.h"

namespace hl {
namespace {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// 16-byte loads, IPT of them in flight per thread per iteration, XOR-folded;
// the fold reaches memory only for one 2^-32-likely value, so the loads
// cannot be dropped and nothing is written.  CONTIG = 0: grid-stride (a
// launch-wide sweep, consecutive workgroups side by side); CONTIG = 1: each
// workgroup streams its own contiguous chunk, as a persistent kernel with one
// workgroup per CU would.
template <int IPT, int CONTIG>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4v* __restrict__ p, size_t n16,
                                                          unsigned* __restrict__ sink) {
  size_t i, end, stride;
  if (CONTIG) {
    const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
    i = (size_t)blockIdx.x * chunk + threadIdx.x;
    end = min(n16, (size_t)(blockIdx.x + 1) * chunk);
    stride = 256;
  } else {
    i = (size_t)blockIdx.x * 256 + threadIdx.x;
    end = n16;
    stride = (size_t)gridDim.x * 256;
  }
  u32x4v acc = {0u, 0u, 0u, 0u};
  for (; i + (IPT - 1) * stride < end; i += IPT * stride) {
    u32x4v v[IPT];
#pragma unroll
    for (int u = 0; u < IPT; ++u) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < IPT; ++u) acc ^= v[u];
  }
  for (; i < end; i += stride) acc ^= p[i];
  const unsigned v = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (v == 0x9E3779B9u) sink[0] = v;
}

template <int IPT, int CONTIG>
hipError_t probe_launch(const void* buf, size_t bytes, int blocks, unsigned* sink, hipStream_t st) {
  hipLaunchKernelGGL((stream_read_kernel<IPT, CONTIG>), dim3(blocks), dim3(256), 0, st, (const u32x4v*)buf,
                     bytes / 16, sink);
  return hipGetLastError();
}

}  // namespace
}  // namespace hl

extern "C" int hl_probe_stream_read_ex(const void* buf, size_t bytes, int blocks, int inflight, int contiguous,
                                       unsigned* sink, void* stream) {
  if (!buf || !sink || bytes < 16 || (bytes & 15) || ((uintptr_t)buf & 15)) return HL_EINVAL;
  if (blocks <= 0) blocks = 1024;
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (inflight == 4) e = contiguous ? hl::probe_launch<4, 1>(buf, bytes, blocks, sink, st) : hl::probe_launch<4, 0>(buf, bytes, blocks, sink, st);
  else if (inflight == 8) e = contiguous ? hl::probe_launch<8, 1>(buf, bytes, blocks, sink, st) : hl::probe_launch<8, 0>(buf, bytes, blocks, sink, st);
  else if (inflight == 16) e = contiguous ? hl::probe_launch<16, 1>(buf, bytes, blocks, sink, st) : hl::probe_launch<16, 0>(buf, bytes, blocks, sink, st);
  else return HL_EINVAL;
  return e == hipSuccess ? HL_OK : HL_EHIP;
}

extern "C" int hl_probe_stream_read(const void* buf, size_t bytes, int blocks, unsigned* sink, void* stream) {
  return hl_probe_stream_read_ex(buf, bytes, blocks, 4, 0, sink, stream);
}
