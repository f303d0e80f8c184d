// A plain streaming read: the HBM read rate a kernel that does nothing but
// read 16-byte vectors reaches on this GPU.  It is the measured ceiling the
// GEMMs' byte rates are set beside (the published 8 TB/s is the memory
// interface's peak, which no kernel here reaches).  Measurement only: no
// counterpart in the reference.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxr_moe {
namespace {

// Grid-stride over n vectors, four loads in flight per thread, each with the
// non-temporal hint (every byte is read once: measured on this GPU, 224 MB
// streams at 6.4-6.8 TB/s that way against 5.6-6.0 with plain loads, over
// grids of 256 to 4096 workgroups).  Every vector is folded into an XOR that
// is stored (to the caller's sink word) only when it equals a constant, so
// the compiler keeps the loads.
constexpr int kReadThreads = 256, kReadUnroll = 4, kReadGrid = 4096;
__global__ __launch_bounds__(kReadThreads) void read_probe_kernel(const u32x4_t* __restrict__ p,
                                                                  int64_t n, uint32_t* sink) {
  uint32_t acc = 0u;
  const int64_t stride = (int64_t)gridDim.x * kReadThreads * kReadUnroll;
  for (int64_t i = (int64_t)blockIdx.x * kReadThreads * kReadUnroll + threadIdx.x; i < n;
       i += stride) {
    u32x4_t v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const int64_t j = i + (int64_t)kReadThreads * u;
      v[u] = j < n ? __builtin_nontemporal_load(p + j) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) *sink = acc;
}

}  // namespace

hipError_t launch_read_probe(const void* buf, size_t bytes, uint32_t* sink, hipStream_t s) {
  if (bytes < 16) return hipSuccess;
  ProfileScope prof("read_probe", s);
  read_probe_kernel<<<kReadGrid, kReadThreads, 0, s>>>(static_cast<const u32x4_t*>(buf),
                                                       (int64_t)(bytes / 16), sink);
  return hipGetLastError();
}

}  // namespace mlxr_moe
