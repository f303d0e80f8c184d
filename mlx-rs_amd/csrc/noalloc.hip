// The block forward for callers that cannot allocate device memory (code
// under graph capture, tight serving loops, harnesses that forbid
// hipMalloc): its scratch is a file-scope device array of the library,
// one copy per GPU, instead of a caller workspace.
//
// The array's name is a host-side stand-in in host code, not a device
// address: the host learns each device's address once, with that device
// current, through hipGetSymbolAddress, and passes only that address to the
// kernels (as the workspace of mlxr_moe_block_forward, whose kernels and
// checks this entry shares).  Nothing here allocates: no hipMalloc, no
// hipFree, no library routine that allocates.  The array keeps the last
// call's contents; nothing in it needs to start at zero (the routing kernel
// clears the status word, every other scratch value is written before it
// is read).  Calls that overlap on one GPU (two streams, two threads) share
// the array and race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/mlxr_moe.h"
#include "nn.hpp"

namespace mlxr_moe {
namespace {

static __device__ __align__(256) char scratch[MLXR_MOE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The scratch array's device address on `dev`, looked up once per device
// with that device current (the caller's current device is restored).
void* scratch_on(int dev, std::string* err) {
  if (dev < 0 || dev >= kMaxDevices) {
    *err = "block_forward_noalloc: device " + std::to_string(dev) +
           " out of range";
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[dev]) return g_ptr[dev];
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  void* p = nullptr;
  if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur >= 0 && cur != dev) {
    const hipError_t r = hipSetDevice(cur);
    if (e == hipSuccess) e = r;
  }
  if (e != hipSuccess || !p) {
    *err = std::string("block_forward_noalloc: scratch address: ") +
           hipGetErrorString(e);
    return nullptr;
  }
  g_ptr[dev] = p;
  return p;
}

}  // namespace
}  // namespace mlxr_moe

using namespace mlxr_moe;

// Also the set-up call: it resolves the array's address on the current
// device (when there is one), so that a later call made under graph capture
// runs no lookup.
extern "C" size_t mlxr_moe_noalloc_scratch_size(void) {
  int dev = -1;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0) {
    std::string err;
    (void)scratch_on(dev, &err);  // a failure is reported by the entry itself
  }
  return MLXR_MOE_NOALLOC_SCRATCH_BYTES;
}

extern "C" int mlxr_moe_block_forward_noalloc(const mlxr_moe_block* block,
                                              const void* x, int64_t T,
                                              void* out, int32_t* topk_idx,
                                              float* topk_w,
                                              mlxr_moe_stream stream) {
  if (!block) return capi_fail("block_forward_noalloc: null module");
  const Status st = nn::Qwen35MoeBlock(*block).validate();
  if (!st.ok) return capi_fail(st.what);
  if (T < 0) return capi_fail("block_forward_noalloc: bad T");
  const size_t need = mlxr_moe_block_workspace_size(block, T);
  if (need > (size_t)MLXR_MOE_NOALLOC_SCRATCH_BYTES)
    return capi_fail("block_forward_noalloc: T = " + std::to_string(T) +
                     " needs " + std::to_string(need) +
                     " bytes of scratch, more than the library's " +
                     std::to_string(MLXR_MOE_NOALLOC_SCRATCH_BYTES) +
                     "-byte array; call mlxr_moe_block_forward with a "
                     "workspace");
  if (T == 0) return 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = -1;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess)
    return capi_fail(std::string("block_forward_noalloc: stream device: ") +
                     hipGetErrorString(e));
  std::string err;
  void* ws = scratch_on(dev, &err);
  if (!ws) return capi_fail(err);
  return mlxr_moe_block_forward(block, x, T, out, topk_idx, topk_w, ws,
                                MLXR_MOE_NOALLOC_SCRATCH_BYTES, stream);
}
