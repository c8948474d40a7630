// noalloc.hip — mlxq_linear_noalloc: the fused linear forward with its LoRA staging buffers in a
// static device array instead of a caller workspace, for callers that cannot allocate device
// memory.  A promoted result (a bf16 product with an f32 bias, f32 LoRA factors or the f32 GELU)
// also stages the bf16 product [M, N] there.
//
// The array is a file-scope __device__ object, so every GPU the library runs on holds its own
// copy (MLXQ_NOALLOC_SCRATCH_BYTES) from the first call on that GPU until the process ends.  In
// host code its name is only a host-side stand-in; the device address is resolved once per device
// with hipGetSymbolAddress (with that device current) and only that address is ever handed to
// kernels.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two
// streams, two threads) race on it.  Nothing in the array needs to start at zero: the LoRA
// preparation writes every byte the epilogues later read (x.A and B^T zero-padded to the padded
// rank), and the product is written in full before it is read, all on the call's own stream.
#include <hip/hip_runtime.h>

#include <mutex>

#include "mlxq_common.h"

namespace mlxq {
namespace {

__device__ __align__(256) unsigned char scratch[MLXQ_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's `scratch`, resolved on the first call per device.
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return set_error(MLXQ_EDEVICE, "linear_noalloc: no current device");
  if (dev >= kMaxDevices)
    return set_error(MLXQ_EUNSUPPORTED, "linear_noalloc: device %d beyond the %d supported", dev,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(MLXQ_EDEVICE, "linear_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MLXQ_OK;
}

}  // namespace
}  // namespace mlxq

using namespace mlxq;

extern "C" int mlxq_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K,
                                   const uint32_t* wq, const void* scales, const void* biases,
                                   int sb_dtype, int64_t N, int group_size, int bits,
                                   const mlxq_epilogue* epilogue, void* y, void* stream) {
  const size_t need = mlxq_linear_workspace_size(x_dtype, sb_dtype, M, N, epilogue);
  if (need > (size_t)MLXQ_NOALLOC_SCRATCH_BYTES)
    return set_error(MLXQ_EINVAL,
                     "linear_noalloc: M=%lld N=%lld needs %zu bytes of scratch, more than the "
                     "%zu-byte static buffer (use mlxq_linear with a workspace)",
                     (long long)M, (long long)N, need, (size_t)MLXQ_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc != MLXQ_OK) return rc;
  }
  return mlxq_linear(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, epilogue,
                     y, ws, need, stream);
}
