// rk_abi.hip -- library-wide C ABI entry points: status strings, ABI
// version and the per-device compute-unit cache used by the split planner.
#include <hip/hip_runtime.h>
#include <string.h>

#include "rk_host.h"
#include "rotatek_hip.h"

namespace rk {

int current_device_cus(int* device_out) {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (device_out) *device_out = dev;
  if (dev < 64 && cache[dev] > 0) return cache[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cache[dev] = cus;
  return cus;
}

bool device_has_coherent_tickets() {
  static int cache[64] = {0};  // 0 unknown, 1 yes, 2 no
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return false;
  if (dev < 64 && cache[dev] != 0) return cache[dev] == 1;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return false;
  const bool ok = strncmp(prop.gcnArchName, "gfx942", 6) == 0 || strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  if (dev < 64) cache[dev] = ok ? 1 : 2;
  return ok;
}

}  // namespace rk

extern "C" const char* rk_strerror(int status) {
  switch (status) {
    case RK_OK: return "success";
    case RK_ERR_NULL: return "a required tensor or pointer is NULL";
    case RK_ERR_RANK: return "tensor has the wrong number of dimensions";
    case RK_ERR_DTYPE: return "unsupported or mismatched dtype";
    case RK_ERR_SHAPE: return "tensor shapes disagree";
    case RK_ERR_HEADS: return "H_q / num_kv_groups does not equal H_kv";
    case RK_ERR_HEAD_DIM: return "head_dim must be 1..128";
    case RK_ERR_KEEP_DIM: return "kept channels out of range (decode 0..head_dim, prefill 1..head_dim)";
    case RK_ERR_STRIDE: return "negative or overflowing stride";
    case RK_ERR_WORKSPACE: return "workspace is NULL, misaligned (256 B) or too small";
    case RK_ERR_ARG: return "invalid argument";
    case RK_ERR_HIP: return "HIP runtime error";
    case RK_ERR_NO_DEVICE: return "no HIP device available";
    case RK_ERR_SCRATCH: return "workspace needed exceeds the allocation-free scratch (RK_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

extern "C" int rk_abi_version(void) { return RK_ABI_VERSION; }

extern "C" int rk_device_cu_count(int device, int* status) {
  int cus = 0;
  const hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (status) *status = (e == hipSuccess) ? RK_OK : RK_ERR_NO_DEVICE;
  return e == hipSuccess ? cus : 0;
}
