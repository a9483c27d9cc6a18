// moeq_moe_forward_static: the layer forward for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  Its scratch memory is one file-scope
// device array per GPU, `scratch`, of MOEQ_STATIC_SCRATCH_BYTES, which the
// code object holds for as long as the process runs.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// the device address of each GPU's copy is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is
// handed to kernels.  Every call on one GPU shares its array; calls that
// overlap on one GPU (two streams, two threads) race.  The forward leaves no
// state in the array that a later call relies on: every buffer it reads is
// written earlier in the same call, so nothing needs clearing.
#include <mutex>

#include "common.h"

using namespace moeq;

namespace {

static_assert(MOEQ_STATIC_SCRATCH_BYTES % 256 == 0, "scratch size");

static __device__ __align__(256) unsigned char scratch[MOEQ_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void *g_scratch[kMaxDevices];
hipError_t g_status[kMaxDevices];

}  // namespace

extern "C" int moeq_moe_forward_static(const moeq_moe *m, const void *x, int64_t T, void *out,
                                       int out_dtype, void *logits_out, void *stream) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MOEQ_ERR_HIP, "moe_forward_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MOEQ_ERR_UNSUPPORTED, "moe_forward_static: device %d (at most %d devices)", dev, kMaxDevices);
  // once per device, with that device current: the address of its copy
  std::call_once(g_once[dev], [dev] {
    g_status[dev] = hipGetSymbolAddress(&g_scratch[dev], HIP_SYMBOL(scratch));
  });
  if (g_status[dev] != hipSuccess || !g_scratch[dev])
    return fail(MOEQ_ERR_HIP, "moe_forward_static: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(g_status[dev]));
  if (m && T > 0) {
    const size_t need = moeq_moe_workspace_size(m, T);
    if (need > size_t(MOEQ_STATIC_SCRATCH_BYTES))
      return fail(MOEQ_ERR_WORKSPACE,
                  "moe_forward_static: T=%lld needs %zu bytes of scratch, more than the %zu-byte static array "
                  "(use moeq_moe_forward with a workspace)",
                  (long long)T, need, size_t(MOEQ_STATIC_SCRATCH_BYTES));
  }
  return moeq_moe_forward(m, x, T, out, out_dtype, logits_out, g_scratch[dev], MOEQ_STATIC_SCRATCH_BYTES, stream);
}
