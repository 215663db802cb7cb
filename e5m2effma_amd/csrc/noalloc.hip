// noalloc.hip -- e5ma_gemm_noalloc: e5ma_gemm_ex (include/e5m2effma_ext.h) with the library's own fixed
// per-device scratch in place of a caller workspace, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
// in the reference.  Nothing here allocates: the scratch is a file-scope device array, reserved on each
// device when the library's code object loads there and held until the process ends.
//
// Its only user is split-K: FP32 partials, every element written by the split kernels before the
// reduce kernel reads it, so nothing in it has to start at zero.  Every call on a device shares that
// device's array and leaves its last contents there: two calls whose work overlaps on one device
// (different streams, no ordering between them) race on it.
#include <mutex>

#include "e5m2effma_ext.h"
#include "e5ma_host.hpp"

namespace e5ma {
namespace {

// The most split-K workspace any GEMM asks for (kMaxWorkspace = 64 MiB), so the scratch serves every
// split e5ma_gemm_ex would choose with a full workspace.
constexpr size_t kScratchBytes = kMaxWorkspace;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

// The device address of each device's copy of scratch, looked up once per device with that device
// current.  In host code the name `scratch` is only a stand-in for the symbol; it is never passed to a
// kernel or a copy.
struct ScratchSlot {
  std::once_flag once;
  void *ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

Workspace device_scratch(int dev, Call &call) {
  ScratchSlot &slot = g_scratch[dev];
  std::call_once(slot.once, [&slot] {
    void *p = nullptr;
    slot.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (slot.err == hipSuccess) slot.ptr = p;
    else (void)hipGetLastError();
  });
  if (call.hip(slot.err, "e5ma_gemm_noalloc: hipGetSymbolAddress of the scratch")) return Workspace{};
  call.need(slot.ptr != nullptr, E5MA_HIP_ERROR, "e5ma_gemm_noalloc: the scratch of device %d has no address", dev);
  return call.ok() ? Workspace{slot.ptr, kScratchBytes} : Workspace{};
}

}  // namespace
}  // namespace e5ma

extern "C" e5ma_status e5ma_gemm_noalloc(e5ma_op transa, e5ma_op transb, int m, int n, int k, float alpha,
                                         const e5ma_tensor *A, int lda, const e5ma_tensor *B, int ldb, float beta,
                                         const e5ma_tensor *C, int ldc, const e5ma_tensor *D, int ldd,
                                         const e5ma_tensor *bias, hipStream_t stream) {
  e5ma::WorkspaceSource src;
  src.per_device = e5ma::device_scratch;
  return e5ma::gemm_entry("e5ma_gemm_noalloc", transa, transb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, D, ldd,
                          bias, src, stream);
}
