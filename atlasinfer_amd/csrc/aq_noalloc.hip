// aq_noalloc.hip -- aq_qlinear without a caller workspace: the split-K
// partial sums live in a static device array owned by the library.
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): the same
// kernels as aq_qlinear, with `scratch` below in place of the workspace
// argument.  The array is a file-scope __device__ variable, so every GPU the
// library runs on holds its own copy, at its own address, from the moment the
// code object loads until the process ends; the address is looked up once per
// device (hipGetSymbolAddress with that device current) and only that
// address is ever handed to a kernel.  The split-K planner bounds the split
// by the scratch size, exactly as it bounds it by a caller's workspace, so
// no call needs more than kScratchBytes.  Each split part writes every
// element of its partial-sum slice before the reduce kernel reads it, so
// nothing has to start at zero.  All calls on one GPU share its array: calls
// that overlap in time on one GPU (two streams, two host threads) race.
#include <mutex>

#include "aq_common.h"

namespace {

constexpr int64_t kScratchBytes = AQ_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::once_flag g_once[kMaxDevices];
void* g_addr[kMaxDevices];
hipError_t g_err[kMaxDevices];

// Device address of `scratch` on the current device (first call per device
// looks it up); nullptr with the HIP error in *err on failure.
void* scratch_on_current_device(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::call_once(g_once[dev], [dev]() {
    void* p = nullptr;
    g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_addr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
  });
  *err = g_err[dev];
  return g_addr[dev];
}

}  // namespace

extern "C" int aq_qlinear_noalloc(const void* x, int64_t M, int64_t K, int64_t N, const void* codes,
                                  const void* scales, int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols,
                                  const void* vals, const int32_t* tile_ptr, const uint32_t* tile_ent,
                                  int64_t tile_max, const void* bias, void* y, void* stream) {
  hipError_t e = hipSuccess;
  void* ws = scratch_on_current_device(&e);
  if (ws == nullptr) return aq::check_hip(e == hipSuccess ? hipErrorUnknown : e, "aq_qlinear_noalloc: scratch address");
  // the planner never asks for more than it is given: the split is bounded
  // by kScratchBytes (aq_qlinear_grouped's workspace rule)
  return aq_qlinear(x, M, K, N, codes, scales, G, fmt, row_ptr, cols, vals, tile_ptr, tile_ent, tile_max, bias, y, ws,
                    kScratchBytes, stream);
}
