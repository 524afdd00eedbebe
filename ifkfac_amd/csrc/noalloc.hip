// ifk_precondition_apply_bf16_noalloc: the per-step apply of the four solves
// with its scratch in a device array of this library instead of a
// caller-supplied workspace, for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).  No counterpart in the reference.
//
// The scratch is the file-scope array `scratch` below.  On the host its name
// is only a stand-in for the symbol: its device address, which differs per
// GPU, comes from hipGetSymbolAddress on the first call on each device (with
// that device current) and is kept per device; only that address ever goes
// into a kernel argument.  Every call on one GPU shares the array, so calls
// that overlap on one GPU (on different streams, or from different threads)
// race.  Nothing in the array has to start at zero: the apply writes each
// intermediate before reading it.  Its four products each have a triangular
// operand, so the GEMM dispatcher keeps them on this library's kernels
// (hipBLASLt, which allocates when it makes a handle, takes only plain
// products).
#include "../../include/ifkfac_hip.h"

#include <mutex>

#include "common.h"
#include "linalg.h"

namespace ifk {

constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;   // 64 MiB per GPU
constexpr int NOALLOC_MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_dev[NOALLOC_MAX_DEVICES];

// Device address of `scratch` on the current device (which must be the
// stream's), looked up once per device.
static int scratch_address(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    set_error("precondition_apply_bf16_noalloc: no usable current device");
    return IFK_ERR_HIP;
  }
  if (s != nullptr) {
    int sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || sdev != dev) {
      set_error("precondition_apply_bf16_noalloc: the stream's device is not the current device");
      return IFK_ERR_INVALID;
    }
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      set_error("precondition_apply_bf16_noalloc: hipGetSymbolAddress of the scratch array failed");
      return IFK_ERR_HIP;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return IFK_OK;
}

}  // namespace ifk

using namespace ifk;

extern "C" {

int ifk_precondition_apply_bf16_noalloc(void* stream, const float* grad, int64_t n_out,
                                        int64_t n_in, int64_t ldg, const void* Z_Xb,
                                        const void* Z_Xt, int64_t ldzx, const void* Z_Gb,
                                        const void* Z_Gt, int64_t ldzg, float* nat, int64_t ldn) {
  if (n_out < 1 || n_in < 1) {
    set_error("precondition_apply_bf16_noalloc: invalid arguments");
    return IFK_ERR_INVALID;
  }
  if (n_out > ((int64_t)1 << 24) || n_in > ((int64_t)1 << 24) ||
      precondition_apply_b_min_ws(n_out, n_in) > NOALLOC_SCRATCH_BYTES) {
    set_error("precondition_apply_bf16_noalloc: n_out x n_in too large for the 64 MiB scratch "
              "(three bf16 n_out x n_in buffers must fit: at most about 11.18 million "
              "elements; use ifk_precondition_apply_bf16)");
    return IFK_ERR_INVALID;
  }
  hipStream_t s = (hipStream_t)stream;
  void* ws = nullptr;
  int rc = scratch_address(s, &ws);
  if (rc != IFK_OK) return rc;
  return precondition_apply_b_fit(s, grad, n_out, n_in, ldg, (const bf16_t*)Z_Xb,
                                  (const bf16_t*)Z_Xt, ldzx, (const bf16_t*)Z_Gb,
                                  (const bf16_t*)Z_Gt, ldzg, nat, ldn, ws, NOALLOC_SCRATCH_BYTES);
}

}  // extern "C"
