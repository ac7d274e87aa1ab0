// sdm_noalloc.hip -- sdm_rt_forward_noalloc: sdm_rt_forward on a fixed scratch array of the library instead of a
// caller's workspace, for callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops).  It runs the same kernels as sdm_rt_forward.
#include <mutex>

#include "sdm_common.h"

namespace sdmrt {

// the forward's workspace (plans, their sizes, the progress counters and partial sums of the out-norm exchange):
// 128 MiB per device, enough for B * T = 16,384 positions of 12 heads at M = 1,024 and k = 8
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(128) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];   // the array's device address on each device (set on first use there)
static std::mutex g_scratch_mu;

// the current device's copy of the scratch array (its address looked up once per device, that device current)
int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_err(SDM_RT_ELAUNCH, "no current HIP device");
  if (dev < 0 || dev >= kMaxDevices) return set_err(SDM_RT_EUNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_err(SDM_RT_ELAUNCH, "cannot find the scratch array on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SDM_RT_OK;
}

}  // namespace sdmrt

using namespace sdmrt;

extern "C" {

size_t sdm_rt_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int sdm_rt_forward_noalloc(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz,
                           int64_t kz_row_stride, const void* qz, int64_t qz_row_stride, const void* v,
                           int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                           sdm_rt_dtype in_dtype, const uint8_t* reset, void* r_out, int64_t out_row_stride,
                           sdm_rt_dtype out_dtype, const float* state_in_mem, const float* state_in_cnt,
                           float* state_out_mem, float* state_out_cnt, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  if (p.total > kNoAllocScratchBytes)
    return set_err(SDM_RT_ENOSPACE,
                   "sdm_rt_forward_noalloc: the call needs %zu bytes of scratch, above its fixed %zu; use "
                   "sdm_rt_forward with a workspace", p.total, kNoAllocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_ptr(&ws))) return rc;
  return sdm_rt_forward(dims, params, kz, kz_row_stride, qz, qz_row_stride, v, v_row_stride, gate_logits,
                        gate_row_stride, in_dtype, reset, r_out, out_row_stride, out_dtype, state_in_mem,
                        state_in_cnt, state_out_mem, state_out_cnt, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
