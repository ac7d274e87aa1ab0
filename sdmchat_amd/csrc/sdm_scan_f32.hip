// sdm_scan_f32.hip -- scan_kernel instantiated for f32 values (the kernel is in sdm_scan.h).
#include "sdm_scan.h"

namespace sdmrt {

int launch_scan_f32(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st) {
  return out_dtype == SDM_RT_BF16 ? launch_scan_v<float, bf16_t>(p, a, st) : launch_scan_v<float, float>(p, a, st);
}

}  // namespace sdmrt
