// sdm_scan_bf16.hip -- scan_kernel instantiated for bf16 values (the kernel is in sdm_scan.h).
#include "sdm_scan.h"

namespace sdmrt {

int launch_scan_bf16(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st) {
  return out_dtype == SDM_RT_BF16 ? launch_scan_v<bf16_t, bf16_t>(p, a, st) : launch_scan_v<bf16_t, float>(p, a, st);
}

}  // namespace sdmrt
