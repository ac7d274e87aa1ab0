// sdm_pick_bf16.hip -- pick_scan_kernel instantiated for bf16 values (the kernel is in sdm_pick.h).
#include "sdm_pick.h"

namespace sdmrt {

int launch_pick_scan_bf16(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st) {
  return out_dtype == SDM_RT_BF16 ? launch_pick_scan_t<bf16_t, bf16_t>(p, a, st) : launch_pick_scan_t<bf16_t, float>(p, a, st);
}

}  // namespace sdmrt
