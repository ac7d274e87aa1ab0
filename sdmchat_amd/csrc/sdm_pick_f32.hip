// sdm_pick_f32.hip -- pick_scan_kernel instantiated for f32 values (the kernel is in sdm_pick.h).
#include "sdm_pick.h"

namespace sdmrt {

int launch_pick_scan_f32(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st) {
  return out_dtype == SDM_RT_BF16 ? launch_pick_scan_t<float, bf16_t>(p, a, st) : launch_pick_scan_t<float, float>(p, a, st);
}

}  // namespace sdmrt
