// sdm_plan_f32.hip -- plan_kernel instantiated for f32 address inputs (the kernel is in sdm_plan.h).
#include "sdm_plan.h"

namespace sdmrt {

int launch_plan_f32(const Plan& p, const PlanArgs& a, hipStream_t st, bool pick) {
  return by_half<PlanLaunch, float>(p.half, p, a, st, pick);
}

}  // namespace sdmrt
