// sdm_plan_bf16.hip -- plan_kernel instantiated for bf16 address inputs (the kernel is in sdm_plan.h).
#include "sdm_plan.h"

namespace sdmrt {

int launch_plan_bf16(const Plan& p, const PlanArgs& a, hipStream_t st, bool pick) {
  return by_half<PlanLaunch, bf16_t>(p.half, p, a, st, pick);
}

}  // namespace sdmrt
