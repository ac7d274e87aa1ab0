// sdm_decode_f32.hip -- the single-launch decode step (decode_fused_kernel) for float32 projections.
#include "sdm_decode.h"

namespace sdmrt {

int launch_decode_fused_f32(const Plan& p, const DecodeArgs& a, hipStream_t st) {
  return by_half<DecodeFusedLaunch, float>(p.half, p, a, st);
}

}  // namespace sdmrt
