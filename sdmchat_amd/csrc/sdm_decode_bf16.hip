// sdm_decode_bf16.hip -- the single-launch decode step (decode_fused_kernel) for bfloat16 projections.
#include "sdm_decode.h"

namespace sdmrt {

int launch_decode_fused_bf16(const Plan& p, const DecodeArgs& a, hipStream_t st) {
  return by_half<DecodeFusedLaunch, bf16_t>(p.half, p, a, st);
}

}  // namespace sdmrt
