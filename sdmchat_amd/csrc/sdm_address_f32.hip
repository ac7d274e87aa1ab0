// sdm_address_f32.hip -- the addressing kernels of sdm_address.h instantiated for f32 addresses.
#include "sdm_address.h"

namespace sdmrt {

int launch_address_f32(const Plan& p, const AddrArgs& a, hipStream_t st) {
  return by_half<AddressLaunch, float>(p.half, p, a, st);
}

}  // namespace sdmrt
