// sdm_address_bf16.hip -- the addressing kernels of sdm_address.h instantiated for bf16 addresses.
#include "sdm_address.h"

namespace sdmrt {

int launch_address_bf16(const Plan& p, const AddrArgs& a, hipStream_t st) {
  return by_half<AddressLaunch, bf16_t>(p.half, p, a, st);
}

}  // namespace sdmrt
