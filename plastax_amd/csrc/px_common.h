// px_common.h -- pieces shared by the library's translation units: the
// per-thread error text behind plx_last_error() and the device Philox.
#pragma once

#ifndef __HIPCC_RTC__  // (hipRTC compiles of site programs bring their own runtime header)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

struct plx_forward_desc;

namespace plx_detail {
extern thread_local std::string g_last_error;
int fail(int code, const char* what);
int check_launch(const char* what);
// plx_forward_bucket's checks of d and its launch: *grid workgroups (0: no
// rows, nothing to launch) of *block lanes.
int forward_launch_shape(const plx_forward_desc* d, const char* who, unsigned* grid, unsigned* block);
}  // namespace plx_detail
#endif

namespace px {

// First word of Philox-4x32-10 in the plastax mapping (rng.py:109-141): the
// counter block is (ctr_lo, ctr_hi, seed_lo, seed_hi), the key (seed_lo,
// seed_hi); ten rounds with the Salmon et al. (SC'11) multipliers and Weyl
// increments.
__device__ __forceinline__ uint32_t philox32(uint64_t seed, uint64_t counter) {
  uint32_t x0 = static_cast<uint32_t>(counter), x1 = static_cast<uint32_t>(counter >> 32);
  uint32_t x2 = static_cast<uint32_t>(seed), x3 = static_cast<uint32_t>(seed >> 32);
  uint32_t k0 = x2, k1 = x3;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * x0, hi0 = __umulhi(0xD2511F53u, x0);
    const uint32_t lo1 = 0xCD9E8D57u * x2, hi1 = __umulhi(0xCD9E8D57u, x2);
    const uint32_t n0 = hi1 ^ x1 ^ k0, n2 = hi0 ^ x3 ^ k1;
    x0 = n0;
    x1 = lo1;
    x2 = n2;
    x3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return x0;
}

}  // namespace px
