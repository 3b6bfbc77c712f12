// Host-side declarations shared between the runtime (runtime.cpp) and the
// kernel translation units. Not part of the public C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "th_device.h"

namespace th {

// One limb-polynomial transform. In strided mode job i reads src + i*stride,
// writes dst + i*stride and uses limb limb_base + i % limb_mod.
struct NttJob {
  const uint64_t* src;
  uint64_t* dst;
  uint32_t limb;
  uint32_t pad_;
};

struct NttArgs {
  const LimbConst* lc;
  const NttJob* jobs;  // non-null: explicit job list
  const uint64_t* src;
  uint64_t* dst;
  uint64_t stride;
  uint32_t limb_mod;
  uint32_t limb_base;
};

// Launch njobs forward (inverse=false) or inverse negacyclic NTTs of size 2^logn.
hipError_t launch_ntt(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s);
// Dynamic LDS bytes the NTT kernel for 2^logn uses (for occupancy reports).
size_t ntt_lds_bytes(int logn);
// Supported transform sizes.
constexpr int NTT_MIN_LOGN = 10;
constexpr int NTT_MAX_LOGN = 15;

}  // namespace th
