// Host-side declarations shared between the runtime (runtime.cpp) and the
// kernel translation units. Not part of the public C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "th_device.h"

namespace th {

// Operation applied to every coefficient as an NTT loads it (fused producer
// of the transform's input; the result is what gets transformed):
//   NONE     x = src[i]
//   MUL      x = src[i] * aux[i] mod q                    (ct x pt, ciphertext.rs:422-429)
//   RESCALE  x = (src[i] - (aux[i] mod q)) * q_last^{-1} mod q, aux = coefficient-domain
//            last limb of the same component             (rescale, ciphertext.rs:505-522)
//   DOT      x = src[i] + aux[i] * key[i] mod q, src = c0, aux = c1, key = s
//                                                         (decrypt, ciphertext.rs:332-341)
enum NttLoad : uint32_t { NTT_LOAD_NONE = 0, NTT_LOAD_MUL = 1, NTT_LOAD_RESCALE = 2, NTT_LOAD_DOT = 3 };

// One limb-polynomial transform. In strided mode job i reads src + i*stride,
// writes dst + i*stride and uses limb limb_base + i % limb_mod.
struct NttJob {
  const uint64_t* src;
  uint64_t* dst;
  const uint64_t* aux;  // second operand of the load operation (null for NONE)
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
  uint32_t load;              // NttLoad (explicit job lists only)
  uint32_t pad_;
  const BarrettConst* bc;     // per limb (MUL, DOT)
  const RescaleConst* rc;     // per output limb at the input's level (RESCALE)
  const uint64_t* key;        // secret key, L x N (DOT)
};

// Launch njobs forward (inverse=false) or inverse negacyclic NTTs of size 2^logn.
hipError_t launch_ntt(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s);
// Supported transform sizes.
constexpr int NTT_MIN_LOGN = 10;
constexpr int NTT_MAX_LOGN = 15;

}  // namespace th
