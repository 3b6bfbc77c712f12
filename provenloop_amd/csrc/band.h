// The sampler's boundary-band test, shared by the device sampler
// (sample_device.h) and the host check of its arithmetic (host_math_check.cpp).
#pragma once

namespace th {

// Where a Gaussian sample's rounding could depend on the math library:
// t = z * 3.19 within `band` of a rounding boundary k + 1/2, or |t| >= 2^52,
// or not finite. The device's log/cos differ from glibc's (which the
// reference calls through Rust std) by a few ulps, so |t_device - t_glibc|
// stays below about 2^-45 (|z| < 8.7, |t| < 28); with the default band of
// 2^-36 (bands are at least 2^-40) every sample whose rounded value could
// differ from glibc's is flagged, and the host redraws it with glibc.
// t - floor(t) and its difference from 1/2 are exact for |t| < 2^52. A
// constexpr function, so host and device code call the same definition.
constexpr bool near_rounding_boundary(double t, double band) {
  if (!(__builtin_fabs(t) < 0x1p52)) return true;
  return __builtin_fabs((t - __builtin_floor(t)) - 0.5) < band;
}

}  // namespace th
