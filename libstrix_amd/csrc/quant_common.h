// SPDX-License-Identifier: MIT
// Per-lane pieces of the activation quantizers, shared by the quantizer
// kernels and the fused router (which quantizes the tokens it routes).
#pragma once

#include "strix_common.h"

namespace strix {

template <bool F16>
__device__ __forceinline__ void load8(const uint16_t* p, float v[8]) {
  const u32x4 raw = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = act_to_f32<F16>(raw[i] & 0xffffu);
    v[2 * i + 1] = act_to_f32<F16>(raw[i] >> 16);
  }
}

// x / sc correctly rounded, as far as the e4m3 rounding that follows can
// tell. x * RN(1/sc) is within 1.5 ulp of x / sc, so both round to the same
// e4m3 value unless the product lies in e4m3's subnormal range or within 4
// ulp of an e4m3 rounding midpoint (low 20 mantissa bits near 0x80000); those
// elements, and groups whose scale is subnormal (1/sc would overflow), take
// the IEEE division. tests/test_e4m3_quotient.py checks the argument on the
// CPU for every 16-bit x against sampled group maxima.
__device__ __forceinline__ float div_for_e4m3(float x, float sc, float r, bool fast) {
  float q = x * r;
  const uint32_t b = __float_as_uint(q) & 0x7fffffffu;
  const int d = (int)(b & 0xfffffu) - 0x80000;
  if (!fast || b - 1u < (121u << 23) - 1u || (unsigned)(d + 4) <= 8u) q = __fdiv_rn(x, sc);
  return q;
}

__device__ __forceinline__ int q_i8(float x, float s) {
  float r = __builtin_rintf(__fdiv_rn(x, s));
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

// One lane's share of the 1x128 quantization of group g of row m: elements
// [16 sub, 16 sub + 16) of the group (8 lanes per group, aligned to 8 lanes
// of the wave). Every lane of the wave must call it, live or not: the group
// max is an 8-lane butterfly; lanes with live == false load and store
// nothing. FP8 selects e4m3 (s = max/448), otherwise int8 (s = max/127).
template <bool F16, bool FP8>
__device__ __forceinline__ void quant128_lane(const uint16_t* __restrict__ x, int64_t ldx, uint8_t* __restrict__ q,
                                              int64_t ldq, float* __restrict__ s, int64_t lds, uint32_t m,
                                              uint32_t g, int sub, bool live) {
  const int64_t k = (int64_t)g * 128 + sub * 16;
  float v[16];
  if (live) {
    const uint16_t* p = x + (int64_t)m * ldx + k;
    load8<F16>(p, v);
    load8<F16>(p + 8, v + 8);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.0f;
  }
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
  for (int o = 4; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  const float qmax = FP8 ? 448.0f : 127.0f;
  const float sc = mx > 0.0f ? __fdiv_rn(mx, qmax) : 1.0f;
  if (!live) return;
  if (sub == 0) s[(int64_t)m * lds + g] = sc;
  const bool fast = sc >= 0x1p-126f;
  const float rs = FP8 ? __fdiv_rn(1.0f, sc) : 0.0f;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float* u = v + 4 * j;
    if constexpr (FP8) {
      int r = 0;
      r = cvt_pk_e4m3<false>(div_for_e4m3(u[0], sc, rs, fast), div_for_e4m3(u[1], sc, rs, fast), r);
      r = cvt_pk_e4m3<true>(div_for_e4m3(u[2], sc, rs, fast), div_for_e4m3(u[3], sc, rs, fast), r);
      w[j] = (uint32_t)r;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[j] |= (uint32_t)(q_i8(u[i], sc) & 0xff) << (8 * i);
    }
  }
  uint2* out = reinterpret_cast<uint2*>(q + (int64_t)m * ldq + k);  // output rows are 8-byte aligned
  out[0] = make_uint2(w[0], w[1]);
  out[1] = make_uint2(w[2], w[3]);
}

}  // namespace strix
