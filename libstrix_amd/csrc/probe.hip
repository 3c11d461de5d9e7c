// SPDX-License-Identifier: MIT
// One-wave probes that pin the fragment conventions every kernel relies on
// (the gfx950 counterpart of the reference's _wmma_bf16_tile probe,
// csrc/testing/wmma_layout_test.hip:12-36, tests/test_wmma_layout.py).
//
// Each probe computes D[16][16] = A[16][K] . B[16][K]^T with the operand and
// result layouts declared in strix_common.h, so a wrong assumption about
// MFMA lanes shows up as a wrong matrix product. The global->LDS probe checks
// where global_load_lds_dwordx4 puts each lane's 16 bytes.
#include "capi_internal.h"
#include "strix_common.h"

namespace strix {
namespace {

__device__ __forceinline__ void store_tile(float* d, const v4f& acc) {
  const int l = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) d[(4 * (l >> 4) + i) * 16 + (l & 15)] = acc[i];
}

__global__ void __launch_bounds__(64) probe_bf16_kernel(const uint16_t* a, const uint16_t* b, float* d, int K) {
  const int l = threadIdx.x, r = l & 15, g = l >> 4;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += 32) {
    bf16x8 af, bf;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      af[j] = __builtin_bit_cast(__bf16, a[r * K + k0 + 8 * g + j]);
      bf[j] = __builtin_bit_cast(__bf16, b[r * K + k0 + 8 * g + j]);
    }
    acc = mfma_bf16(af, bf, acc);
  }
  store_tile(d, acc);
}

__global__ void __launch_bounds__(64) probe_fp8_kernel(const uint8_t* a, const uint8_t* b, float* d, int K) {
  const int l = threadIdx.x, r = l & 15, g = l >> 4;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += 128) {
    const u32x4* pa0 = reinterpret_cast<const u32x4*>(a + r * K + k0 + 16 * g);
    const u32x4* pa1 = reinterpret_cast<const u32x4*>(a + r * K + k0 + 64 + 16 * g);
    const u32x4* pb0 = reinterpret_cast<const u32x4*>(b + r * K + k0 + 16 * g);
    const u32x4* pb1 = reinterpret_cast<const u32x4*>(b + r * K + k0 + 64 + 16 * g);
    v8i af, bf;
    const u32x4 x0 = *pa0, x1 = *pa1, y0 = *pb0, y1 = *pb1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      af[j] = x0[j]; af[4 + j] = x1[j];
      bf[j] = y0[j]; bf[4 + j] = y1[j];
    }
    acc = mfma_fp8(af, bf, acc);
  }
  store_tile(d, acc);
}

__global__ void __launch_bounds__(64) probe_i8_kernel(const int8_t* a, const int8_t* b, int* d, int K) {
  const int l = threadIdx.x, r = l & 15, g = l >> 4;
  v4i acc = {0, 0, 0, 0};
  for (int k0 = 0; k0 < K; k0 += 64) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(a + r * K + k0 + 16 * g);
    const u32x4 y = *reinterpret_cast<const u32x4*>(b + r * K + k0 + 16 * g);
    v4i af, bf;
#pragma unroll
    for (int j = 0; j < 4; ++j) { af[j] = x[j]; bf[j] = y[j]; }
    acc = mfma_i8(af, bf, acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) d[(4 * (l >> 4) + i) * 16 + (l & 15)] = acc[i];
}

// Lane l copies source bytes [16*perm(l), +16) straight into LDS; the LDS
// image is then written out linearly. With perm(l) = 63 - l the output is the
// source with its 16-byte chunks reversed iff lane l lands at LDS byte 16*l.
__global__ void __launch_bounds__(64) probe_g2l_kernel(const uint8_t* src, uint8_t* dst) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[1024];
  const int l = threadIdx.x;
  g2l_b128(src + 16 * (63 - l), lds);
  wait_vmem();
  __syncthreads();
  *reinterpret_cast<u32x4*>(dst + 16 * l) = *reinterpret_cast<const u32x4*>(lds + 16 * l);
}

}  // namespace
}  // namespace strix

using namespace strix;

extern "C" {

int strix_probe_mfma(int kind, const void* a, const void* b, void* d, int64_t K, void* stream) {
  STRIX_REQUIRE(kind >= 0 && kind <= 2, "probe_mfma: kind 0 (bf16), 1 (e4m3) or 2 (int8)");
  const int step = kind == 0 ? 32 : (kind == 1 ? 128 : 64);
  STRIX_REQUIRE(K > 0 && K % step == 0, "probe_mfma: K must be a positive multiple of %d", step);
  STRIX_REQUIRE(aligned(a, 16) && aligned(b, 16), "probe_mfma: operands must be 16-byte aligned");
  STRIX_ARCH_GATE();
  hipStream_t st = as_stream(stream);
  if (kind == 0)
    hipLaunchKernelGGL(probe_bf16_kernel, dim3(1), dim3(64), 0, st, (const uint16_t*)a, (const uint16_t*)b,
                       (float*)d, (int)K);
  else if (kind == 1)
    hipLaunchKernelGGL(probe_fp8_kernel, dim3(1), dim3(64), 0, st, (const uint8_t*)a, (const uint8_t*)b,
                       (float*)d, (int)K);
  else
    hipLaunchKernelGGL(probe_i8_kernel, dim3(1), dim3(64), 0, st, (const int8_t*)a, (const int8_t*)b, (int*)d,
                       (int)K);
  return check_launch("probe_mfma");
}

int strix_probe_g2l(const uint8_t* src, uint8_t* dst, void* stream) {
  STRIX_REQUIRE(aligned(src, 16) && aligned(dst, 16), "probe_g2l: buffers must be 16-byte aligned");
  STRIX_ARCH_GATE();
  hipLaunchKernelGGL(probe_g2l_kernel, dim3(1), dim3(64), 0, as_stream(stream), src, dst);
  return check_launch("probe_g2l");
}

}  // extern "C"

// Conversion probes: what gfx950's converters produce, pinned against the
// format definitions by tests (they decide which decoders the GEMMs may use).
namespace strix {
namespace {

// out[s][b][j] (bf16 bits), j = 0,1: v_cvt_scalef32_pk_bf16_fp4 of byte b
// (placed in byte lane `sel` of the source dword) with scale scales[s].
// The pair is read as one 32-bit word: taking its elements one at a time
// (r[0], r[1]) compiled to code that returned the low element twice.
template <int SEL>
__device__ void cvt_fp4_one(uint32_t b, float sc, uint16_t* o) {
  const uint32_t r = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(b << (8 * SEL), sc, SEL));
  o[0] = (uint16_t)(r & 0xffffu);
  o[1] = (uint16_t)(r >> 16);
}
__global__ void probe_cvt_kernel(const float* scales, int nscales, uint16_t* fp4_out, float* fp8_out,
                                 uint16_t* bf16_out, const float* bf16_in, int nbf16) {
  const int b = threadIdx.x;  // 0..255
  for (int s = 0; s < nscales; ++s) {
    uint16_t* o = fp4_out + ((int64_t)s * 4 * 256 + b) * 2;
    cvt_fp4_one<0>(b, scales[s], o);
    cvt_fp4_one<1>(b, scales[s], o + 256 * 2);
    cvt_fp4_one<2>(b, scales[s], o + 2 * 256 * 2);
    cvt_fp4_one<3>(b, scales[s], o + 3 * 256 * 2);
  }
  // v_cvt_pk_f32_fp8 on the low word: byte b in byte 0 and 0x00 in byte 1.
  const f32x2_t f = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
  fp8_out[b] = f[0];
  for (int i = b; i < nbf16; i += 256) bf16_out[i] = __builtin_bit_cast(uint16_t, (__bf16)bf16_in[i]);
}
}  // namespace
}  // namespace strix

extern "C" int strix_probe_cvt(const float* scales, int64_t nscales, uint16_t* fp4_out, float* fp8_out,
                               uint16_t* bf16_out, const float* bf16_in, int64_t nbf16, void* stream) {
  STRIX_REQUIRE(nscales >= 1 && nscales <= 64, "probe_cvt: 1..64 scales");
  STRIX_ARCH_GATE();
  hipLaunchKernelGGL(strix::probe_cvt_kernel, dim3(1), dim3(256), 0, strix::as_stream(stream), scales, (int)nscales,
                     fp4_out, fp8_out, bf16_out, bf16_in, (int)nbf16);
  return strix::check_launch("probe_cvt");
}
