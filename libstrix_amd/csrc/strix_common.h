// SPDX-License-Identifier: MIT
// gfx950 (CDNA4, MI355X) device contract for every libstrix_amd kernel.
//
// Replaces the gfx1151 wave32/WMMA header of the reference
// (csrc/strix_common.h:1-229): wave64, MFMA fragment types, bf16/fp8 value
// helpers and the error plumbing of the C ABI.
//
// MFMA fragment convention used by all kernels (pinned on the GPU by
// strix_probe_mfma_* and tests/test_gpu_mfma_layout.py):
//
//   16x16 f32/i32 result (4 VGPRs per lane):
//       lane l holds D[row = 4*(l/16) + i][col = l%16], i = 0..3.
//   A operand (16 x K): lane l supplies row l%16; B operand (K x 16): lane l
//   supplies column l%16. The K values a lane supplies are indexed by
//   (l/16, element). A and B use the same (l/16, element) -> k assignment, so
//   any fixed permutation of K inside one instruction gives the same sum;
//   kernels pick the permutation that makes their loads contiguous:
//       8-bit, 16x16x128 (fp8):  32 bytes/lane = two 16-byte halves,
//                                 half h covers k = 64h + 16*(l/16) + [0,16)
//       8-bit, 16x16x64  (i8):   16 bytes/lane,  k = 16*(l/16) + [0,16)
//       16-bit, 16x16x32 (bf16/f16): 8 values/lane, k = 8*(l/16) + [0,8)
//
// In every GEMM the weight rows (N) are the MFMA rows and the activation
// rows (tokens, M) are the MFMA columns, so a lane's four results are four
// consecutive weight rows of one token.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace strix {

constexpr int kWave = 64;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ MFMA
// e4m3 x e4m3 -> f32, 16x16x128 (format code 0 for both operands, no
// per-block exponent scale: the zero scale operands select the unscaled form).
__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// i8 x i8 -> i32, 16x16x64.
__device__ __forceinline__ v4i mfma_i8(const v4i& a, const v4i& b, const v4i& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// bf16 x bf16 -> f32, 16x16x32.
__device__ __forceinline__ v4f mfma_bf16(const bf16x8& a, const bf16x8& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// f16 x f16 -> f32, 16x16x32.
__device__ __forceinline__ v4f mfma_f16(const f16x8& a, const f16x8& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ values
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even: gfx950's v_cvt_pk_bf16_f32
// (pinned equal to torch's cast by the converter probe test).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Activation element loads: 16-bit storage, bf16 (IS_F16=false) or fp16.
template <bool IS_F16>
__device__ __forceinline__ float act_to_f32(uint32_t bits16) {
  if constexpr (IS_F16) return f16_bits_to_f32(bits16);
  else return bf16_bits_to_f32(bits16);
}
template <bool IS_F16>
__device__ __forceinline__ uint32_t f32_to_act_bits(float x) {
  if constexpr (IS_F16) return f32_to_f16_bits(x);
  else return f32_to_bf16_bits(x);
}

// Two e4m3fn bytes (bytes 0,1 of d when WORD_HI is false, else 2,3) -> fp32
// with gfx950's v_cvt_pk_f32_fp8 (pinned against every code by the probe test).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <bool WORD_HI>
__device__ __forceinline__ f32x2_t e4m3x2_to_f32(uint32_t d) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)d, WORD_HI);
}

// OCP e4m3fn byte -> fp32, exact (bias 7, no infinities, S.1111.111 = NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24;
  const uint32_t em = b & 0x7fu;
  if (em == 0x7fu) return __uint_as_float(0x7fc00000u | s);
  if (em < 8u) {  // subnormal: m * 2^-9
    return __uint_as_float(s | __float_as_uint((float)em * 0.001953125f));
  }
  return __uint_as_float(s | ((em + (120u << 3)) << 20));
}

// Two fp32 -> two e4m3 bytes (round to nearest even), written into the low
// (WORD_HI=false) or high half of `old`. gfx950's converter is OCP e4m3fn.
template <bool WORD_HI>
__device__ __forceinline__ int cvt_pk_e4m3(float a, float b, int old) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, WORD_HI);
}

// ------------------------------------------------------------------ waves
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) x = fmaxf(x, __shfl_xor(x, s, kWave));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) x += __shfl_xor(x, s, kWave);
  return x;
}

// Direct global -> LDS copy of 16 bytes per lane (gfx950 global_load_lds_dwordx4):
// lane l's 16 bytes land at lds_base + 16*l. lds_base must be wave-uniform.
__device__ __forceinline__ void g2l_b128(const void* gptr, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}
// 4 bytes per lane: lane l's word lands at lds_base + 4*l.
__device__ __forceinline__ void g2l_b32(const void* gptr, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)lds_base, 4, 0, 0);
}
// Wait until every global->LDS copy this wave issued has landed.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier for LDS hand-offs that leaves global->LDS copies in
// flight. __syncthreads() carries a release fence, for which the compiler
// waits on every outstanding vector memory operation (vmcnt(0)), draining a
// multi-stage copy pipeline at each barrier. Here the caller waits for the
// copies it needs with an explicit vmcnt; the barrier only orders this wave's
// LDS reads (lgkmcnt(0)) and, through the memory clobber, keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ------------------------------------------------------------------ activations
enum Act : int { kActSilu = 0, kActGeluTanh = 1 };

// SiLU(g) = g / (1 + e^-g).
__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }
// GELU, tanh form: 0.5 g (1 + tanh(z)), z = sqrt(2/pi) (g + 0.044715 g^3);
// tanh(z) = 1 - 2 / (e^{2z} + 1), which saturates cleanly at both ends.
__device__ __forceinline__ float gelu_tanh_f(float g) {
  const float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
  const float t = 1.0f - 2.0f / (__expf(2.0f * z) + 1.0f);
  return 0.5f * g * (1.0f + t);
}
template <int ACT>
__device__ __forceinline__ float gate_act(float g) {
  if constexpr (ACT == kActGeluTanh) return gelu_tanh_f(g);
  else return silu_f(g);
}

}  // namespace strix
