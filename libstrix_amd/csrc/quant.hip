// SPDX-License-Identifier: MIT
// Activation quantizers in front of the 8-bit MFMA GEMMs.
//
//   int8 per token      s[m]    = max_k |x[m,k]| / 127   (1 if the row is 0)
//                       q[m,k]  = clamp(rint(x[m,k] / s[m]), -127, 127)
//   int8 per 128-group  s[m,g]  = max_{k in g} |x[m,k]| / 127 (1 if 0), same q
//                       (reference convention: csrc/gemm/w8a8_wmma_gemm.hip:15-21,
//                        tests/test_moe_w4a8.py:24-36)
//   e4m3 per 128-group  s[m,g]  = max_{k in g} |x[m,k]| / 448 (1 if 0)
//                       q[m,k]  = e4m3_rne(x[m,k] / s[m,g])
//
// The division is IEEE (correctly rounded), so the CPU oracle reproduces q
// bit for bit; the e4m3 quantizer gets the same bytes from a reciprocal
// product, with the division kept where the product could round
// differently. In the 128-group quantizers each lane owns 16 consecutive
// elements (two 16-byte loads); a group is 8 lanes, so the group max is an
// 8-lane butterfly (quant_common.h).
#include "capi_internal.h"
#include "quant_common.h"
#include "strix_common.h"

namespace strix {
namespace {

// One 256-thread block per row.
template <bool F16>
__global__ void __launch_bounds__(256)
    int8_quant_token_kernel(const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ q,
                            int64_t ldq, float* __restrict__ s, int K) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const uint16_t* xr = x + m * ldx;
  float mx = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    float v[8];
    load8<F16>(xr + k, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
  }
  mx = wave_max(mx);
  if (lane_id() == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = mx > 0.0f ? __fdiv_rn(mx, 127.0f) : 1.0f;
  if (threadIdx.x == 0) s[m] = sc;
  int8_t* qr = q + m * ldq;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    float v[8];
    load8<F16>(xr + k, v);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) lo |= (uint32_t)(q_i8(v[i], sc) & 0xff) << (8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) hi |= (uint32_t)(q_i8(v[4 + i], sc) & 0xff) << (8 * i);
    *reinterpret_cast<uint2*>(qr + k) = make_uint2(lo, hi);
  }
}

// 128-element groups. Thread t of the grid handles elements [16t, 16t+16) of
// the flattened [M, K] view (row-major by groups), 8 lanes per group: two
// 16-byte loads in flight per lane, and the group's (row, column) from one
// 32-bit division (the host bounds the group count below 2^28).
// FP8 selects the e4m3 quantizer, otherwise int8.
template <bool F16, bool FP8>
__global__ void __launch_bounds__(256)
    quant_group128_kernel(const uint16_t* __restrict__ x, int64_t ldx, uint8_t* __restrict__ q,
                          int64_t ldq, float* __restrict__ s, int64_t lds, uint32_t groups_per_row,
                          uint32_t total_groups) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const uint32_t grp = t >> 3;
  const int sub = (int)(t & 7u);
  const bool live = grp < total_groups;
  const uint32_t m = live ? grp / groups_per_row : 0u;
  const uint32_t g = live ? grp - m * groups_per_row : 0u;
  quant128_lane<F16, FP8>(x, ldx, q, ldq, s, lds, m, g, sub, live);
}

template <bool F16>
__global__ void __launch_bounds__(256)
    int8_dequant_group128_kernel(const int8_t* __restrict__ q, int64_t ldq, const float* __restrict__ s,
                                 int64_t lds, uint16_t* __restrict__ out, int64_t ldo, int chunks_per_row,
                                 int64_t total_chunks) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= total_chunks) return;
  const int64_t m = t / chunks_per_row;
  const int64_t k = (t % chunks_per_row) * 8;
  const uint2 raw = *reinterpret_cast<const uint2*>(q + m * ldq + k);
  const float sc = s[m * lds + k / 128];
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = i < 2 ? raw.x : raw.y;
    const float a = (float)(int8_t)((w >> (16 * (i & 1))) & 0xffu) * sc;
    const float b = (float)(int8_t)((w >> (16 * (i & 1) + 8)) & 0xffu) * sc;
    o[i] = F16 ? (f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16)) : pack_bf16x2(a, b);
  }
  *reinterpret_cast<u32x4*>(out + m * ldo + k) = u32x4{o[0], o[1], o[2], o[3]};
}

int check_act(const char* op, const void* x, int x_dtype, int64_t ldx, const void* q, int64_t ldq,
              int64_t M, int64_t K) {
  STRIX_REQUIRE(x_dtype == STRIX_BF16 || x_dtype == STRIX_F16,
                "%s: activation must be float16 or bfloat16", op);
  STRIX_REQUIRE(M >= 0 && K >= 0, "%s: negative size", op);
  STRIX_REQUIRE(K % 8 == 0, "%s: K must be a multiple of 8, got K=%lld", op, (long long)K);
  STRIX_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: activation row stride must be >= K and a multiple of 8",
                op);
  STRIX_REQUIRE(ldq >= K && ldq % 8 == 0, "%s: output row stride must be >= K and a multiple of 8", op);
  STRIX_REQUIRE(M == 0 || (aligned(x, 16) && aligned(q, 8)),
                "%s: activation must be 16-byte aligned and output 8-byte aligned", op);
  STRIX_REQUIRE(M <= INT32_MAX && K <= INT32_MAX, "%s: sizes overflow 32-bit indexing", op);
  return STRIX_OK;
}

}  // namespace
}  // namespace strix

using namespace strix;

extern "C" {

int strix_int8_quant_per_token(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                               float* s, int64_t M, int64_t K, void* stream) {
  int rc = check_act("int8_quant_per_token", x, x_dtype, ldx, q, ldq, M, K);
  if (rc) return rc;
  if (M == 0) return STRIX_OK;
  STRIX_REQUIRE(K > 0, "int8_quant_per_token: K must be positive");
  STRIX_ARCH_GATE();
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (x_dtype == STRIX_F16)
    hipLaunchKernelGGL(int8_quant_token_kernel<true>, dim3((unsigned)M), dim3(256), 0,
                       as_stream(stream), xp, ldx, q, ldq, s, (int)K);
  else
    hipLaunchKernelGGL(int8_quant_token_kernel<false>, dim3((unsigned)M), dim3(256), 0,
                       as_stream(stream), xp, ldx, q, ldq, s, (int)K);
  return check_launch("int8_quant_per_token");
}

static int quant_group128(const char* op, bool fp8, const void* x, int x_dtype, int64_t ldx,
                          void* q, int64_t ldq, float* s, int64_t lds, int64_t M, int64_t K,
                          void* stream) {
  int rc = check_act(op, x, x_dtype, ldx, q, ldq, M, K);
  if (rc) return rc;
  STRIX_REQUIRE(K % 128 == 0, "%s: K must be a multiple of 128, got K=%lld", op, (long long)K);
  STRIX_REQUIRE(lds >= K / 128, "%s: scale row stride must be >= K/128", op);
  if (M == 0 || K == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  const int64_t groups = M * (K / 128);
  STRIX_REQUIRE(groups < (int64_t(1) << 28), "%s: %lld groups of 128 exceed the 2^28 limit", op,
                (long long)groups);
  const int64_t threads = groups * 8;
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  uint8_t* qp = static_cast<uint8_t*>(q);
  const uint32_t gpr = (uint32_t)(K / 128);
  const uint32_t ngroups = (uint32_t)groups;
  hipStream_t st = as_stream(stream);
  if (fp8) {
    if (x_dtype == STRIX_F16)
      hipLaunchKernelGGL((quant_group128_kernel<true, true>), dim3(blocks), dim3(256), 0, st, xp,
                         ldx, qp, ldq, s, lds, gpr, ngroups);
    else
      hipLaunchKernelGGL((quant_group128_kernel<false, true>), dim3(blocks), dim3(256), 0, st, xp,
                         ldx, qp, ldq, s, lds, gpr, ngroups);
  } else {
    if (x_dtype == STRIX_F16)
      hipLaunchKernelGGL((quant_group128_kernel<true, false>), dim3(blocks), dim3(256), 0, st, xp,
                         ldx, qp, ldq, s, lds, gpr, ngroups);
    else
      hipLaunchKernelGGL((quant_group128_kernel<false, false>), dim3(blocks), dim3(256), 0, st, xp,
                         ldx, qp, ldq, s, lds, gpr, ngroups);
  }
  return check_launch(op);
}

int strix_int8_quant_group128(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                              float* s, int64_t lds, int64_t M, int64_t K, void* stream) {
  return quant_group128("int8_quant_group128", false, x, x_dtype, ldx, q, ldq, s, lds, M, K,
                        stream);
}

int strix_int8_dequant_group128(const int8_t* q, int64_t ldq, const float* s, int64_t lds, void* out,
                                int out_dtype, int64_t ldo, int64_t M, int64_t K, void* stream) {
  const char* op = "int8_dequant_group128";
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(M >= 0 && K >= 0 && K % 128 == 0, "%s: K must be a non-negative multiple of 128", op);
  STRIX_REQUIRE(ldq >= K && ldq % 8 == 0 && ldo >= K && ldo % 8 == 0, "%s: row strides must be >= K, multiples of 8", op);
  STRIX_REQUIRE(lds >= K / 128, "%s: scale row stride must be >= K/128", op);
  STRIX_REQUIRE(M == 0 || (aligned(q, 8) && aligned(out, 16)), "%s: q must be 8-byte and out 16-byte aligned", op);
  if (M == 0 || K == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  const int cpr = (int)(K / 8);
  const int64_t total = M * cpr;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (out_dtype == STRIX_F16)
    hipLaunchKernelGGL(int8_dequant_group128_kernel<true>, dim3(blocks), dim3(256), 0, as_stream(stream), q, ldq,
                       s, lds, o, ldo, cpr, total);
  else
    hipLaunchKernelGGL(int8_dequant_group128_kernel<false>, dim3(blocks), dim3(256), 0, as_stream(stream), q, ldq,
                       s, lds, o, ldo, cpr, total);
  return check_launch(op);
}

int strix_fp8_quant_group128(const void* x, int x_dtype, int64_t ldx, uint8_t* q, int64_t ldq,
                             float* s, int64_t lds, int64_t M, int64_t K, void* stream) {
  return quant_group128("fp8_quant_group128", true, x, x_dtype, ldx, q, ldq, s, lds, M, K, stream);
}

}  // extern "C"
