// SPDX-License-Identifier: MIT
// 16-bit MFMA GEMMs over dequantized weights for gfx950: bf16 (or fp16)
// activations x weights decoded to bf16 (fp16) and contracted with
// mfma_f32_16x16x32_bf16 (_f16). Dense and MoE (grouped over aligned sorted
// ids), with the same fused epilogues as the 8-bit kernels.
//
// Weight formats (decode is exact except where a scale is applied in fp32
// and the product rounded once to bf16/fp16):
//   BF16      bf16 [E][N][K], copied as is
//   MXFP4     e2m1 nibbles [E][N][K/2] (low nibble = even k) + e8m0 [E][N][K/32],
//             value = e2m1 * 2^(e-127), e == 0 is a zero block
//             (csrc/gemm/mxfp4_wmma_gemm.hip:14-23; tests/test_mxfp4.py:28-95)
//   INT4_ZP   uint4 [E][N][K/2] bytes (= int32 [E][N][K/8], k = 8w+j in nibble j),
//             scales [E][N][K/G] bf16/fp16, zero points uint8 [E][N/2][K/G]
//             (even n in the low nibble); value = (q - z) * s
//   INT4_SYM  same packing, value = (q - 8) * s (csrc/moe/moe_gemm_w4a16.hip:7-14)
//   FP8       e4m3fn [E][N][K] with fp32 128x128 block scales [E][N/128][K/128]
//             or per-channel scales [E][N] (csrc/moe/moe_gemm_w8a16.hip:15-36)
//   INT8      int8 [E][N][K] with per-channel scales [E][N] (W8A16)
//
// Kernels:
//   stream16: decode shapes. Each wave decodes its weight rows in registers
//             (16 bytes of packed weights per lane per chunk), waves split K
//             and reduce through LDS.
//   tiled16:  prefill. Each 64-K stage, the block's threads decode the weight
//             tile once into LDS (the swizzled 128-byte row layout of
//             gemm_common.h), token rows arrive by direct global->LDS copy, and
//             every wave reads both operands as MFMA fragments.
#include <type_traits>

#include "capi_internal.h"
#include "gemm_common.h"
#include "strix_common.h"

namespace strix {
namespace {

// kWInt4Ex: uint4b8 (q - 8) in vLLM's RDNAHybridW4A16 order: each little-endian
// 32-bit word holds 8 consecutive K values, nibble j carrying k = 0 2 4 6 1 3 5 7
// (csrc/gemm/w4a16_wmma_gemm.hip:1-8, 82-89). kWU8b128: uint8 bytes, value b - 128.
enum WFmt : int { kWBf16 = 0, kWMxfp4 = 1, kWInt4Zp = 2, kWInt4Sym = 3, kWFp8 = 4, kWInt8 = 5, kWInt4Ex = 6,
                  kWU8b128 = 7 };
enum SKind : int { kSF32 = 0, kSBf16 = 1, kSF16 = 2, kSE8m0 = 3 };

template <int FMT>
struct FmtInfo {
  static constexpr int bits = (FMT == kWBf16) ? 16 : ((FMT == kWFp8 || FMT == kWInt8 || FMT == kWU8b128) ? 8 : 4);
};

struct G16 {
  const uint8_t* w;  // weights, row stride ldw and expert stride w_es in bytes
  int64_t ldw, w_es;
  const void* ws;    // scales: element strides per expert / per scale row / per K group
  int64_t ws_es, ws_ns, ws_ks;
  int ws_kind;       // SKind
  int ws_kgroup;     // K elements per scale along K (0: one scale for all K)
  int ws_nblock;     // weight rows per scale row (128 for fp8 block scales, else 1)
  const uint8_t* wz; // int4 zero points [E][N/2][K/G]
  int64_t wz_es, wz_ns, wz_ks;
  const uint16_t* a; // activations (bf16 or fp16), row stride lda elements
  int64_t lda;
  const uint16_t* bias;  // dense only: output-dtype bias, row stride bias_rs (0 = [N])
  int64_t bias_rs;
  void* out;
  int64_t ldo;
  int out_f16;
  int M, N, K, n_out, gate_off;
  const int32_t* sorted_ids;
  int64_t sorted_len;
  const int32_t* expert_ids;
  const int32_t* num_post;
  int num_slots, top_k;
  const float* topk_w;
  int64_t a_rows;    // MoE: activation rows (for the 32-bit offset check of ring16)
  int ring16;        // MoE int4 decode: 1 = through ring16 where it applies
};

// Scale of weight row n (within an expert) at K position k.
__device__ __forceinline__ float wscale(const G16& p, int e, int n, int k) {
  const int64_t idx = (int64_t)e * p.ws_es + (int64_t)(n / p.ws_nblock) * p.ws_ns +
                      (p.ws_kgroup ? (int64_t)(k / p.ws_kgroup) * p.ws_ks : 0);
  switch (p.ws_kind) {
    case kSF32: return static_cast<const float*>(p.ws)[idx];
    case kSBf16: return bf16_bits_to_f32(static_cast<const uint16_t*>(p.ws)[idx]);
    case kSF16: return f16_bits_to_f32(static_cast<const uint16_t*>(p.ws)[idx]);
    default: {
      const uint32_t b = static_cast<const uint8_t*>(p.ws)[idx];
      return __uint_as_float(b << 23);  // 2^(b-127); b == 0 gives +0: the zero block
    }
  }
}

// Split form of wscale/wzero for prefetching: the raw bits are loaded with
// the weights and turned into values when the weights are decoded.
__device__ __forceinline__ int64_t wscale_row(const G16& p, int e, int n) {
  return (int64_t)e * p.ws_es + (int64_t)(n / p.ws_nblock) * p.ws_ns;
}
// The scale encoding: fixed by the format for MXFP4 (e8m0), else the runtime
// kind. A compile-time kind keeps the streaming loops free of branches that
// would make the compiler drain every outstanding load at the loop head.
template <int FMT>
__device__ __forceinline__ int scale_kind(const G16& p) {
  if constexpr (FMT == kWMxfp4) return kSE8m0;
  else return p.ws_kind;
}
template <int FMT>
__device__ __forceinline__ uint32_t wscale_raw(const G16& p, int64_t row_idx, int k) {
  const int64_t idx = row_idx + (p.ws_kgroup ? (int64_t)(k / p.ws_kgroup) * p.ws_ks : 0);
  switch (scale_kind<FMT>(p)) {
    case kSF32: return static_cast<const uint32_t*>(p.ws)[idx];
    case kSBf16:
    case kSF16: return static_cast<const uint16_t*>(p.ws)[idx];
    default: return static_cast<const uint8_t*>(p.ws)[idx];
  }
}
template <int FMT>
__device__ __forceinline__ float wscale_value(const G16& p, uint32_t raw) {
  switch (scale_kind<FMT>(p)) {
    case kSF32: return __uint_as_float(raw);
    case kSBf16: return bf16_bits_to_f32(raw);
    case kSF16: return f16_bits_to_f32(raw);
    default: return __uint_as_float(raw << 23);  // 2^(b-127); b == 0 gives +0: the zero block
  }
}
__device__ __forceinline__ int64_t wzero_row(const G16& p, int e, int n) {
  return (int64_t)e * p.wz_es + (int64_t)(n >> 1) * p.wz_ns;
}
__device__ __forceinline__ uint32_t wzero_raw(const G16& p, int64_t row_idx, int k) {
  return p.wz[row_idx + (int64_t)(k / p.ws_kgroup) * p.wz_ks];
}

__device__ __forceinline__ float wzero(const G16& p, int e, int n, int k) {
  const uint32_t b = p.wz[(int64_t)e * p.wz_es + (int64_t)(n >> 1) * p.wz_ns + (int64_t)(k / p.ws_kgroup) * p.wz_ks];
  return (float)((n & 1) ? (b >> 4) : (b & 15));
}

template <bool F16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (F16) return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
  else return pack_bf16x2(lo, hi);
}

// e2m1 magnitude code (3 bits) -> fp32 bits for a unit scale.
__device__ __forceinline__ float e2m1_mag(uint32_t c) {
  const uint32_t e = c >> 1, m = c & 1;
  const uint32_t bits = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3f000000u : 0u);
  return __uint_as_float(bits);
}

// MXFP4 -> bf16 by table. With an e8m0 scale 2^(b-127) every decoded value
// is exact in bf16, and for 2 <= b <= 252 it stays a normal number, so its
// bits are the unit-scale bits of the magnitude plus (b-127) in the exponent
// field. The 8-entry table of scaled magnitudes is split into a low-byte and
// a high-byte table of 8 bytes each, which v_perm_b32 indexes with four
// 3-bit magnitude codes at a time; the sign bit goes into the high byte. An
// e8m0 of 0 is the zero block (signed zeros, like value * 0). Other exponents
// take the scalar path.
struct Mxfp4Lut {
  uint32_t lo_l, lo_h, hi_l, hi_h;  // bytes of the table entries 0..3 / 4..7
};
__device__ __forceinline__ bool mxfp4_lut_ok(uint32_t b) { return b == 0u || (b >= 2u && b <= 252u); }
__device__ __forceinline__ Mxfp4Lut mxfp4_lut(uint32_t b) {
  // Unit-scale bf16 bits of the magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6.
  const int dlt = ((int)b - 127) << 7;
  auto e = [&](int base) -> uint32_t { return b == 0u ? 0u : (uint32_t)(base + dlt); };
  const uint32_t t01 = e(0x3F00) << 16;
  const uint32_t t23 = e(0x3F80) | (e(0x3FC0) << 16);
  const uint32_t t45 = e(0x4000) | (e(0x4040) << 16);
  const uint32_t t67 = e(0x4080) | (e(0x40C0) << 16);
  Mxfp4Lut t;
  t.lo_l = __builtin_amdgcn_perm(t23, t01, 0x06040200u);
  t.lo_h = __builtin_amdgcn_perm(t67, t45, 0x06040200u);
  t.hi_l = __builtin_amdgcn_perm(t23, t01, 0x07050301u);
  t.hi_h = __builtin_amdgcn_perm(t67, t45, 0x07050301u);
  return t;
}
// 8 e2m1 codes of d (nibble i = value i) -> 4 dwords of bf16 pairs.
__device__ __forceinline__ void mxfp4_dword_lut(uint32_t d, const Mxfp4Lut& t, uint32_t* out) {
  const uint32_t me = d & 0x07070707u, mo = (d >> 4) & 0x07070707u;  // magnitudes of even / odd values
  const uint32_t lo_e = __builtin_amdgcn_perm(t.lo_h, t.lo_l, me);
  const uint32_t hi_e = __builtin_amdgcn_perm(t.hi_h, t.hi_l, me) | ((d << 4) & 0x80808080u);
  const uint32_t lo_o = __builtin_amdgcn_perm(t.lo_h, t.lo_l, mo);
  const uint32_t hi_o = __builtin_amdgcn_perm(t.hi_h, t.hi_l, mo) | (d & 0x80808080u);
  const uint32_t e01 = __builtin_amdgcn_perm(hi_e, lo_e, 0x05010400u);  // values 0, 2
  const uint32_t e23 = __builtin_amdgcn_perm(hi_e, lo_e, 0x07030602u);  // values 4, 6
  const uint32_t o01 = __builtin_amdgcn_perm(hi_o, lo_o, 0x05010400u);  // values 1, 3
  const uint32_t o23 = __builtin_amdgcn_perm(hi_o, lo_o, 0x07030602u);  // values 5, 7
  out[0] = __builtin_amdgcn_perm(o01, e01, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(o01, e01, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(o23, e23, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(o23, e23, 0x07060302u);
}

// e8m0 exponents whose scaled e2m1 values are all normal bf16 numbers
// (0.5 * 2^(b-127) >= 2^-126 and 6 * 2^(b-127) < 2^128): the products are
// exact, so any correct conversion gives the same bits.
__device__ __forceinline__ bool mxfp4_cvt_ok(uint32_t b) { return b >= 2u && b <= 252u; }
// 8 e2m1 codes of d (nibble i = value i) -> 4 dwords of bf16 pairs scaled by
// 2^(b-127), one gfx950 scaled fp4 -> bf16 conversion per byte.
__device__ __forceinline__ void mxfp4_dword_cvt(uint32_t d, uint32_t b, uint32_t* out) {
  const float sc = __uint_as_float(b << 23);
  out[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 0));
  out[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 1));
  out[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 2));
  out[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 3));
}

// 8 int4 codes of d (nibble i = value i) with zero point z -> 4 dwords of
// 16-bit pairs (q - z) * s, as decode_dword gives them, in about 3 VALU
// operations per value instead of 4.5: zb holds 16 - z in each byte, so a
// byte of (d & 0x0f0f0f0f) + zb is v = q - z + 16 (1..31, no carry between
// bytes), which one byte-to-float conversion takes exactly; fma(v, s, c)
// with c = -16 s (exact) is (v - 16) s = (q - z) s rounded once, the same
// bits as the product. The caller keeps |s| <= 2^123 so that c is finite.
template <bool F16>
__device__ __forceinline__ void int4_dword_fma(uint32_t d, uint32_t zb, float s, float c, uint32_t* out) {
  const uint32_t lo = (d & 0x0f0f0f0fu) + zb, hi = ((d >> 4) & 0x0f0f0f0fu) + zb;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v0 = (float)((lo >> (8 * j)) & 0xffu);
    const float v1 = (float)((hi >> (8 * j)) & 0xffu);
    out[j] = pack2<F16>(__builtin_fmaf(v0, s, c), __builtin_fmaf(v1, s, c));
  }
}

// Decodes one dword of packed weights (8 values for 4-bit formats, 4 for
// 8-bit) into 16-bit values, appending to out[] as packed pairs.
template <int FMT, bool F16>
__device__ __forceinline__ void decode_dword(uint32_t d, float s, float z, uint32_t* out) {
  if constexpr (FMT == kWMxfp4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t byte = (d >> (8 * j)) & 0xffu;
      const uint32_t lo = byte & 15u, hi = byte >> 4;
      float vl = e2m1_mag(lo & 7u) * s, vh = e2m1_mag(hi & 7u) * s;
      vl = (lo & 8u) ? -vl : vl;
      vh = (hi & 8u) ? -vh : vh;
      out[j] = pack2<F16>(vl, vh);
    }
  } else if constexpr (FMT == kWInt4Zp || FMT == kWInt4Sym) {
    const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q0 = (float)((lo >> (8 * j)) & 0xffu);
      const float q1 = (float)((hi >> (8 * j)) & 0xffu);
      out[j] = pack2<F16>((q0 - z) * s, (q1 - z) * s);
    }
  } else if constexpr (FMT == kWFp8) {
    const f32x2_t v01 = e4m3x2_to_f32<false>(d), v23 = e4m3x2_to_f32<true>(d);
    out[0] = pack2<F16>(v01[0] * s, v01[1] * s);
    out[1] = pack2<F16>(v23[0] * s, v23[1] * s);
  } else if constexpr (FMT == kWInt8) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float v0 = (float)(int)(int8_t)((d >> (16 * j)) & 0xffu);
      const float v1 = (float)(int)(int8_t)((d >> (16 * j + 8)) & 0xffu);
      out[j] = pack2<F16>(v0 * s, v1 * s);
    }
  } else if constexpr (FMT == kWU8b128) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float v0 = (float)((int)((d >> (16 * j)) & 0xffu) - 128);
      const float v1 = (float)((int)((d >> (16 * j + 8)) & 0xffu) - 128);
      out[j] = pack2<F16>(v0 * s, v1 * s);
    }
  } else if constexpr (FMT == kWInt4Ex) {
    // lo bytes hold nibbles 0 2 4 6 (k 0 4 1 5), hi bytes nibbles 1 3 5 7 (k 2 6 3 7).
    const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
    auto f = [&](uint32_t w, int b) { return ((float)((w >> (8 * b)) & 0xffu) - 8.0f) * s; };
    out[0] = pack2<F16>(f(lo, 0), f(lo, 2));  // k 0, 1
    out[1] = pack2<F16>(f(hi, 0), f(hi, 2));  // k 2, 3
    out[2] = pack2<F16>(f(lo, 1), f(lo, 3));  // k 4, 5
    out[3] = pack2<F16>(f(hi, 1), f(hi, 3));  // k 6, 7
  }
}

// ============================================================ stream16
// Per chunk a lane holds PV consecutive K values of its weight row: 32 for
// 4-bit weights in 16 bytes (a 64-K tail of a K that is 64 mod 128 uses 8
// bytes, PV 16), 16 for 8-bit, 8 for bf16. MFMA step j of the chunk pairs the
// lane's values 8j..8j+7 with the same K positions of the token rows.
// FOLD (int4 with one scale per 128-K chunk or per row): the MFMAs take the
// raw codes as 16-bit numbers OFF + q (OFF 128 for bf16, 1024 for fp16, whose
// mantissa then holds q itself, so a code becomes a 16-bit value with two
// byte permutes), and each chunk's product is folded into the fp32
// accumulator as s * (P - (OFF + z) * A), with A the chunk's token sums from
// one more MFMA against ones. The per-element decode then costs about one
// VALU operation instead of four; the weights enter the products exactly,
// where the unfolded path first rounds (q - z) * s to 16 bits.
template <int FMT, int NT, int MT, int WAVES, bool MOE, int EPI, int ACT, bool F16, bool FOLD = false>
__global__ void __launch_bounds__(WAVES * 64) stream16_kernel(G16 p) {
  static_assert(!FOLD || FMT == kWInt4Zp || FMT == kWInt4Sym, "folded decode: int4 weights");
  constexpr int BITS = FmtInfo<FMT>::bits;
  constexpr int PV = 128 / BITS;   // K values per lane per full chunk (16 bytes)
  constexpr int CK = 4 * PV;       // K per full chunk
  constexpr int NTH = (EPI == kEpiGated) ? NT / 2 : NT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int m0 = blockIdx.y * (16 * MT);
  int expert = 0;
  if constexpr (MOE) {
    expert = moe_block_expert(p.num_post, p.expert_ids, m0);
    if (expert < 0) return;
  }
  const int nout0 = blockIdx.x * (16 * NTH);
  int wrow[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    int r;
    if constexpr (EPI == kEpiGated) r = s < NTH ? nout0 + 16 * s : p.gate_off + nout0 + 16 * (s - NTH);
    else r = nout0 + 16 * s;
    wrow[s] = min(r + r16, p.N - 1);  // this lane's weight row of subtile s
  }
  const uint8_t* wbase = p.w + (int64_t)expert * p.w_es;
  int brow[MT], orow[MT];
  bool bval[MT];
  {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) mrow[t] = m0 + 16 * t + r16;
    token_rows<MOE, MT>(p, mrow, brow, orow, bval);
  }

  const int nfull = p.K / CK;
  const bool tail = (p.K % CK) != 0;  // 4-bit only: a 64-K tail (K % 64 == 0 is required)
  const int nch = nfull + (tail ? 1 : 0);
  const int per = (nch + WAVES - 1) / WAVES;
  const int c0 = min(nch, wave * per), c1 = min(nch, c0 + per);

  v4f acc[NT][MT];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[s][t] = v4f{0.f, 0.f, 0.f, 0.f};

  // One chunk's MFMAs from its decoded weights and token rows.
  auto mfmas = [&](const uint32_t (&wv)[NT][PV / 2], const u32x4 (&av)[MT][PV / 8], auto steps_tag) {
    constexpr int STEPS = decltype(steps_tag)::value;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < STEPS; ++j)
#pragma unroll
        for (int s = 0; s < NT; ++s) {
          u32x4 wq;
#pragma unroll
          for (int i = 0; i < 4; ++i) wq[i] = wv[s][4 * j + i];
          if constexpr (F16)
            acc[s][t] = mfma_f16(__builtin_bit_cast(f16x8, wq), __builtin_bit_cast(f16x8, av[t][j]), acc[s][t]);
          else
            acc[s][t] = mfma_bf16(__builtin_bit_cast(bf16x8, wq), __builtin_bit_cast(bf16x8, av[t][j]), acc[s][t]);
        }
  };
  const int skind = scale_kind<FMT>(p);
  const int sbytes = skind == kSF32 ? 4 : (skind == kSE8m0 ? 1 : 2);
  const uint32_t smask = sbytes == 4 ? 0xffffffffu : (sbytes == 2 ? 0xffffu : 0xffu);
  // Pointer arithmetic (not integer casts) keeps the loads global, not flat.
  auto word_at = [](const void* base, int64_t byte_off, uint32_t& word, uint32_t& shift) {
    const uint8_t* b8 = static_cast<const uint8_t*>(base);
    const int64_t mis = (int64_t)(reinterpret_cast<uintptr_t>(b8) & 3u);
    const int64_t o = byte_off + mis;
    word = *reinterpret_cast<const uint32_t*>(b8 + ((o & ~(int64_t)3) - mis));
    shift = (uint32_t)(o & 3) * 8u;
  };
  // Scale bits -> value without a branch on the kind.
  auto scale_of = [&](uint32_t raw) {
    const float f32 = __uint_as_float(raw), bf = __uint_as_float(raw << 16), e8 = __uint_as_float(raw << 23);
    const float h = f16_bits_to_f32(raw & 0xffffu);
    return skind == kSF32 ? f32 : skind == kSBf16 ? bf : skind == kSF16 ? h : e8;
  };
  constexpr bool HAS_S = (FMT != kWBf16);
  constexpr bool ZP = (FMT == kWInt4Zp);
  int64_t srow[NT], zrow[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    srow[s] = HAS_S ? wscale_row(p, expert, wrow[s]) : 0;
    zrow[s] = ZP ? wzero_row(p, expert, wrow[s]) : 0;
  }
  // Decodes raw dwords with the raw scale / zero bits of each subtile.
  auto decode = [&](const uint32_t* raw, int ndw, int s, uint32_t sbits, uint32_t zbits, uint32_t* wv) {
    if constexpr (FMT == kWBf16) {
      for (int i = 0; i < ndw; ++i) wv[i] = raw[i];
    } else {
      if constexpr (FMT == kWMxfp4 && !F16) {
        // e8m0 scales: bf16 by table (v_perm), the scalar path only for the
        // rare exponents the table cannot take. A lane's dwords share a scale.
        if (scale_kind<FMT>(p) == kSE8m0 && mxfp4_cvt_ok(sbits)) {
#pragma unroll
          for (int i = 0; i < ndw; ++i) mxfp4_dword_cvt(raw[i], sbits, &wv[4 * i]);
          return;
        }
        if (scale_kind<FMT>(p) == kSE8m0 && mxfp4_lut_ok(sbits)) {
          const Mxfp4Lut t = mxfp4_lut(sbits);
#pragma unroll
          for (int i = 0; i < ndw; ++i) mxfp4_dword_lut(raw[i], t, &wv[4 * i]);
          return;
        }
      }
      const float sc = scale_of(sbits);
      const float z = ZP ? (float)((wrow[s] & 1) ? ((zbits >> 4) & 15u) : (zbits & 15u)) : 8.0f;
      constexpr int PAIRS_PER_DWORD = 32 / BITS / 2;
#pragma unroll
      for (int i = 0; i < ndw; ++i) decode_dword<FMT, F16>(raw[i], sc, z, &wv[i * PAIRS_PER_DWORD]);
    }
  };
  // Full chunks run as a two-deep register pipeline: the raw weights, raw
  // scale bits and token rows of chunk c+1 are in flight while chunk c is
  // decoded and multiplied. Every load is issued unconditionally (the index
  // is clamped to the wave's last chunk), so each wait counts exactly the
  // loads of the later chunk.
  //
  // Scales and zero points arrive as the aligned 32-bit word that holds
  // them, whatever their width (f32, bf16/fp16, e8m0 or zero-point byte),
  // with the bit offset kept beside it: one load form for every scale kind,
  // so the loop has no branch on the kind (the compiler drains all
  // outstanding loads at such a branch), and nothing narrower than a word is
  // carried around the loop (a zero-extended copy would be computed at the
  // loop latch, which would then wait for the chunk just issued). The word
  // lies in the same 4-byte-aligned span as the element, so within the
  // element's page.
  struct Buf {
    uint32_t w[NT][4];
    uint32_t s[NT], z[NT];
    uint32_t ssh[NT], zsh[NT];
    u32x4 a[MT][PV / 8];
  };
  auto load = [&](int c, Buf& b) {
    const int kc = c * CK + g4 * PV;
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      const u32x4 r4 = ldg128(wbase + (int64_t)wrow[s] * p.ldw + (int64_t)kc * BITS / 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) b.w[s][i] = r4[i];
      if constexpr (HAS_S) {
        const int64_t si = srow[s] + (p.ws_kgroup ? (int64_t)(kc / p.ws_kgroup) * p.ws_ks : 0);
        word_at(p.ws, si * sbytes, b.s[s], b.ssh[s]);
      }
      if constexpr (ZP) word_at(p.wz, zrow[s] + (int64_t)(kc / p.ws_kgroup) * p.wz_ks, b.z[s], b.zsh[s]);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const uint16_t* ar = p.a + (int64_t)brow[t] * p.lda + kc;
#pragma unroll
      for (int j = 0; j < PV / 8; ++j) b.a[t][j] = ldg128(ar + 8 * j);
    }
  };
  auto compute = [&](const Buf& b) {
    uint32_t wv[NT][PV / 2];
    if constexpr (FOLD) {
      constexpr uint32_t HI = F16 ? 0x64646464u : 0x43434343u;   // high byte of OFF + q
      constexpr float OFF = F16 ? 1024.0f : 128.0f;
      constexpr uint32_t ONE2 = F16 ? 0x3c003c00u : 0x3f803f80u;  // two 16-bit ones
      float cs[NT], cz[NT];   // this lane's row: scale and -(OFF + z) * scale
#pragma unroll
      for (int s = 0; s < NT; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t d = b.w[s][i];
          const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
          const uint32_t x0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // codes of k 0..3
          const uint32_t x1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // codes of k 4..7
          wv[s][4 * i + 0] = __builtin_amdgcn_perm(HI, x0, 0x04010400u);
          wv[s][4 * i + 1] = __builtin_amdgcn_perm(HI, x0, 0x04030402u);
          wv[s][4 * i + 2] = __builtin_amdgcn_perm(HI, x1, 0x04010400u);
          wv[s][4 * i + 3] = __builtin_amdgcn_perm(HI, x1, 0x04030402u);
        }
        const float sc = scale_of((b.s[s] >> b.ssh[s]) & smask);
        const uint32_t zb = ZP ? (b.z[s] >> b.zsh[s]) & 0xffu : 0u;
        const float z = ZP ? (float)((wrow[s] & 1) ? (zb >> 4) : (zb & 15u)) : 8.0f;
        cs[s] = sc;
        cz[s] = -(OFF + z) * sc;
      }
      v4f part[NT][MT], asum[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        asum[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NT; ++s) part[s][t] = v4f{0.f, 0.f, 0.f, 0.f};
      }
      const u32x4 ones = {ONE2, ONE2, ONE2, ONE2};
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < PV / 8; ++j) {
#pragma unroll
          for (int s = 0; s < NT; ++s) {
            u32x4 wq;
#pragma unroll
            for (int i = 0; i < 4; ++i) wq[i] = wv[s][4 * j + i];
            if constexpr (F16)
              part[s][t] = mfma_f16(__builtin_bit_cast(f16x8, wq), __builtin_bit_cast(f16x8, b.a[t][j]), part[s][t]);
            else
              part[s][t] = mfma_bf16(__builtin_bit_cast(bf16x8, wq), __builtin_bit_cast(bf16x8, b.a[t][j]), part[s][t]);
          }
          if constexpr (F16)
            asum[t] = mfma_f16(__builtin_bit_cast(f16x8, ones), __builtin_bit_cast(f16x8, b.a[t][j]), asum[t]);
          else
            asum[t] = mfma_bf16(__builtin_bit_cast(bf16x8, ones), __builtin_bit_cast(bf16x8, b.a[t][j]), asum[t]);
        }
      // Element i of a lane's result is weight row 4*g4 + i of the subtile:
      // its scale terms come from the lane that decoded that row (lane 4*g4 + i).
#pragma unroll
      for (int s = 0; s < NT; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float si = __shfl(cs[s], 4 * g4 + i, 64);
          const float zi = __shfl(cz[s], 4 * g4 + i, 64);
#pragma unroll
          for (int t = 0; t < MT; ++t)
            acc[s][t][i] = fmaf(zi, asum[t][i], fmaf(si, part[s][t][i], acc[s][t][i]));
        }
      return;
    }
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      const uint32_t sbits = HAS_S ? (b.s[s] >> b.ssh[s]) & smask : 0u;
      decode(b.w[s], 4, s, sbits, ZP ? (b.z[s] >> b.zsh[s]) & 0xffu : 0u, wv[s]);
    }
    mfmas(wv, b.a, std::integral_constant<int, PV / 8>{});
  };
  const int f1 = min(c1, nfull);
  if (c0 < f1) {
    // One exit, at the loop test: a break between the two halves makes the
    // structurized loop carry a path on which B's loads are still pending at
    // the loop head, and the compiler then drains every load there.
    Buf A, B;
    load(c0, A);
    int c = c0;
    for (; c + 1 < f1; c += 2) {
      load(c + 1, B);
      compute(A);
      load(min(c + 2, f1 - 1), A);
      compute(B);
    }
    if (c < f1) compute(A);
  }
  // A 4-bit K that is 64 mod 128 ends with a half chunk (8 bytes per lane).
  if constexpr (FMT != kWBf16 && BITS == 4 && !FOLD) {
    if (tail && c1 == nch && c0 < c1) {
      const int kc = nfull * CK + g4 * (PV / 2);
      uint32_t wv[NT][PV / 2];
#pragma unroll
      for (int s = 0; s < NT; ++s) {
        const uint2 r2 = *reinterpret_cast<const uint2*>(wbase + (int64_t)wrow[s] * p.ldw + (int64_t)kc * BITS / 8);
        const uint32_t raw[2] = {r2.x, r2.y};
        decode(raw, 2, s, wscale_raw<FMT>(p, srow[s], kc), ZP ? wzero_raw(p, zrow[s], kc) : 0u, wv[s]);
      }
      u32x4 av[MT][PV / 8];
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < PV / 16; ++j) av[t][j] = ldg128(p.a + (int64_t)brow[t] * p.lda + kc + 8 * j);
      mfmas(wv, av, std::integral_constant<int, PV / 16>{});
    }
  }

  constexpr int TILES = NT * MT;
  __shared__ float red[WAVES > 1 ? WAVES * TILES * 4 * 64 : 1];
  if constexpr (WAVES > 1) {
#pragma unroll
    for (int s = 0; s < NT; ++s)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wave * TILES + s * MT + t) * 4 + i) * 64 + lane] = acc[s][t][i];
    __syncthreads();
  }
#pragma unroll
  for (int so = 0; so < NTH; ++so)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int o = so * MT + t;
      if (WAVES > 1 && (o % WAVES) != wave) continue;
      float g[4], u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (WAVES > 1) {
          float sg = 0.f, su = 0.f;
          for (int w = 0; w < WAVES; ++w) {
            sg += red[((w * TILES + so * MT + t) * 4 + i) * 64 + lane];
            if constexpr (EPI == kEpiGated) su += red[((w * TILES + (so + NTH) * MT + t) * 4 + i) * 64 + lane];
          }
          g[i] = sg;
          u[i] = su;
        } else {
          g[i] = acc[so][t][i];
          u[i] = (EPI == kEpiGated) ? acc[so + NTH][t][i] : 0.f;
        }
      }
      if (!bval[t]) continue;
      const int col0 = nout0 + 16 * so + 4 * g4;
      if constexpr (!MOE && EPI == kEpiStore) {
        if (p.bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (col0 + i < p.n_out) {
              const uint32_t b = p.bias[(int64_t)orow[t] * p.bias_rs + col0 + i];
              g[i] += p.out_f16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b);
            }
        }
      }
      finish_float4<EPI, ACT, MOE>(p, orow[t], col0, g, u);
    }
}

// ============================================================ ring16
// int4 expert decode (MoE block_m 16) through an LDS ring, the 16-bit
// counterpart of ring8. One wave owns NT = 2 weight subtiles (a gated
// gate/up pair, or two plain subtiles) of one expert block over a range of
// K; KS waves of a block split K, each with its own ring, and add their
// partial sums through LDS at the end in a fixed order. Each ring slot is a
// 256-K step filled by direct global->LDS copies: whole 128-byte lines of
// packed weights (8 rows per copy, chunks XOR-swizzled like ring8), the
// step's TQ token rows (512 bytes of bf16/fp16 each, 2 rows per copy,
// swizzled by row), and one 4-byte-per-lane copy of the step's two 128-K
// scale elements per weight row (lanes 0..31) and zero-point bytes per row
// pair (lanes 32..47). Every wave issues the same copies per step, so
// `s_waitcnt vmcnt` counts exactly the steps still in flight.
//
// Within a 128-K group lane (r16, g4) takes the 32 contiguous K of bytes
// 16*g4.. of its row (one 16-byte LDS read) and MFMA j of the group the 8 K
// of dword j; the token operand follows the same K order. The codes enter
// the MFMA as OFF + q and each group is folded as s * (P - (OFF + z) * A),
// A being the group's token sums from MFMAs against ones (the folded decode
// of stream16). Scales must be bf16/fp16 with 128-element groups and K a
// multiple of 256; the host checks this and the alignments.
__device__ __forceinline__ int tok_swz(int row) { return row & 15; }

template <int FMT, int TQ, int KS, int R, int EPI, int ACT, bool F16>
__global__ void __launch_bounds__(64 * KS) ring16_kernel(G16 p) {
  static_assert(FMT == kWInt4Zp || FMT == kWInt4Sym, "int4 weights");
  static_assert(TQ == 2 || TQ == 8 || TQ == 16, "token rows per slot");
  constexpr bool ZP = (FMT == kWInt4Zp);
  constexpr bool GATED = (EPI == kEpiGated);
  constexpr int NT = 2;
  constexpr int NTH = GATED ? 1 : 2;
  constexpr int WQ = 2 * NT;                 // weight copies per step (8 rows x 128 B)
  constexpr int TC = TQ / 2;                 // token copies per step (2 rows x 512 B)
  constexpr int PER = WQ + TC + 1;           // copies per step and wave
  constexpr int T_OFF = NT * 2048;
  constexpr int S_OFF = T_OFF + TQ * 512;
  constexpr int SLOT = S_OFF + 256;
  static_assert((R - 2) * PER < 64, "vmcnt counts at most 63 copies");
  static_assert(KS == 1 || R * SLOT >= NT * 4 * 64 * 4, "a wave's ring holds its partial sums");
  constexpr float OFF = F16 ? 1024.0f : 128.0f;
  constexpr uint32_t HI = F16 ? 0x64646464u : 0x43434343u;
  constexpr uint32_t ONE2 = F16 ? 0x3c003c00u : 0x3f803f80u;
  __shared__ __attribute__((aligned(1024))) uint8_t ring_all[KS * R * SLOT];

  const int lane = threadIdx.x & 63;
  const int kw = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* ring = ring_all + kw * (R * SLOT);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int m0 = blockIdx.y * 16;
  const int expert = moe_block_expert(p.num_post, p.expert_ids, m0);
  if (expert < 0) return;
  const int nout0 = blockIdx.x * (16 * NTH);
  int wrow0[NT];
  wrow0[0] = nout0;
  wrow0[1] = GATED ? p.gate_off + nout0 : nout0 + 16;
  const uint8_t* wbase = p.w + (int64_t)expert * p.w_es;

  // Weight copy q: subtile q/2, rows 8*(q%2) + lane/8 of it; LDS position
  // lane%8 of the row holds the row's 16-byte chunk (lane%8) ^ swz(row).
  const int crow = lane >> 3;
  uint32_t woff[WQ];
#pragma unroll
  for (int q = 0; q < WQ; ++q) {
    const int row = 8 * (q & 1) + crow;
    const int wr = min(wrow0[q >> 1] + row, p.N - 1);
    woff[q] = (uint32_t)wr * (uint32_t)p.ldw + 16u * (uint32_t)((lane & 7) ^ lds_swz(row));
  }
  // Token copy c: rows 2c + lane/32, chunk (lane%32) ^ tok_swz(row) of the row's 512 bytes.
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(p.a);
  uint32_t toff[TC];
  {
    int mrow[TC], br[TC], orw[TC];
    bool v[TC];
#pragma unroll
    for (int c = 0; c < TC; ++c) mrow[c] = m0 + 2 * c + (lane >> 5);
    token_rows<true, TC>(p, mrow, br, orw, v);
#pragma unroll
    for (int c = 0; c < TC; ++c) {
      const int row = 2 * c + (lane >> 5);
      toff[c] = (uint32_t)br[c] * (uint32_t)(p.lda * 2) + 16u * (uint32_t)((lane & 31) ^ tok_swz(row));
    }
  }
  // Scale / zero-point word of this lane (element index of the step-0 word).
  const int srow_l = min(wrow0[(lane >> 4) & 1] + r16, p.N - 1);  // lanes 0..31: subtile lane/16, row lane%16
  const uint16_t* sbase = static_cast<const uint16_t*>(p.ws);
  const int64_t sidx = wscale_row(p, expert, srow_l);
  int64_t zidx = 0;
  if constexpr (ZP) {
    const int q = lane & 15;                                          // lanes 32..47 (and 48..63 again)
    const int zr = min(wrow0[q >> 3] + 2 * (q & 7), p.N - 2);
    zidx = wzero_row(p, expert, zr);
  }
  const bool zlane = ZP && lane >= 32;
  auto x_addr = [&](int st) -> const void* {
    if (zlane) {
      const uint8_t* za = p.wz + zidx + (int64_t)(2 * st) * p.wz_ks;
      return reinterpret_cast<const void*>(reinterpret_cast<uintptr_t>(za) & ~(uintptr_t)3);
    }
    return sbase + sidx + (int64_t)(2 * st) * p.ws_ks;
  };

  auto issue = [&](int st, int slot) {
    uint8_t* dst = ring + slot * SLOT;
    const uint8_t* wb = wbase + (int64_t)st * 128;
    const uint8_t* ab = abase + (int64_t)st * 512;
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
      uint32_t o = woff[q];
      asm volatile("" : "+v"(o));
      g2l_b128(wb + o, dst + q * 1024);
    }
#pragma unroll
    for (int c = 0; c < TC; ++c) {
      uint32_t o = toff[c];
      asm volatile("" : "+v"(o));
      g2l_b128(ab + o, dst + T_OFF + c * 1024);
    }
    g2l_b32(x_addr(st), dst + S_OFF);
  };

  const int trow = TQ == 16 ? r16 : (r16 & (TQ - 1));   // token row this lane reads
  v4f acc[NT];
#pragma unroll
  for (int s2 = 0; s2 < NT; ++s2) acc[s2] = v4f{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {ONE2, ONE2, ONE2, ONE2};
  const int skind = p.ws_kind;
  auto sval = [&](uint32_t h) { return skind == kSF16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h); };

  const int nst_all = p.K >> 8;
  const int st0 = KS == 1 ? 0 : kw * nst_all / KS;
  const int st1 = KS == 1 ? nst_all : (kw + 1) * nst_all / KS;
#pragma unroll
  for (int s0 = 0; s0 < R - 1; ++s0)
    if (st0 + s0 < st1) issue(st0 + s0, s0);
  int slot = 0;
  for (int st = st0; st < st1; ++st) {
    constexpr int AHEAD = R - 2;
    if (st + AHEAD <= st1 - 1) wait_vmcnt<AHEAD * PER>();
    else wait_vmcnt<0>();
    const uint8_t* sl = ring + slot * SLOT;
    u32x4 bq[2][4], wr[NT][2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bq[gi][j] = lds128(sl + T_OFF + trow * 512 + 16 * ((16 * gi + 4 * g4 + j) ^ tok_swz(trow)));
#pragma unroll
    for (int s2 = 0; s2 < NT; ++s2)
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
        wr[s2][gi] = lds128(sl + s2 * 2048 + r16 * 128 + 16 * ((4 * gi + g4) ^ lds_swz(r16)));
    // Scale and zero-point terms of the lane's four result rows 4*g4 + i.
    uint32_t sw[NT][4], zw[NT][4];
#pragma unroll
    for (int s2 = 0; s2 < NT; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 4 * g4 + i;
        sw[s2][i] = *reinterpret_cast<const uint32_t*>(sl + S_OFF + 4 * (16 * s2 + n));
        zw[s2][i] = ZP ? *reinterpret_cast<const uint32_t*>(sl + S_OFF + 4 * (32 + 8 * s2 + (n >> 1))) : 0u;
      }
    // The consumed slot of the last step is free: every read of it is done.
    const int next = st + R - 1;
    if (next < st1) issue(next, slot == 0 ? R - 1 : slot - 1);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      v4f asum = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (F16) asum = mfma_f16(__builtin_bit_cast(f16x8, ones), __builtin_bit_cast(f16x8, bq[gi][j]), asum);
        else asum = mfma_bf16(__builtin_bit_cast(bf16x8, ones), __builtin_bit_cast(bf16x8, bq[gi][j]), asum);
      }
#pragma unroll
      for (int s2 = 0; s2 < NT; ++s2) {
        v4f part = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t d = wr[s2][gi][j];
          const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
          const uint32_t x0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // codes of k 0..3
          const uint32_t x1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // codes of k 4..7
          u32x4 wq;
          wq[0] = __builtin_amdgcn_perm(HI, x0, 0x04010400u);
          wq[1] = __builtin_amdgcn_perm(HI, x0, 0x04030402u);
          wq[2] = __builtin_amdgcn_perm(HI, x1, 0x04010400u);
          wq[3] = __builtin_amdgcn_perm(HI, x1, 0x04030402u);
          if constexpr (F16) part = mfma_f16(__builtin_bit_cast(f16x8, wq), __builtin_bit_cast(f16x8, bq[gi][j]), part);
          else part = mfma_bf16(__builtin_bit_cast(bf16x8, wq), __builtin_bit_cast(bf16x8, bq[gi][j]), part);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = 4 * g4 + i;
          const float sc = sval((sw[s2][i] >> (16 * gi)) & 0xffffu);
          float z = 8.0f;
          if constexpr (ZP) {
            const int zr = min(wrow0[s2] + 2 * (n >> 1), p.N - 2);
            const uintptr_t za = reinterpret_cast<uintptr_t>(p.wz) +
                                 (uintptr_t)(wzero_row(p, expert, zr) + (int64_t)(2 * st + gi) * p.wz_ks);
            const uint32_t zb = (zw[s2][i] >> (8u * (uint32_t)(za & 3u))) & 0xffu;
            z = (float)((n & 1) ? (zb >> 4) : (zb & 15u));
          }
          acc[s2][i] = fmaf(-(OFF + z) * sc, asum[i], fmaf(sc, part[i], acc[s2][i]));
        }
      }
    }
    slot = slot == R - 1 ? 0 : slot + 1;
  }

  if constexpr (KS > 1) {
    wait_vmcnt<0>();
    float* red = reinterpret_cast<float*>(ring);
#pragma unroll
    for (int s2 = 0; s2 < NT; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(s2 * 4 + i) * 64 + lane] = acc[s2][i];
    __syncthreads();
    if (kw != 0) return;
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      const float* rw = reinterpret_cast<const float*>(ring_all + w * (R * SLOT));
#pragma unroll
      for (int s2 = 0; s2 < NT; ++s2)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[s2][i] += rw[(s2 * 4 + i) * 64 + lane];
    }
  }
  if (nout0 >= p.n_out) return;
  int brow, orow;
  bool bval;
  token_row<true>(p, m0 + r16, brow, orow, bval);
  if (!bval) return;
#pragma unroll
  for (int so = 0; so < NTH; ++so) {
    float g[4], u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g[i] = acc[so][i];
      u[i] = GATED ? acc[1][i] : 0.f;
    }
    finish_float4<EPI, ACT, true>(p, orow, nout0 + 16 * so + 4 * g4, g, u);
  }
}

// ============================================================ tiled16
// One 64-K stage per LDS buffer: weight rows 0..BN-1 (decoded by the block's
// threads), token rows BN..BN+BM-1 (direct copies), 128 bytes per row,
// swizzled. Three buffers and a two-deep register pipeline of raw weights:
// while stage kb is computed, stage kb+1 is decoded into LDS from registers
// loaded two steps earlier, the token rows of stage kb+2 are in flight, and
// the raw weights of stage kb+3 are being fetched. Every load is issued
// unconditionally (indices past the end are clamped, their buffers never
// read), so each wait counts exactly the loads of later stages.
//
// NP > 0 specializes the waves: WM x WN consumer waves only run the MFMAs
// of stage kb while NP producer waves issue every load and decode stage
// kb+1 into LDS, so with one wave of each kind per SIMD the decode ALU work
// runs under the MFMAs instead of in turn with them. NP == 0: every wave
// decodes its share, then computes.
template <int FMT, int BM, int BN, int WM, int WN, int NP, bool MOE, int EPI, int ACT, bool F16, bool RAWL = false>
__global__ void __launch_bounds__((WM * WN + NP) * 64) tiled16_kernel(G16 p, int tiles_m, int tiles_n, int group_m) {
  constexpr int W = WM * WN;                 // MFMA waves
  constexpr int PW = NP > 0 ? NP : W;        // waves that load and decode
  constexpr int T = PW * 64;                 // their threads
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int MT = TM / 16, NT = TN / 16;
  constexpr int SA = BN / 16;
  constexpr int STAGES = 3;
  constexpr int STAGE = (BN + BM) * 128;
  constexpr int BITS = FmtInfo<FMT>::bits;
  constexpr bool DIRECT_W = (FMT == kWBf16);
  constexpr int PV = DIRECT_W ? 8 : 128 / BITS;  // K values per 16-byte weight piece
  constexpr int PPR = 64 / PV;                   // pieces per row per stage
  constexpr int PIECES = BN * PPR;
  constexpr int PPT = DIRECT_W ? 0 : (PIECES + T - 1) / T;  // pieces per thread (the last round may be partial)
  constexpr int ACOPY = BM / 8;                  // token row copies (8 rows each)
  constexpr int WCOPY = DIRECT_W ? BN / 8 : 0;
  static_assert((ACOPY + WCOPY) % PW == 0, "copies split evenly over the loading waves");
  constexpr int CPW = (ACOPY + WCOPY) / PW;
  constexpr bool GATED = (EPI == kEpiGated);
  constexpr int NTH = GATED ? NT / 2 : NT;
  static_assert(!GATED || NT % 2 == 0, "gated wave tiles pair gate and up subtiles");
  // RAWL: the packed 4-bit weights of a stage, with one 4-byte word of scale
  // bits per row and one of zero-point bits per row pair, arrive by direct
  // global->LDS copies into one of RS raw slots; producers decode from there.
  // No producer load then targets a register, so no compiler-inserted wait
  // can drain the copies in flight: each wait is the explicit count below.
  constexpr bool ZPF = (FMT == kWInt4Zp);
  constexpr int RS = RAWL ? 3 : 0;
  constexpr int RAW_W = BN * 32;                    // 64 K of 4-bit values per row
  constexpr int RAW_S = RAW_W;                      // scale words: BN x 4 bytes
  constexpr int RAW_Z = RAW_S + BN * 4;             // zero-point words: BN/2 x 4 bytes
  constexpr int RAWSLOT = RAW_Z + (ZPF ? BN * 2 : 0);
  constexpr int RQ = RAWL ? BN / 32 : 0;            // 1 KiB raw weight copies per stage
  constexpr int SQ = RAWL ? BN / 64 : 0;            // 4-byte-per-lane scale copies per stage
  constexpr int ZQ = (RAWL && ZPF) ? BN / 128 + (BN % 128 ? 1 : 0) : 0;  // zero-point copies
  static_assert(!RAWL || (BITS == 4 && NP > 0 && RQ % PW == 0 && SQ + ZQ <= PW && BN % 64 == 0),
                "raw-in-LDS decode: 4-bit weights, producer waves, copies split evenly");
  static_assert(STAGES * STAGE + RS * RAWSLOT <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE + RS * RAWSLOT];
  uint8_t* const rawbase = smem + STAGES * STAGE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const bool is_prod = NP == 0 || wave >= W;
  const bool is_cons = NP == 0 || wave < W;
  // Index among the loading waves. MFMA waves never load; their (unused)
  // copy and piece slots are computed as loading wave 0's so that every
  // address formed in the set-up below stays in range.
  const int pwave = NP > 0 ? max(wave - W, 0) : wave;
  const int ptid = NP > 0 ? max(tid - W * 64, 0) : tid;
  const int wm = wave % WM, wn = (wave / WM) % WN;
  int tm, tn, expert = 0;
  if constexpr (MOE) {
    if (!moe_tile(*p.num_post, BM, tm, tn)) return;
    // Checked after the token-row loads below are issued, so the two
    // lookups share one memory round trip.
    expert = p.expert_ids[tm];
  } else {
    dense_tile(blockIdx.x, tiles_m, tiles_n, group_m, tm, tn);
  }
  const int m0 = tm * BM;
  // MoE epilogue rows, loaded before the K loop (dense rows are arithmetic;
  // the register-staged raw-weight path has no registers to spare for them).
  constexpr bool PRE = MOE && RAWL;
  EpiRow erow[PRE ? MT : 1];
  // MoE: a consumer wave runs the MFMAs of its 16-row token subtiles up to
  // the last one that holds a routed row (an expert's last row tile is
  // mostly padding), and none when all its rows are padding; it still takes
  // part in every copy, decode and barrier.
  int mt_live = MT;
  if constexpr (PRE) {
    if (is_cons) {
      int mrow[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) mrow[t] = m0 + wm * TM + 16 * t + r16;
      epi_rows<MOE, MT>(p, mrow, erow);
      int live = 0;
#pragma unroll
      for (int t = 0; t < MT; ++t)
        if (__ballot(erow[t].valid)) live = t + 1;
      mt_live = live;
    }
  } else if constexpr (MOE) {
    constexpr int NJ = (TM + 63) / 64;
    int mrow[NJ], br[NJ], orw[NJ];
    bool v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) mrow[j] = m0 + wm * TM + 64 * j + lane;
    token_rows<true, NJ>(p, mrow, br, orw, v);
    int hi = -1;   // highest routed row of the wave's TM rows
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint64_t mask = __ballot(v[j] && 64 * j + lane < TM);
      if (mask) hi = 64 * j + 63 - __builtin_clzll(mask);
    }
    mt_live = (hi + 16) / 16;
  }
  const bool do_mma = is_cons && mt_live > 0;
  auto wrow_of = [&](int r) -> int {  // weight row of LDS weight row r (0..BN-1)
    if constexpr (GATED) {
      const int base = tn * (BN / 2);
      return r < BN / 2 ? base + r : p.gate_off + base + (r - BN / 2);
    } else {
      return tn * BN + r;
    }
  };

  // Direct copies (token rows, and bf16 weight rows): 8 rows x 128 B each.
  constexpr int CPB = CPW > 0 ? CPW : 1;
  uint32_t qoff[CPB];
  bool qis_w[CPB];
  int qbr[CPB];
  {
    int mrow[CPB], orw[CPB];
    bool v[CPB];
#pragma unroll
    for (int j = 0; j < CPB; ++j) {
      const int row = 8 * (pwave + PW * j) + (lane >> 3);
      mrow[j] = m0 + (DIRECT_W ? row - BN : row);   // token rows (unused for weight rows)
    }
    token_rows<MOE, CPB>(p, mrow, qbr, orw, v);
  }
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int q = pwave + PW * j;
    const int row = 8 * q + (lane >> 3);  // LDS row: weights first when copied directly
    if (DIRECT_W && row < BN) {
      const int r = min(wrow_of(row), p.N - 1);
      qoff[j] = (uint32_t)r * (uint32_t)p.ldw;
      qis_w[j] = true;
    } else {
      qoff[j] = (uint32_t)qbr[j] * (uint32_t)(p.lda * 2);
      qis_w[j] = false;
    }
    qoff[j] += 16 * ((lane & 7) ^ lds_swz(row + (DIRECT_W ? 0 : BN)));
  }
  if constexpr (MOE) {
    if (expert < 0) return;
  }
  const uint8_t* wbase = p.w + (int64_t)expert * p.w_es;
  // Decoded weight pieces of this thread: (LDS row, piece index within the row).
  int prow[PPT > 0 ? PPT : 1], pidx[PPT > 0 ? PPT : 1], pgrow[PPT > 0 ? PPT : 1];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int pi = min(ptid + T * j, PIECES - 1);  // surplus threads repeat the last piece (same bytes, same slot)
    prow[j] = pi / PPR;
    pidx[j] = pi % PPR;
    pgrow[j] = min(wrow_of(prow[j]), p.N - 1);
  }
  constexpr int PB = PPT > 0 ? PPT : 1;
  constexpr bool ZP = (FMT == kWInt4Zp);
  // Raw weights of one stage with their scale bits (and zero-point bytes).
  struct WBuf {
    u32x4 w[PB];
    uint32_t s[PB];
    uint32_t z[PB];
  };
  int64_t srow[PB], zrow[PB];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    srow[j] = wscale_row(p, expert, pgrow[j]);
    zrow[j] = ZP ? wzero_row(p, expert, pgrow[j]) : 0;
  }
  auto load_w = [&](int kb, WBuf& b) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int k = kb * 64 + pidx[j] * PV;
      b.w[j] = ldg128(wbase + (int64_t)pgrow[j] * p.ldw + (int64_t)k * BITS / 8);
      if constexpr (!DIRECT_W) b.s[j] = wscale_raw<FMT>(p, srow[j], k);
      if constexpr (ZP) b.z[j] = wzero_raw(p, zrow[j], k);
    }
  };
  auto copy_a = [&](int kb, int buf) {
    uint8_t* st = smem + buf * STAGE;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int q = pwave + PW * j;
      const uint8_t* base = qis_w[j] ? wbase + (int64_t)kb * 128 : reinterpret_cast<const uint8_t*>(p.a) + (int64_t)kb * 128;
      g2l_b128(base + qoff[j], st + (DIRECT_W ? q : q + BN / 8) * 1024);
    }
  };
  // One 16-byte raw piece with its scale bits and zero-point byte.
  struct WBuf1 {
    u32x4 w;
    uint32_t s, z;
  };
  auto decode_piece = [&](uint8_t* st, int j, const WBuf1& b) {
    const float sc = wscale_value<FMT>(p, b.s);
    const uint32_t zi = ZP ? ((pgrow[j] & 1) ? (b.z >> 4) : (b.z & 15)) : 8u;
    const float z = (float)zi;
    uint32_t v[PV / 2];
    constexpr int PAIRS_PER_DWORD = 32 / BITS / 2;
    if constexpr (FMT == kWInt4Zp || FMT == kWInt4Sym) {
      if (__builtin_fabsf(sc) <= 0x1p123f) {
        const uint32_t zb = (16u - zi) * 0x01010101u;
        const float c = -16.0f * sc;
#pragma unroll
        for (int i = 0; i < 4; ++i) int4_dword_fma<F16>(b.w[i], zb, sc, c, &v[4 * i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) decode_dword<FMT, F16>(b.w[i], sc, z, &v[i * PAIRS_PER_DWORD]);
      }
    } else if constexpr (FMT == kWMxfp4 && !F16) {
      if (scale_kind<FMT>(p) == kSE8m0 && mxfp4_cvt_ok(b.s)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) mxfp4_dword_cvt(b.w[i], b.s, &v[4 * i]);
      } else if (scale_kind<FMT>(p) == kSE8m0 && mxfp4_lut_ok(b.s)) {
        const Mxfp4Lut t = mxfp4_lut(b.s);
#pragma unroll
        for (int i = 0; i < 4; ++i) mxfp4_dword_lut(b.w[i], t, &v[4 * i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) decode_dword<FMT, F16>(b.w[i], sc, z, &v[i * PAIRS_PER_DWORD]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) decode_dword<FMT, F16>(b.w[i], sc, z, &v[i * PAIRS_PER_DWORD]);
    }
    const int row = prow[j];
#pragma unroll
    for (int c = 0; c < PV / 8; ++c) {
      const int chunk = pidx[j] * (PV / 8) + c;
      u32x4 o;
      o[0] = v[4 * c]; o[1] = v[4 * c + 1]; o[2] = v[4 * c + 2]; o[3] = v[4 * c + 3];
      *reinterpret_cast<u32x4*>(st + row * 128 + 16 * (chunk ^ lds_swz(row))) = o;
    }
  };
  auto decode_w = [&](int buf, const WBuf& b) {
    uint8_t* st = smem + buf * STAGE;
#pragma unroll
    for (int j = 0; j < PPT; ++j) decode_piece(st, j, WBuf1{b.w[j], b.s[j], b.z[j]});
  };

  // ---- RAWL copies. Raw copy c of a stage: rows 32c..32c+31, lane l takes
  // row 32c + l/2, bytes 16*(l&1) of its 32-byte stage slice (LDS slot order
  // is row-major, so lane l lands at 16*l of the copy's KiB). Every producer
  // wave also issues exactly one 4-byte-per-lane copy per stage: waves
  // 0..SQ-1 the scale words of rows 64w..64w+63, wave SQ the zero-point words
  // of row pairs 0..63 (int4 with zero points), the others repeat the last
  // of these (same bytes to the same place), so every producer wave counts
  // the same number of copies per stage.
  constexpr int RQPW = RAWL ? RQ / PW : 0;
  uint32_t roff[RQPW > 0 ? RQPW : 1];
#pragma unroll
  for (int j = 0; j < RQPW; ++j) {
    const int c = pwave + PW * j;
    const int row = 32 * c + (lane >> 1);
    roff[j] = (uint32_t)min(wrow_of(row), p.N - 1) * (uint32_t)p.ldw + 16u * (uint32_t)(lane & 1);
  }
  const int nxq = SQ + ZQ;
  const int xq = RAWL ? min(pwave, nxq - 1) : 0;     // this wave's 4-byte copy
  const bool x_is_z = ZPF && xq >= SQ;
  const int sbytes = scale_kind<FMT>(p) == kSF32 ? 4 : (scale_kind<FMT>(p) == kSE8m0 ? 1 : 2);
  int64_t xrow = 0;   // element index of the row's (pair's) first scale (zero point)
  if constexpr (RAWL) {
    if (x_is_z) {
      const int pr = 64 * (xq - SQ) + lane;           // LDS row pair
      xrow = wzero_row(p, expert, min(wrow_of(2 * min(pr, BN / 2 - 1)), p.N - 1));
    } else {
      const int row = 64 * xq + lane;
      xrow = wscale_row(p, expert, min(wrow_of(row), p.N - 1));
    }
  }
  // Byte address of the K-group element of stage kb for the 4-byte copy.
  auto x_addr = [&](int kb) -> const uint8_t* {
    if (x_is_z) return p.wz + xrow + (int64_t)((kb * 64) / p.ws_kgroup) * p.wz_ks;
    const int64_t idx = xrow + (int64_t)((kb * 64) / p.ws_kgroup) * p.ws_ks;
    return static_cast<const uint8_t*>(p.ws) + idx * sbytes;
  };
  auto dma_raw = [&](int kb, int slot) {
    uint8_t* rs = rawbase + slot * RAWSLOT;
    const uint8_t* wb = wbase + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < RQPW; ++j) {
      uint32_t o = roff[j];
      asm volatile("" : "+v"(o));
      g2l_b128(wb + o, rs + (pwave + PW * j) * 1024);
    }
    const uint8_t* a = x_addr(kb);
    const uint8_t* aw = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(a) & ~(uintptr_t)3);
    g2l_b32(aw, rs + (x_is_z ? RAW_Z + (xq - SQ) * 256 : RAW_S + xq * 256));
  };
  // A stage's raw pieces of this thread as read from its raw slot: packed
  // weights, scale word, zero-point word.
  struct RawRegs {
    u32x4 w[PB];
    uint32_t sw[PB], zw[PB];
  };
  auto read_raw = [&](int slot, RawRegs& r) {
    const uint8_t* rs = rawbase + slot * RAWSLOT;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      r.w[j] = lds128(rs + prow[j] * 32 + 16 * pidx[j]);
      r.sw[j] = *reinterpret_cast<const uint32_t*>(rs + RAW_S + 4 * prow[j]);
      r.zw[j] = ZPF ? *reinterpret_cast<const uint32_t*>(rs + RAW_Z + 4 * (prow[j] >> 1)) : 0u;
    }
  };
  // Decode of stage kb's raw pieces into LDS buffer buf (same pieces as decode_w).
  auto decode_regs = [&](int kb, const RawRegs& r, int buf) {
    uint8_t* st = smem + buf * STAGE;
    const int g = (kb * 64) / p.ws_kgroup;   // the stage's first K group
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      WBuf1 b;
      b.w = r.w[j];
      const uintptr_t sa = reinterpret_cast<uintptr_t>(p.ws) + (uintptr_t)((srow[j] + (int64_t)g * p.ws_ks) * sbytes);
      uint32_t sh = (uint32_t)(sa & 3u) * 8u;
      if constexpr (FMT == kWMxfp4) sh += 8u * (uint32_t)pidx[j];   // two 32-K groups per stage, bytes in a row
      b.s = sbytes == 4 ? r.sw[j] : (r.sw[j] >> sh) & (sbytes == 2 ? 0xffffu : 0xffu);
      b.z = 0;
      if constexpr (ZPF) {
        const uintptr_t za = reinterpret_cast<uintptr_t>(p.wz) + (uintptr_t)(zrow[j] + (int64_t)g * p.wz_ks);
        b.z = (r.zw[j] >> ((uint32_t)(za & 3u) * 8u)) & 0xffu;
      }
      decode_piece(st, j, b);
    }
  };

  int aidx[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    if constexpr (GATED) aidx[s] = s < NTH ? wn * NTH + s : SA / 2 + wn * NTH + (s - NTH);
    else aidx[s] = wn * NT + s;
  }
  const uint32_t frag0 = (uint32_t)r16 * 128 + 16 * ((g4) ^ lds_swz(r16));
  const uint32_t frag1 = (uint32_t)r16 * 128 + 16 * ((4 + g4) ^ lds_swz(r16));

  v4f acc[NT][MT];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[s][t] = v4f{0.f, 0.f, 0.f, 0.f};

  const int nkb = p.K >> 6;
  auto clampk = [&](int kb) { return kb < nkb ? kb : nkb - 1; };
  auto compute = [&](int kb) {
    const uint8_t* st = smem + (kb % STAGES) * STAGE;
    auto mma = [&](const u32x4& a, const u32x4& b, v4f& c) {
      if constexpr (F16) c = mfma_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c);
      else c = mfma_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c);
    };
    u32x4 af0[NT], af1[NT];
#pragma unroll
    for (int s = 0; s < NT; ++s) af0[s] = lds128(st + aidx[s] * 2048 + frag0);
#pragma unroll
    for (int step = 0; step < 2; ++step) {
      const uint32_t fo = step ? frag1 : frag0;
      u32x4 bq[3];
      bq[0] = lds128(st + (SA + wm * MT) * 2048 + fo);
      if (MT > 1) bq[1] = lds128(st + (SA + wm * MT + 1) * 2048 + fo);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if (t + 2 < MT) bq[(t + 2) % 3] = lds128(st + (SA + wm * MT + t + 2) * 2048 + fo);
        if (step == 0 && t == MT - 2) {
#pragma unroll
          for (int s = 0; s < NT; ++s) af1[s] = lds128(st + aidx[s] * 2048 + frag1);
        }
        if (!MOE || t < mt_live) {
#pragma unroll
          for (int s = 0; s < NT; ++s) mma(step ? af1[s] : af0[s], bq[t % 3], acc[s][t]);
        }
        // One scheduling region per token row: the read two rows ahead goes
        // out before this row's MFMAs, so each fragment has about seven MFMAs
        // of cover before its use (the compiler's own order waited on every
        // pair of reads right after issuing them; C4 T=2048 2-7 % faster,
        // bit-identical).
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // Iteration kb: copies of stage kb were issued at kb-2, followed by the raw
  // weights (and scale, zero-point loads) of kb+2 and the copies of kb+1.
  constexpr int LPW = DIRECT_W ? 0 : (RAWL ? RQPW + 1 : PPT * (2 + (ZP ? 1 : 0)));  // weight loads per stage
  if constexpr (RAWL) {
    // Iteration kb: stage kb's token copies and raw(kb+1) have landed; raw
    // copies run three stages ahead of their decode, token copies two ahead
    // of their use. int4 producers issue the copies of later stages before
    // decoding raw(kb+1) (config 5 2 % faster); MXFP4 producers, whose
    // decode is shorter, decode first (4 % faster than the other order, and
    // than starting the raw reads before the copies).
    RawRegs cur;
    if (is_prod) {
      dma_raw(0, 0);
      copy_a(0, 0);
      dma_raw(clampk(1), 1);
      copy_a(clampk(1), 1);
      dma_raw(clampk(2), 2);
      wait_vmcnt<2 * LPW + CPW>();   // raw(0) and tokens(0)
    }
    lds_barrier();
    if (is_prod) {
      read_raw(0, cur);
      decode_regs(0, cur, 0);
    }
    for (int kb = 0; kb < nkb; ++kb) {
      if (is_prod) wait_vmcnt<LPW + CPW>();   // raw(kb+1), tokens(kb)
      lds_barrier();
      if (is_prod) {
        constexpr bool COPIES_FIRST = (FMT == kWInt4Zp || FMT == kWInt4Sym);
        if constexpr (COPIES_FIRST) {
          dma_raw(clampk(kb + 3), (kb + 3) % 3);
          copy_a(clampk(kb + 2), (kb + 2) % STAGES);
        }
        read_raw((kb + 1) % 3, cur);
        decode_regs(clampk(kb + 1), cur, (kb + 1) % STAGES);
        if constexpr (!COPIES_FIRST) {
          dma_raw(clampk(kb + 3), (kb + 3) % 3);
          copy_a(clampk(kb + 2), (kb + 2) % STAGES);
        }
      }
      if (do_mma) compute(kb);
    }
  }
  auto body = [&](int kb, WBuf& wdec) {
    if (is_prod) {
      wait_vmcnt<LPW + CPW>();
      if constexpr (NP == 0) decode_w((kb + 1) % STAGES, wdec);
    }
    lds_barrier();
    if (is_prod) {
      if constexpr (NP > 0) decode_w((kb + 1) % STAGES, wdec);
      load_w(clampk(kb + 3), wdec);
      copy_a(clampk(kb + 2), (kb + 2) % STAGES);
    }
    if (do_mma) compute(kb);
  };
  if constexpr (!RAWL) {
    WBuf wA, wB;  // raw weights of even / odd stages
    if (is_prod) {
      load_w(0, wA);
      copy_a(0, 0);
      wait_vmcnt<0>();
      decode_w(0, wA);
      load_w(clampk(1), wB);
      copy_a(clampk(1), 1);
      load_w(clampk(2), wA);
    }
    int kb = 0;
    for (; kb + 1 < nkb; kb += 2) {
      body(kb, wB);
      body(kb + 1, wA);
    }
    if (kb < nkb) body(kb, wB);
  }
  // Copies of clamped stages may still be landing: none may outlive the block.
  wait_vmem();
  if (!is_cons) return;

  EpiRow elate[PRE ? 1 : MT];   // rows not loaded before the loop, as one batch here
  if constexpr (!PRE) {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) mrow[t] = m0 + wm * TM + 16 * t + r16;
    epi_rows<MOE, MT>(p, mrow, elate);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const EpiRow e = PRE ? erow[PRE ? t : 0] : elate[PRE ? 0 : t];
    const int orw = e.orow;
    if (!e.valid) continue;
#pragma unroll
    for (int so = 0; so < NTH; ++so) {
      float g[4], u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[i] = acc[so][t][i];
        u[i] = GATED ? acc[so + NTH][t][i] : 0.f;
      }
      const int col0 = GATED ? (tn * (BN / 2) + 16 * (wn * NTH + so) + 4 * g4) : (tn * BN + 16 * (wn * NT + so) + 4 * g4);
      if constexpr (!MOE && EPI == kEpiStore) {
        if (p.bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (col0 + i < p.n_out) {
              const uint32_t b = p.bias[(int64_t)orw * p.bias_rs + col0 + i];
              g[i] += p.out_f16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b);
            }
        }
      }
      finish_float4_tw<EPI, ACT, MOE>(p, orw, col0, g, u, e.tw);
    }
  }
}

// ============================================================ whole-matrix dequant
// out[n, k] = decode(w[n, k]) in bf16; one thread per 16-byte piece.
template <int FMT>
__global__ void __launch_bounds__(256) dequant_kernel(G16 p, uint16_t* out, int64_t ldo) {
  constexpr int BITS = FmtInfo<FMT>::bits;
  constexpr int PV = 128 / BITS;
  const int64_t pieces_per_row = p.K / PV;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.N * pieces_per_row) return;
  const int n = (int)(i / pieces_per_row);
  const int k = (int)(i % pieces_per_row) * PV;
  const u32x4 raw = ldg128(p.w + (int64_t)n * p.ldw + (int64_t)k * BITS / 8);
  const float sc = wscale(p, 0, n, k);
  const float z = (FMT == kWInt4Zp) ? wzero(p, 0, n, k) : 8.0f;
  uint32_t v[PV / 2];
  constexpr int PAIRS_PER_DWORD = 32 / BITS / 2;
  bool done = false;
  if constexpr (FMT == kWMxfp4) {
    const uint32_t b = p.ws_kind == kSE8m0 ? wscale_raw<FMT>(p, wscale_row(p, 0, n), k) : 1u;
    if (p.ws_kind == kSE8m0 && mxfp4_cvt_ok(b)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) mxfp4_dword_cvt(raw[j], b, &v[4 * j]);
      done = true;
    } else if (p.ws_kind == kSE8m0 && mxfp4_lut_ok(b)) {
      const Mxfp4Lut t = mxfp4_lut(b);
#pragma unroll
      for (int j = 0; j < 4; ++j) mxfp4_dword_lut(raw[j], t, &v[4 * j]);
      done = true;
    }
  }
  if (!done) {
#pragma unroll
    for (int j = 0; j < 4; ++j) decode_dword<FMT, false>(raw[j], sc, z, &v[j * PAIRS_PER_DWORD]);
  }
  uint16_t* o = out + (int64_t)n * ldo + k;
#pragma unroll
  for (int c = 0; c < PV / 8; ++c) {
    u32x4 q;
    q[0] = v[4 * c]; q[1] = v[4 * c + 1]; q[2] = v[4 * c + 2]; q[3] = v[4 * c + 3];
    *reinterpret_cast<u32x4*>(o + 8 * c) = q;
  }
}

// ============================================================ launchers
template <int FMT, int NT, int MT, int WAVES, bool MOE, int EPI, int ACT, bool F16>
int launch_stream16(const G16& p, int grid_y, hipStream_t st, const char* op) {
  constexpr int NTH = (EPI == kEpiGated) ? NT / 2 : NT;
  const int grid_x = (p.n_out + 16 * NTH - 1) / (16 * NTH);
  // int4 with one scale per 128-K chunk (or per row) and no 64-K tail: the folded decode.
  if constexpr (FMT == kWInt4Zp || FMT == kWInt4Sym) {
    if ((p.ws_kgroup == 128 || p.ws_kgroup == 0) && p.K % 128 == 0) {
      hipLaunchKernelGGL((stream16_kernel<FMT, NT, MT, WAVES, MOE, EPI, ACT, F16, true>), dim3(grid_x, grid_y),
                         dim3(WAVES * 64), 0, st, p);
      return check_launch(op);
    }
  }
  hipLaunchKernelGGL((stream16_kernel<FMT, NT, MT, WAVES, MOE, EPI, ACT, F16>), dim3(grid_x, grid_y), dim3(WAVES * 64), 0,
                     st, p);
  return check_launch(op);
}

template <int FMT, int BM, int BN, int WM, int WN, int NP, bool MOE, int EPI, int ACT, bool F16, bool RAWL>
int launch_tiled16_as(const G16& p, int grid_y_moe, hipStream_t st, const char* op) {
  constexpr int COLS = (EPI == kEpiGated) ? BN / 2 : BN;
  constexpr int THREADS = (WM * WN + NP) * 64;
  const int tiles_n = (p.n_out + COLS - 1) / COLS;
  if constexpr (MOE) {
    hipLaunchKernelGGL((tiled16_kernel<FMT, BM, BN, WM, WN, NP, MOE, EPI, ACT, F16, RAWL>), dim3(tiles_n, grid_y_moe),
                       dim3(THREADS), 0, st, p, 0, tiles_n, 0);
  } else {
    const int tiles_m = (p.M + BM - 1) / BM;
    hipLaunchKernelGGL((tiled16_kernel<FMT, BM, BN, WM, WN, NP, MOE, EPI, ACT, F16, RAWL>), dim3(tiles_m * tiles_n),
                       dim3(THREADS), 0, st, p, tiles_m, tiles_n, 8);
  }
  return check_launch(op);
}

// The raw-in-LDS producer path takes 4-bit weights whose per-stage scale
// (and zero point) of a row is one element of one 4-byte word: MXFP4 with
// e8m0 scales (two groups of 32 per 64-K stage, in adjacent bytes of a row
// with an even stride), or int4 with 64- or 128-element groups and 2- or
// 4-byte scales. It needs the three decoded stages plus three raw slots in
// LDS.
template <int FMT, int BM, int BN, int NP>
constexpr bool raw_lds_fits() {
  return FmtInfo<FMT>::bits == 4 && NP > 0 && FMT != kWInt4Ex && BN % 64 == 0 && (BN / 32) % NP == 0 &&
         BN / 64 + (BN + 127) / 128 <= NP && (BN + BM) * 128 * 3 + 3 * (BN * 36 + BN * 2) <= 160 * 1024;
}

template <int FMT, int BM, int BN, int NP>
bool raw_lds_ok(const G16& p) {
  if constexpr (!raw_lds_fits<FMT, BM, BN, NP>()) return false;
  else {
    if (FMT == kWMxfp4) return p.ws_kind == kSE8m0 && p.ws_kgroup == 32 && p.ws_ks == 1 && p.ws_ns % 2 == 0 &&
                               p.ws_es % 2 == 0 && (reinterpret_cast<uintptr_t>(p.ws) & 1u) == 0;
    if (p.ws_kgroup != 64 && p.ws_kgroup != 128) return false;
    const int sb = p.ws_kind == kSF32 ? 4 : 2;
    return (p.ws_kind == kSF32 || p.ws_kind == kSBf16 || p.ws_kind == kSF16) &&
           (reinterpret_cast<uintptr_t>(p.ws) % sb) == 0;
  }
}

template <int FMT, int BM, int BN, int WM, int WN, int NP, bool MOE, int EPI, int ACT, bool F16>
int launch_tiled16(const G16& p, int grid_y_moe, hipStream_t st, const char* op) {
  if constexpr (raw_lds_fits<FMT, BM, BN, NP>()) {
    if (raw_lds_ok<FMT, BM, BN, NP>(p))
      return launch_tiled16_as<FMT, BM, BN, WM, WN, NP, MOE, EPI, ACT, F16, true>(p, grid_y_moe, st, op);
  }
  return launch_tiled16_as<FMT, BM, BN, WM, WN, NP, MOE, EPI, ACT, F16, false>(p, grid_y_moe, st, op);
}

// ring16 takes int4 experts with bf16/fp16 scales per 128-K group (and zero
// points) laid out so that each step's two scale elements of a row, and the
// two zero-point bytes of a row pair, sit in one aligned 4-byte word; K a
// multiple of 256 and 16-byte aligned weight and token rows.
template <int FMT>
bool ring16_ok(const G16& p, int64_t a_rows) {
  if constexpr (FMT != kWInt4Zp && FMT != kWInt4Sym) return false;
  else {
    auto al = [](const void* q, uintptr_t a) { return (reinterpret_cast<uintptr_t>(q) % a) == 0; };
    bool ok = p.K % 256 == 0 && p.ws_kgroup == 128 && (p.ws_kind == kSBf16 || p.ws_kind == kSF16) &&
              p.ws_ks == 1 && p.ws_nblock == 1 && p.ws_ns % 2 == 0 && p.ws_es % 2 == 0 && al(p.ws, 4) &&
              p.ldw % 16 == 0 && p.w_es % 16 == 0 && al(p.w, 16) && (p.lda * 2) % 16 == 0 && al(p.a, 16) &&
              p.gate_off % 2 == 0 && p.N % 2 == 0 && (uint64_t)p.N * (uint64_t)p.ldw < (1ull << 32) &&
              (uint64_t)a_rows * (uint64_t)(p.lda * 2) < (1ull << 32);
    if (FMT == kWInt4Zp)
      ok = ok && p.wz_ks == 1 && p.wz_ns % 2 == 0 && p.wz_es % 2 == 0 && al(p.wz, 4);
    return ok;
  }
}

// Token rows per slot: a block holds at most min(16, tokens) routed rows
// (an expert takes each token once), and its routed rows come first.
template <int FMT, int EPI, int ACT, bool F16>
int launch_ring16(const G16& p, int num_blocks, hipStream_t st, const char* op) {
  constexpr int NTH = (EPI == kEpiGated) ? 1 : 2;
  const int grid_x = (p.n_out + 16 * NTH - 1) / (16 * NTH);
  const int64_t tokens = (p.num_slots + p.top_k - 1) / p.top_k;
  const int tq = tokens <= 2 ? 2 : (tokens <= 8 ? 8 : 16);
  const int64_t live = std::min<int64_t>(num_blocks, p.num_slots);
  const int steps = p.K / 256;
  // K-split waves: the most of 1..4 that leaves every wave a step and stays
  // within about six waves per CU.
  int ks = 1;
  for (int c : {2, 3, 4})
    if (c <= steps && (int64_t)grid_x * live * c <= 6 * cu_count()) ks = c;
  auto go = [&](auto tq_tag, auto ks_tag) {
    constexpr int TQ_ = decltype(tq_tag)::value;
    constexpr int KS_ = decltype(ks_tag)::value;
    hipLaunchKernelGGL((ring16_kernel<FMT, TQ_, KS_, 3, EPI, ACT, F16>), dim3(grid_x, num_blocks), dim3(64 * KS_), 0,
                       st, p);
  };
  auto with_ks = [&](auto tq_tag) {
    if (ks == 4) go(tq_tag, std::integral_constant<int, 4>{});
    else if (ks == 3) go(tq_tag, std::integral_constant<int, 3>{});
    else if (ks == 2) go(tq_tag, std::integral_constant<int, 2>{});
    else go(tq_tag, std::integral_constant<int, 1>{});
  };
  if (tq == 2) with_ks(std::integral_constant<int, 2>{});
  else if (tq == 8) with_ks(std::integral_constant<int, 8>{});
  else with_ks(std::integral_constant<int, 16>{});
  return check_launch(op);
}

template <int FMT, int EPI, int ACT, bool F16>
int moe16_dispatch(const G16& p, int block_m, int num_blocks, hipStream_t st, const char* op) {
  constexpr int NTS = (EPI == kEpiGated) ? 2 : 1;
  switch (block_m) {
    case 16: {
      // int4 with K of at least four 256-K steps: the LDS ring (C5's w13 at
      // T=1 11.3 -> 7.9 us). Shorter K stays on stream16 (C5's w2, K=768:
      // 5.8 us there against 7.0-7.5 on the ring).
      if constexpr (FMT == kWInt4Zp || FMT == kWInt4Sym) {
        if (p.ring16 && p.K >= 1024 && ring16_ok<FMT>(p, p.a_rows))
          return launch_ring16<FMT, EPI, ACT, F16>(p, num_blocks, st, op);
      }
      // Four K-split waves, or two when K holds fewer than 12 chunks (a
      // fourth wave would get none): C5's w2 (K=768, six chunks) 8.8 -> 7.0
      // us at T=1, 25.2 -> 20.6 us at T=8; longer K is faster with four
      // (and than with eight: C5's w13 at T=1 11.4 vs 12.7 us).
      constexpr int CK = 4 * (128 / FmtInfo<FMT>::bits);
      if ((p.K + CK - 1) / CK < 12) return launch_stream16<FMT, NTS, 1, 2, true, EPI, ACT, F16>(p, num_blocks, st, op);
      return launch_stream16<FMT, NTS, 1, 4, true, EPI, ACT, F16>(p, num_blocks, st, op);
    }
    case 32: return launch_stream16<FMT, NTS, 2, 4, true, EPI, ACT, F16>(p, num_blocks, st, op);
    case 64: return launch_tiled16<FMT, 64, 256, 1, 4, 4, true, EPI, ACT, F16>(p, num_blocks, st, op);
    case 128: return launch_tiled16<FMT, 128, 256, 2, 2, 4, true, EPI, ACT, F16>(p, num_blocks, st, op);
    case 256: return launch_tiled16<FMT, 256, 128, 2, 2, 4, true, EPI, ACT, F16>(p, num_blocks, st, op);
    default: return set_error(STRIX_ERR_INVALID, "%s: block_m must be 16, 32, 64, 128 or 256, got %d", op, block_m);
  }
}

template <int FMT, bool F16>
int dense16_dispatch(const G16& p, hipStream_t st, const char* op, int cfg) {
  const int M = p.M;
  if (cfg < 0) cfg = M <= 16 ? 0 : (M <= 32 ? 1 : (M <= 64 ? 2 : 3));
  switch (cfg) {
    // Two waves split K: fewer, longer waves stream better than eight (M=1
    // MXFP4 17408x5120: 32.0 -> 26.0 us; FP8 W8A16: 27.5 -> 24.0 us; on
    // narrow N, 5760x2880 and 2048x7168, eight are no faster).
    case 0: return launch_stream16<FMT, 1, 1, 2, false, kEpiStore, kActSilu, F16>(p, (M + 15) / 16, st, op);
    case 1: return launch_stream16<FMT, 1, 2, 2, false, kEpiStore, kActSilu, F16>(p, (M + 31) / 32, st, op);
    case 2: return launch_stream16<FMT, 1, 4, 4, false, kEpiStore, kActSilu, F16>(p, (M + 63) / 64, st, op);
    case 3: return launch_tiled16<FMT, 128, 256, 2, 2, 4, false, kEpiStore, kActSilu, F16>(p, 0, st, op);
    case 4: return launch_tiled16<FMT, 256, 128, 2, 2, 4, false, kEpiStore, kActSilu, F16>(p, 0, st, op);
    case 5: return launch_tiled16<FMT, 64, 256, 1, 4, 4, false, kEpiStore, kActSilu, F16>(p, 0, st, op);
    // Sweep points: every wave decodes and computes.
    case 6: return launch_tiled16<FMT, 128, 256, 2, 4, 0, false, kEpiStore, kActSilu, F16>(p, 0, st, op);
    case 7: return launch_tiled16<FMT, 128, 128, 2, 2, 0, false, kEpiStore, kActSilu, F16>(p, 0, st, op);
    default: return set_error(STRIX_ERR_INVALID, "%s: cfg must be in 0..7, got %d", op, cfg);
  }
}

// ------------------------------------------------------------ argument checks
int check_scale_kind(const char* op, int kind) {
  STRIX_REQUIRE(kind >= kSF32 && kind <= kSE8m0, "%s: unknown scale dtype code %d", op, kind);
  return STRIX_OK;
}

struct MoeArgs {
  void* c; int64_t ldc; int c_dtype;
  const void* a; int64_t lda; int a_dtype;
  const int32_t* sorted_ids; int64_t sorted_len; const int32_t* expert_ids; int64_t num_blocks;
  const int32_t* num_post; const float* topk_w; int64_t num_slots; int64_t top_k; int64_t block_m;
  int silu_mul; int activation; int64_t N; int64_t K;
};

template <int FMT>
int run_moe16(const char* op, const MoeArgs& m, G16 p, void* stream) {
  STRIX_REQUIRE(m.a_dtype == STRIX_BF16 || m.a_dtype == STRIX_F16, "%s: activations must be bfloat16 or float16", op);
  STRIX_REQUIRE(m.c_dtype == STRIX_BF16 || m.c_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(m.K % 64 == 0, "%s: K must be a multiple of 64, got K=%lld", op, (long long)m.K);
  STRIX_REQUIRE(m.N % 16 == 0 && (!m.silu_mul || m.N % 32 == 0), "%s: N must be a multiple of 16 (32 when gated)", op);
  STRIX_REQUIRE(m.top_k >= 1, "%s: top_k must be >= 1", op);
  STRIX_REQUIRE(m.num_blocks * m.block_m >= m.sorted_len, "%s: expert_ids.numel() * block_m must cover sorted_ids", op);
  STRIX_REQUIRE(m.lda >= m.K && m.lda % 8 == 0 && aligned(m.a, 16), "%s: activation rows must be >= K, 16-byte aligned", op);
  const int64_t n_out = m.silu_mul ? m.N / 2 : m.N;
  STRIX_REQUIRE(m.ldc >= n_out && m.ldc % 4 == 0 && aligned(m.c, 8), "%s: output rows must be >= %lld, 8-byte aligned", op,
                (long long)n_out);
  STRIX_REQUIRE(m.activation == kActSilu || m.activation == kActGeluTanh, "%s: unknown activation", op);
  STRIX_REQUIRE(aligned(p.w, 16) && p.ldw % 16 == 0, "%s: weight rows must be 16-byte aligned", op);
  STRIX_REQUIRE(m.num_slots <= INT32_MAX && m.N <= INT32_MAX && m.K <= INT32_MAX, "%s: sizes overflow 32-bit indexing",
                op);
  STRIX_REQUIRE(fits_u32_rows(m.num_slots, m.lda * 2, m.K * 2) && fits_u32_rows(m.N, p.ldw, p.ldw),
                "%s: an operand spans more than 4 GiB (the kernels use 32-bit row offsets); split the call", op);
  int rc = check_scale_kind(op, p.ws_kind);
  if (rc) return rc;
  if (m.num_blocks == 0 || m.sorted_len == 0 || m.num_slots == 0 || m.N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  p.a = static_cast<const uint16_t*>(m.a); p.lda = m.lda;
  p.out = m.c; p.ldo = m.ldc; p.out_f16 = m.c_dtype == STRIX_F16;
  p.M = (int)m.num_slots; p.N = (int)m.N; p.K = (int)m.K; p.n_out = (int)n_out; p.gate_off = (int)(m.N / 2);
  p.sorted_ids = m.sorted_ids; p.sorted_len = m.sorted_len; p.expert_ids = m.expert_ids; p.num_post = m.num_post;
  p.num_slots = (int)m.num_slots; p.top_k = (int)m.top_k; p.topk_w = m.topk_w;
  p.a_rows = m.num_slots; p.ring16 = 1;
  hipStream_t st = as_stream(stream);
  const int nb = (int)m.num_blocks, bm = (int)m.block_m;
  const bool f16 = m.a_dtype == STRIX_F16;
  if (m.silu_mul) {
    if (m.activation == kActGeluTanh)
      return f16 ? moe16_dispatch<FMT, kEpiGated, kActGeluTanh, true>(p, bm, nb, st, op)
                 : moe16_dispatch<FMT, kEpiGated, kActGeluTanh, false>(p, bm, nb, st, op);
    return f16 ? moe16_dispatch<FMT, kEpiGated, kActSilu, true>(p, bm, nb, st, op)
               : moe16_dispatch<FMT, kEpiGated, kActSilu, false>(p, bm, nb, st, op);
  }
  return f16 ? moe16_dispatch<FMT, kEpiStore, kActSilu, true>(p, bm, nb, st, op)
             : moe16_dispatch<FMT, kEpiStore, kActSilu, false>(p, bm, nb, st, op);
}

template <int FMT>
int run_dense16(const char* op, G16 p, const void* x, int x_dtype, int64_t ldx, void* out, int64_t ldo, int out_dtype,
                int64_t M, int64_t N, int64_t K, int cfg, void* stream) {
  STRIX_REQUIRE(x_dtype == STRIX_BF16 || x_dtype == STRIX_F16, "%s: activations must be bfloat16 or float16", op);
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size", op);
  STRIX_REQUIRE(ldx >= K && ldx % 8 == 0 && aligned(x, 16), "%s: activation rows must be >= K, 16-byte aligned", op);
  STRIX_REQUIRE(ldo >= N && ldo % 4 == 0 && aligned(out, 8), "%s: output rows must be >= N, 8-byte aligned", op);
  STRIX_REQUIRE(aligned(p.w, 16) && p.ldw % 16 == 0, "%s: weight rows must be 16-byte aligned", op);
  STRIX_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, "%s: sizes overflow 32-bit indexing", op);
  STRIX_REQUIRE(fits_u32_rows(M, ldx * 2, K * 2) && fits_u32_rows(N, p.ldw, p.ldw),
                "%s: an operand spans more than 4 GiB (the kernels use 32-bit row offsets); split the call", op);
  int rc = check_scale_kind(op, p.ws_kind);
  if (rc) return rc;
  if (M == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  p.a = static_cast<const uint16_t*>(x); p.lda = ldx;
  p.out = out; p.ldo = ldo; p.out_f16 = out_dtype == STRIX_F16;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.n_out = (int)N;
  hipStream_t st = as_stream(stream);
  return x_dtype == STRIX_F16 ? dense16_dispatch<FMT, true>(p, st, op, cfg) : dense16_dispatch<FMT, false>(p, st, op, cfg);
}

G16 g16_weights(const void* w, int64_t w_es, int64_t ldw, const void* s, int s_kind, int64_t s_es, int64_t s_ns,
                int64_t s_ks, int kgroup, int nblock) {
  G16 p = {};
  p.w = static_cast<const uint8_t*>(w); p.w_es = w_es; p.ldw = ldw;
  p.ws = s; p.ws_kind = s_kind; p.ws_es = s_es; p.ws_ns = s_ns; p.ws_ks = s_ks; p.ws_kgroup = kgroup;
  p.ws_nblock = nblock;
  return p;
}

}  // namespace
}  // namespace strix

using namespace strix;

extern "C" {

#define STRIX_MOE16_ARGS STRIX_MOE16_PARAMS
#define STRIX_MOE16_PACK                                                                                            \
  MoeArgs m{c, ldc, c_dtype, a, lda, a_dtype, sorted_ids, sorted_len, expert_ids, num_blocks, num_post, topk_weights, \
            num_slots, top_k, block_m, silu_mul, activation, N, K}

int strix_moe_gemm_mxfp4(const uint8_t* w, int64_t w_es, int64_t ldw, const uint8_t* scales, int64_t s_es, int64_t s_ns,
                         STRIX_MOE16_ARGS) {
  STRIX_MOE16_PACK;
  const char* op = "moe_gemm_mxfp4";
  STRIX_REQUIRE(ldw * 2 >= K, "%s: weight rows must hold K/2 bytes", op);
  return run_moe16<kWMxfp4>(op, m, g16_weights(w, w_es, ldw, scales, kSE8m0, s_es, s_ns, 1, 32, 1), stream);
}

int strix_moe_gemm_w4a16_zp(const uint8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind, int64_t s_es,
                            int64_t s_ns, const uint8_t* zeros, int64_t z_es, int64_t z_ns, int64_t group,
                            STRIX_MOE16_ARGS) {
  STRIX_MOE16_PACK;
  const char* op = "moe_gemm_w4a16_zp";
  STRIX_REQUIRE(group == 32 || group == 64 || group == 128, "%s: group_size must be 32, 64 or 128", op);
  STRIX_REQUIRE(K % group == 0, "%s: K must be a multiple of group_size", op);
  STRIX_REQUIRE(s_kind == kSBf16 || s_kind == kSF16 || s_kind == kSF32, "%s: scales must be bf16, fp16 or fp32", op);
  G16 p = g16_weights(w, w_es, ldw, scales, s_kind, s_es, s_ns, 1, (int)group, 1);
  p.wz = zeros; p.wz_es = z_es; p.wz_ns = z_ns; p.wz_ks = 1;
  return run_moe16<kWInt4Zp>(op, m, p, stream);
}

int strix_moe_gemm_w4a16(const uint8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind, int64_t s_es,
                         int64_t s_ns, int64_t group, STRIX_MOE16_ARGS) {
  STRIX_MOE16_PACK;
  const char* op = "moe_gemm_w4a16";
  STRIX_REQUIRE(group == 32 || group == 64 || group == 128, "%s: group_size must be 32, 64 or 128", op);
  STRIX_REQUIRE(s_kind == kSBf16 || s_kind == kSF16 || s_kind == kSF32, "%s: scales must be bf16, fp16 or fp32", op);
  return run_moe16<kWInt4Sym>(op, m, g16_weights(w, w_es, ldw, scales, s_kind, s_es, s_ns, 1, (int)group, 1), stream);
}

int strix_moe_gemm_bf16(const uint16_t* w, int64_t w_es, int64_t ldw, STRIX_MOE16_ARGS) {
  STRIX_MOE16_PACK;
  // ldw in elements for the bf16 layout; the kernels use byte strides.
  return run_moe16<kWBf16>("moe_gemm_bf16", m, g16_weights(w, w_es * 2, ldw * 2, nullptr, kSF32, 0, 0, 0, 0, 1), stream);
}

// fp8 weights, W8A16: block scales [E][N/128][K/128] (nblock 128, kgroup 128) or per channel [E][N] (kgroup 0).
int strix_moe_gemm_fp8_w8a16(const uint8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind, int64_t s_es,
                             int64_t s_ns, int64_t s_ks, int block_scales, STRIX_MOE16_ARGS) {
  STRIX_MOE16_PACK;
  const char* op = "moe_gemm_fp8";
  STRIX_REQUIRE(!block_scales || (K % 128 == 0), "%s: K must be a multiple of 128 with block scales", op);
  G16 p = block_scales ? g16_weights(w, w_es, ldw, scales, s_kind, s_es, s_ns, s_ks, 128, 128)
                       : g16_weights(w, w_es, ldw, scales, s_kind, s_es, s_ns, 0, 0, 1);
  return run_moe16<kWFp8>(op, m, p, stream);
}

int strix_moe_gemm_w8a16(const int8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind, int64_t s_es,
                         int64_t s_ns, STRIX_MOE16_ARGS) {
  STRIX_MOE16_PACK;
  return run_moe16<kWInt8>("moe_gemm_w8a16", m, g16_weights(w, w_es, ldw, scales, s_kind, s_es, s_ns, 0, 0, 1), stream);
}

// Dense MXFP4 W4A16 (mxfp4_wmma_gemm): w [N, ldw >= K/2] u8, scales e8m0 [N, s_ld], bias (may be NULL).
int strix_mxfp4_gemm(const uint8_t* w, int64_t ldw, const uint8_t* scales, int64_t s_ld, const void* x, int x_dtype,
                     int64_t ldx, const void* bias, int64_t bias_rs, void* out, int64_t ldo, int out_dtype, int64_t M,
                     int64_t N, int64_t K, int cfg, void* stream) {
  const char* op = "mxfp4_wmma_gemm";
  STRIX_REQUIRE(K % 64 == 0, "%s: K must be a multiple of 64, got K=%lld", op, (long long)K);
  G16 p = g16_weights(w, 0, ldw, scales, kSE8m0, 0, s_ld, 1, 32, 1);
  p.bias = static_cast<const uint16_t*>(bias);
  p.bias_rs = bias_rs;
  return run_dense16<kWMxfp4>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
}

// Dense FP8 W8A16 (fp8_wmma_gemm / _raw): bf16 or fp16 activations, block or channel scales.
int strix_fp8_w8a16_gemm(const uint8_t* w, int64_t ldw, const float* scales, int64_t s_ld, int block_scales,
                         const void* x, int x_dtype, int64_t ldx, void* out, int64_t ldo, int out_dtype, int64_t M,
                         int64_t N, int64_t K, int cfg, void* stream) {
  const char* op = "fp8_wmma_gemm";
  STRIX_REQUIRE(K % 64 == 0, "%s: K must be a multiple of 64, got K=%lld", op, (long long)K);
  STRIX_REQUIRE(!block_scales || K % 128 == 0, "%s: K must be a multiple of 128 with block scales", op);
  G16 p = block_scales ? g16_weights(w, 0, ldw, scales, kSF32, 0, s_ld, 1, 128, 128)
                       : g16_weights(w, 0, ldw, scales, kSF32, 0, 1, 0, 0, 1);
  return run_dense16<kWFp8>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
}

// Dense weight-only GEMM over any packed weight format: out[m, n] =
// sum_k x[m, k] * decode(w[n, k]) (+ bias), scale of (n, k) at
// scales[(n / nblock) * s_ns + (k / kgroup) * s_ks] (kgroup 0: one per row group).
int strix_w16_gemm(int fmt, const uint8_t* w, int64_t ldw, const void* scales, int s_kind, int64_t s_ns,
                   int64_t s_ks, int64_t kgroup, int64_t nblock, const void* x, int x_dtype, int64_t ldx,
                   const void* bias, int64_t bias_rs, void* out, int64_t ldo, int out_dtype, int64_t M, int64_t N,
                   int64_t K, int cfg, void* stream) {
  const char* op = "w16_gemm";
  STRIX_REQUIRE(fmt == kWMxfp4 || fmt == kWInt4Sym || fmt == kWFp8 || fmt == kWInt8 || fmt == kWInt4Ex ||
                    fmt == kWU8b128,
                "%s: unsupported weight format %d", op, fmt);
  STRIX_REQUIRE(K % 64 == 0, "%s: K must be a multiple of 64, got K=%lld", op, (long long)K);
  const int piece = (fmt == kWFp8 || fmt == kWInt8 || fmt == kWU8b128) ? 16 : 32;  // K values sharing a scale read
  STRIX_REQUIRE(kgroup >= 0 && (kgroup == 0 || (kgroup % piece == 0 && K % kgroup == 0)),
                "%s: scale group (%lld) must be 0 or a multiple of %d dividing K", op, (long long)kgroup, piece);
  STRIX_REQUIRE(nblock >= 1, "%s: rows per scale row must be >= 1", op);
  G16 p = g16_weights(w, 0, ldw, scales, s_kind, 0, s_ns, s_ks, (int)kgroup, (int)nblock);
  p.bias = static_cast<const uint16_t*>(bias);
  p.bias_rs = bias_rs;
  switch (fmt) {
    case kWMxfp4: return run_dense16<kWMxfp4>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
    case kWInt4Sym: return run_dense16<kWInt4Sym>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
    case kWFp8: return run_dense16<kWFp8>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
    case kWInt8: return run_dense16<kWInt8>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
    case kWInt4Ex: return run_dense16<kWInt4Ex>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
    default: return run_dense16<kWU8b128>(op, p, x, x_dtype, ldx, out, ldo, out_dtype, M, N, K, cfg, stream);
  }
}

// Whole-matrix dequant to bf16: fmt 1 MXFP4 (e8m0 scales [N, s_ld]), 4 FP8 (block
// scales [N/128, s_ld] or channel [N]), 3 INT4 symmetric plain nibbles (group g, scales [N, s_ld]).
int strix_dequant_bf16(int fmt, const uint8_t* w, int64_t ldw, const void* scales, int s_kind, int64_t s_ld,
                       int64_t kgroup, int64_t nblock, uint16_t* out, int64_t ldo, int64_t N, int64_t K, void* stream) {
  const char* op = fmt == kWMxfp4 ? "mxfp4_dequant" : (fmt == kWFp8 ? "fp8_dequant" : "w4a16_dequant");
  STRIX_REQUIRE(fmt == kWMxfp4 || fmt == kWFp8 || fmt == kWInt4Sym || fmt == kWInt4Ex || fmt == kWInt8 ||
                    fmt == kWU8b128,
                "%s: unsupported format %d", op, fmt);
  const int bits = (fmt == kWFp8 || fmt == kWInt8 || fmt == kWU8b128) ? 8 : 4;
  const int pv = 128 / bits;
  STRIX_REQUIRE(K % pv == 0, "%s: K must be a multiple of %d", op, pv);
  STRIX_REQUIRE(aligned(w, 16) && ldw % 16 == 0 && aligned(out, 16) && ldo % 8 == 0, "%s: rows must be 16-byte aligned", op);
  int rc = check_scale_kind(op, s_kind);
  if (rc) return rc;
  if (N == 0 || K == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G16 p = g16_weights(w, 0, ldw, scales, s_kind, 0, s_ld, 1, (int)kgroup, (int)nblock);
  if (kgroup == 0) p.ws_ns = s_ld;  // per-channel: one scale per row (s_ld = stride between rows)
  p.N = (int)N;
  p.K = (int)K;
  const int64_t pieces = N * (K / pv);
  const unsigned blocks = (unsigned)((pieces + 255) / 256);
  hipStream_t st = as_stream(stream);
  switch (fmt) {
    case kWMxfp4: hipLaunchKernelGGL(dequant_kernel<kWMxfp4>, dim3(blocks), dim3(256), 0, st, p, out, ldo); break;
    case kWFp8: hipLaunchKernelGGL(dequant_kernel<kWFp8>, dim3(blocks), dim3(256), 0, st, p, out, ldo); break;
    case kWInt4Ex: hipLaunchKernelGGL(dequant_kernel<kWInt4Ex>, dim3(blocks), dim3(256), 0, st, p, out, ldo); break;
    case kWInt8: hipLaunchKernelGGL(dequant_kernel<kWInt8>, dim3(blocks), dim3(256), 0, st, p, out, ldo); break;
    case kWU8b128: hipLaunchKernelGGL(dequant_kernel<kWU8b128>, dim3(blocks), dim3(256), 0, st, p, out, ldo); break;
    default: hipLaunchKernelGGL(dequant_kernel<kWInt4Sym>, dim3(blocks), dim3(256), 0, st, p, out, ldo); break;
  }
  return check_launch(op);
}

}  // extern "C"
