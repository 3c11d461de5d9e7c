// SPDX-License-Identifier: MIT
// 8-bit MFMA GEMMs for gfx950: FP8-block W8A8 (e4m3 x e4m3 16x16x128 MFMA,
// fp32 fold per 128-K block), INT8 per-token W8A8 (i8 x i8 16x16x64 MFMA,
// exact int32 accumulator) and INT8 per-128-group W8A8 (int32 partial per
// group folded into fp32). Dense and MoE (grouped over aligned sorted ids).
//
// Math (reference: csrc/gemm/w8a8_wmma_gemm.hip:15-32 for the group fold,
// csrc/moe/moe_gemm_w8a16.hip:76-404 for the grouped MoE contract):
//   FP8 block   out[m,n] = sum_kb sa[m,kb] * sw[n/128,kb] * sum_{k in kb} qa[m,k] qw[n,k]
//   I8 token    out[m,n] = bf16((float(sum_k qa[m,k] qw[n,k]) * sa[m]) * sw[n])
//   I8 group    out[m,n] = sum_g float(sum_{k in g} qa qw) * (sw[n,g] * sa[m,g])
//
// Two kernel shapes:
//   stream8: no LDS staging. A wave owns NT 16-row weight subtiles and MT
//            16-token subtiles; the waves of a block split K and reduce
//            through LDS. Weights are streamed from HBM exactly once, 16 rows
//            x 64 contiguous bytes per load instruction. Decode (M <= 64) and
//            MoE blocks of 16-64 sorted ids.
//   tiled8:  BM x BN block tile, direct global->LDS copies (no register
//            staging) into a fragment-native layout, two LDS stages of 128 K,
//            conflict-free ds_read_b128 fragment reads. Prefill.
#include <algorithm>
#include <cmath>
#include <utility>

#include "capi_internal.h"
#include "gemm_common.h"
#include "strix_common.h"

namespace strix {
namespace {

enum Kind8 : int { kFp8Block = 0, kI8Token = 1, kI8Group = 2 };

struct G8 {
  const uint8_t* w;  // weight bytes: row n, K block kb at n * ldw + kb * w_kbs
  int64_t ldw, w_es;
  int64_t w_kbs = 128;  // row-major [E][N][ldw]: 128; K-block-major [E][K/128][N][128]: 128 * N
  const float* sw;   // fp8: [E][ceil(N/128)][K/128]; i8: [E][N][G] (G may be 1)
  int64_t sw_es, sw_ns, sw_ks;
  const uint8_t* a;  // activation bytes [rows][lda]
  int64_t lda;
  const float* sa;   // [rows][K/128] (i8 token: [rows], sa_ks = 0)
  int64_t sa_rs, sa_ks;
  void* out;
  int64_t ldo;
  int out_f16;
  int M, N, K;       // dense rows, weight rows per expert, K
  int n_out;         // output columns (N, or N/2 when gated)
  int gate_off;      // gated: first up row (= N/2)
  const int32_t* sorted_ids;
  int64_t sorted_len;
  const int32_t* expert_ids;
  const int32_t* num_post;
  int num_slots, top_k;
  const float* topk_w;
};

__device__ __forceinline__ v8i flip80(const v8i& x) {
  v8i r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = x[i] ^ (int)0x80808080u;
  return r;
}

// Final epilogue for one output subtile: `g` holds the (gate) values, `u` the
// up values when gated. I8 token values arrive as int32 bit patterns and are
// scaled here: (acc * sa[m]) * sw[n].
template <int KIND, int EPI, int ACT, bool MOE>
__device__ __forceinline__ void finish4_tw(const G8& p, int orow, int brow, bool valid, int col0,
                                           const float g[4], const float u[4], float tw) {
  if (!valid) return;
  if constexpr (EPI == kEpiI32) {
    int iv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) iv[i] = __float_as_int(g[i]);
    store4_i32(p, orow, col0, iv);
    return;
  }
  if constexpr (KIND == kI8Token) {
    const float sa = p.sa[(int64_t)brow * p.sa_rs];
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = min(col0 + i, p.N - 1);
      v[i] = ((float)__float_as_int(g[i]) * sa) * p.sw[(int64_t)n * p.sw_ns];
    }
    finish_float4_tw<kEpiStore, ACT, MOE>(p, orow, col0, v, u, tw);
  } else {
    finish_float4_tw<EPI, ACT, MOE>(p, orow, col0, g, u, tw);
  }
}
template <int KIND, int EPI, int ACT, bool MOE>
__device__ __forceinline__ void finish4(const G8& p, int orow, int brow, bool valid, int col0,
                                        const float g[4], const float u[4]) {
  const float tw = (MOE && valid && p.topk_w) ? p.topk_w[orow] : 1.f;
  finish4_tw<KIND, EPI, ACT, MOE>(p, orow, brow, valid, col0, g, u, tw);
}

// ============================================================ stream8
// Decode-shaped GEMM straight from global memory into MFMA registers.
// A block is 4 waves: NS = 4/KS groups of NT 16-row weight subtiles, each
// group's K range split over KS waves (reduced through LDS). Each wave
// streams its K range with a double-buffered register pipeline: the loads of
// batch j+1 (U K-steps of weights, tokens and scales) are in flight while
// batch j runs its MFMAs, so a wave keeps U..2U K-steps outstanding for its
// whole life. Waves are independent streams, so the grid needs no rounds:
// with KS = 1 every 16-row subtile is one long-lived wave.
template <int NT, int MT>
struct Frag8 {
  v8i af[NT];
  v8i bf[MT];
  float sw[NT][4];
  float sa[MT];
};

template <int KIND, int NT, int MT, int KS, bool MOE, int EPI, int ACT, int U, bool WX128, bool TOKL>
__global__ void __launch_bounds__(256) stream8_kernel(G8 p) {
  static_assert(!TOKL || MT == 1, "LDS token staging holds one 16-row token subtile");
  constexpr int NS = 4 / KS;
  static_assert(NS * KS == 4, "4 waves per block");
  constexpr int NTH = (EPI == kEpiGated) ? NT / 2 : NT;  // output subtiles
  constexpr bool INT_ACC = (KIND == kI8Token);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = wave % KS, ns = wave / KS;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int m0 = blockIdx.y * (16 * MT);
  int expert = 0;
  if constexpr (MOE) {
    expert = moe_block_expert(p.num_post, p.expert_ids, m0);
    if (expert < 0) return;
  }
  const int nout0 = (blockIdx.x * NS + ns) * (16 * NTH);
  const bool has_cols = nout0 < p.n_out;  // waves past the last subtile still take part in the reduction

  int wrow0[NT];  // first weight row of each subtile
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    if constexpr (EPI == kEpiGated)
      wrow0[s] = s < NTH ? nout0 + 16 * s : p.gate_off + nout0 + 16 * (s - NTH);
    else
      wrow0[s] = nout0 + 16 * s;
  }
  const uint8_t* wbase = p.w + (int64_t)expert * p.w_es;
  const uint8_t* wp[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    const int r = min(wrow0[s] + r16, p.N - 1);
    wp[s] = wbase + (int64_t)r * p.ldw + 16 * g4;
  }
  int brow[MT], orow[MT];
  bool bval[MT];
  const uint8_t* ap[MT];
  const float* sap[MT];
  {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) mrow[t] = m0 + 16 * t + r16;
    token_rows<MOE, MT>(p, mrow, brow, orow, bval);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    ap[t] = p.a + (int64_t)brow[t] * p.lda + 16 * g4;
    sap[t] = p.sa + (int64_t)brow[t] * p.sa_rs;
  }
  const float* swb = p.sw + (int64_t)expert * p.sw_es;
  const float* swp[NT][4];  // weight-scale row pointers (fp8: one per subtile; int8 group: per lane row)
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // fp8: one scale per 128-row block; the subtile's 16 rows share it, but
      // the per-lane row keeps it a vector load (a scalar load here would be
      // waited for as soon as it is issued).
      if constexpr (KIND == kFp8Block)
        swp[s][i] = swb + (int64_t)(min(wrow0[s] + r16, p.N - 1) >> 7) * p.sw_ns;
      else
        swp[s][i] = swb + (int64_t)min(wrow0[s] + 4 * g4 + i, p.N - 1) * p.sw_ns;
    }

  const int nks = p.K >> 7;
  const int per = (nks + KS - 1) / KS;
  const int kb0 = min(nks, ks * per), kb1 = min(nks, kb0 + per);

  v4f acc[NT][MT];
  v4i acci[NT][MT];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      acc[s][t] = v4f{0.f, 0.f, 0.f, 0.f};
      acci[s][t] = v4i{0, 0, 0, 0};
    }

  // TOKL: the block's 16 token rows live in LDS for the whole K ([row][K]
  // bytes, 16-byte chunks XOR-swizzled by row inside each 128-byte group so
  // the fragment reads of 16 rows hit distinct banks); the register pipeline
  // then carries weights and scales only.
  extern __shared__ __attribute__((aligned(16))) uint8_t tok[];
  const int tok_rows = MOE ? 16 : min(16, p.M - m0);  // rows staged (dense: the valid ones)
  const int tok_r = r16 < tok_rows ? r16 : 0;           // row a lane reads
  const uint8_t* tok_lane = tok + (int64_t)tok_r * p.K;

  using F = Frag8<NT, MT>;
  auto load = [&](int kb, F& f) {
    const int64_t ko = (int64_t)kb * 128, kw = (int64_t)kb * p.w_kbs;
#pragma unroll
    for (int s = 0; s < NT; ++s) f.af[s] = cat8(ldg128(wp[s] + kw), ldg128(wp[s] + kw + 64));
    if constexpr (!TOKL) {
#pragma unroll
      for (int t = 0; t < MT; ++t) f.bf[t] = cat8(ldg128(ap[t] + ko), ldg128(ap[t] + ko + 64));
    }
    if constexpr (KIND != kI8Token) {
#pragma unroll
      for (int t = 0; t < MT; ++t) f.sa[t] = sap[t][(int64_t)kb * p.sa_ks];
#pragma unroll
      for (int s = 0; s < NT; ++s)
#pragma unroll
        for (int i = 0; i < (KIND == kFp8Block ? 1 : 4); ++i) f.sw[s][i] = swp[s][i][(int64_t)kb * p.sw_ks];
    }
  };
  auto step = [&](int kb, F& f) {
    if constexpr (TOKL) {
      const uint8_t* base = tok_lane + kb * 128;
      f.bf[0] = cat8(lds128(base + 16 * (g4 ^ (tok_r & 7))), lds128(base + 16 * ((4 + g4) ^ (tok_r & 7))));
    }
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      v8i af = f.af[s];
      if constexpr (WX128) af = flip80(af);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if constexpr (KIND == kFp8Block) {
          const v4f part = mfma_fp8(af, f.bf[t], v4f{0.f, 0.f, 0.f, 0.f});
          const float c = f.sw[s][0] * f.sa[t];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[s][t][i] = fmaf(part[i], c, acc[s][t][i]);
        } else if constexpr (KIND == kI8Token) {
          acci[s][t] = mfma_i8(lo4(af), lo4(f.bf[t]), acci[s][t]);
          acci[s][t] = mfma_i8(hi4(af), hi4(f.bf[t]), acci[s][t]);
        } else {
          v4i part = mfma_i8(lo4(af), lo4(f.bf[t]), v4i{0, 0, 0, 0});
          part = mfma_i8(hi4(af), hi4(f.bf[t]), part);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[s][t][i] = fmaf((float)part[i], f.sw[s][i] * f.sa[t], acc[s][t][i]);
        }
      }
    }
  };

  // Double-buffered batches, unrolled by two so the buffers never move. No
  // load sits under a branch that skips it on one path: a join of "issued"
  // and "not issued" paths would make every later wait a full vmcnt(0).
  const int nb = (kb1 - kb0) / U;  // whole batches
  int kb = kb0;
  F fa[U], fb[U];
  if (nb >= 1) {
#pragma unroll
    for (int u = 0; u < U; ++u) load(kb + u, fa[u]);
  }
  if constexpr (TOKL) {
    // Stage the token rows while the first weight batch is in flight.
    const int chunks = p.K >> 4;
    for (int idx = threadIdx.x; idx < tok_rows * chunks; idx += 256) {
      const int row = idx / chunks, c = idx - row * chunks;
      int br, orw;
      bool v;
      token_row<MOE>(p, m0 + row, br, orw, v);
      const u32x4 x = ldg128(p.a + (int64_t)br * p.lda + 16 * c);
      const int pos = (c & ~7) | ((c & 7) ^ (row & 7));
      *reinterpret_cast<u32x4*>(tok + (int64_t)row * p.K + 16 * pos) = x;
    }
    __syncthreads();
  }
  if (nb >= 1) {
    int j = 0;
    for (; j + 2 < nb; j += 2) {  // batches j (in fa) and j+1 (in fb), and j+2 follows
#pragma unroll
      for (int u = 0; u < U; ++u) load(kb + U + u, fb[u]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) step(kb + u, fa[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) load(kb + 2 * U + u, fa[u]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) step(kb + U + u, fb[u]);
      kb += 2 * U;
    }
    if (j + 1 < nb) {  // two batches left
#pragma unroll
      for (int u = 0; u < U; ++u) load(kb + U + u, fb[u]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) step(kb + u, fa[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) step(kb + U + u, fb[u]);
      kb += 2 * U;
    } else {  // one batch left
#pragma unroll
      for (int u = 0; u < U; ++u) step(kb + u, fa[u]);
      kb += U;
    }
  }
  for (; kb < kb1; ++kb) {
    F f;
    load(kb, f);
    step(kb, f);
  }

  // Cross-wave reduction over the KS waves of a group: red[wave][tile][i][lane].
  constexpr int TILES = NT * MT;
  __shared__ float red[KS > 1 ? 4 * TILES * 4 * 64 : 1];
  if constexpr (KS > 1) {
#pragma unroll
    for (int s = 0; s < NT; ++s)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = INT_ACC ? __int_as_float(acci[s][t][i]) : acc[s][t][i];
          red[((wave * TILES + s * MT + t) * 4 + i) * 64 + lane] = v;
        }
    __syncthreads();
  }
  if (!has_cols) return;
  // Output subtile o = (so, t) of the group is finished by its wave o % KS.
#pragma unroll
  for (int so = 0; so < NTH; ++so)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int o = so * MT + t;
      if (KS > 1 && (o % KS) != ks) continue;
      float g[4], u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (KS > 1) {
          float sg = 0.f, su = 0.f;
          int ig = 0, iu = 0;
#pragma unroll
          for (int w = 0; w < KS; ++w) {
            const int src = ns * KS + w;
            const float vg = red[((src * TILES + so * MT + t) * 4 + i) * 64 + lane];
            if (INT_ACC) ig += __float_as_int(vg); else sg += vg;
            if constexpr (EPI == kEpiGated) {
              const float vu = red[((src * TILES + (so + NTH) * MT + t) * 4 + i) * 64 + lane];
              if (INT_ACC) iu += __float_as_int(vu); else su += vu;
            }
          }
          g[i] = INT_ACC ? __int_as_float(ig) : sg;
          u[i] = INT_ACC ? __int_as_float(iu) : su;
        } else {
          g[i] = INT_ACC ? __int_as_float(acci[so][t][i]) : acc[so][t][i];
          if constexpr (EPI == kEpiGated) u[i] = INT_ACC ? __int_as_float(acci[so + NTH][t][i]) : acc[so + NTH][t][i];
          else u[i] = 0.f;
        }
      }
      finish4<KIND, EPI, ACT, MOE>(p, orow[t], brow[t], bval[t], nout0 + 16 * so + 4 * g4, g, u);
    }
}

// ============================================================ ring8
// Decode-shaped GEMM through an LDS ring. A block is NW waves; wave w owns NT
// 16-row weight subtiles and all NW waves share one 16-token subtile, over
// the whole K. Each 128-K step is a ring slot filled by direct global->LDS
// copies of whole 128-byte lines (8 operand rows x 128 B per copy: each
// wave's weights, the shared token rows, one 4-byte-per-lane copy of the
// step's scales), XOR-swizzled like the tiled kernel so the MFMA fragment
// reads are conflict-free. R-1 slots are in flight while one is consumed and
// in-flight data costs no registers. Whole-line copies stream from HBM
// markedly faster than the 16-row x 64-byte pattern of register fragments.
//
// KS > 1 (with NW == 1): KS waves of the block split K, each with its own
// ring over a contiguous range of 128-K steps, and add their partial sums
// through LDS at the end. It multiplies the waves, and so the bytes in
// flight per CU, when the output columns alone leave few waves per CU
// (decode on short N, MoE decode over a few experts).
template <int KIND, int NT, bool MOE, int EPI, int ACT, int R, bool WX128, int TQ, int NW, int KS = 1>
__global__ void __launch_bounds__(64 * NW * KS) ring8_kernel(G8 p) {
  constexpr bool GATED = (EPI == kEpiGated);
  constexpr int NTH = GATED ? NT / 2 : NT;
  constexpr bool INT_ACC = (KIND == kI8Token);
  constexpr bool SCALES = (KIND != kI8Token);
  // TQ token copies of 8 rows per slot: 1 when the block has at most 8 token
  // rows (lanes of the missing rows read row 0), 2 for 16 rows, 4 for 32
  // rows (two token subtiles per wave, so the weights stream once up to 32
  // rows).
  static_assert(TQ == 1 || TQ == 2 || TQ == 4, "one, two or four 8-row token copies");
  static_assert(TQ < 4 || (!MOE && NW == 1), "32 token rows: dense, one wave per block");
  constexpr int MT = TQ == 4 ? 2 : 1;               // 16-token subtiles per wave
  constexpr int SAL = 16 * MT;                      // scale lanes of the token rows
  static_assert(NW == 1 || KIND != kI8Group, "int8 group weight scales need one lane per weight row");
  constexpr int WQ = 2 * NT;                        // weight copies per wave and slot
  constexpr int EX = TQ + (SCALES ? 1 : 0);         // shared copies per slot
  static_assert(NW == 1 || EX <= NW, "one shared copy per wave at most");
  static_assert(KS == 1 || NW == 1, "K split and shared token copies do not combine");
  constexpr int E_HI = NW == 1 ? EX : 1;            // shared copies of a wave that has any
  constexpr int TOK_OFF = NW * NT * 2048;
  constexpr int SC_OFF = TOK_OFF + TQ * 1024;
  constexpr int SLOT = SC_OFF + (SCALES ? 256 : 0);
  static_assert((R - 2) * (WQ + E_HI) < 64, "vmcnt counts at most 63 copies");
  static_assert(KS == 1 || R * SLOT >= NT * MT * 4 * 64 * 4, "a wave's ring holds its partial sums");
  __shared__ __attribute__((aligned(1024))) uint8_t ring_all[KS * R * SLOT];

  const int lane = threadIdx.x & 63;
  const int wave = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // K-split wave
  uint8_t* ring = ring_all + kw * (R * SLOT);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int m0 = blockIdx.y * 16 * MT;
  int expert = 0;
  if constexpr (MOE) {
    expert = moe_block_expert(p.num_post, p.expert_ids, m0);
    if (expert < 0) return;
  }
  const int nout0 = (blockIdx.x * NW + wave) * (16 * NTH);
  int wrow0[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    if constexpr (GATED)
      wrow0[s] = s < NTH ? nout0 + 16 * s : p.gate_off + nout0 + 16 * (s - NTH);
    else
      wrow0[s] = nout0 + 16 * s;
  }
  const uint8_t* wbase = p.w + (int64_t)expert * p.w_es;

  // Weight copy q of this wave moves its operand rows 8q..8q+7; lane l takes
  // row 8q + l/8 and writes LDS position l%8 of that row with the row's chunk
  // (l%8) ^ swz(row).
  const int crow = lane >> 3;
  const uint8_t* wsrc[WQ];
#pragma unroll
  for (int q = 0; q < WQ; ++q) {
    const int row = 8 * q + crow;
    const int wr = min(wrow0[row >> 4] + (row & 15), p.N - 1);
    wsrc[q] = wbase + (int64_t)wr * p.ldw + 16 * ((lane & 7) ^ lds_swz(row & 15));
  }
  // Shared copy of this wave (NW > 1: wave e < EX issues shared copy e; NW == 1:
  // the only wave issues all EX): e < TQ is token rows 8e..8e+7, e == TQ the scales.
  const int e0 = NW == 1 ? 0 : wave;
  const int ne = NW == 1 ? EX : (wave < EX ? 1 : 0);
  const uint8_t* tsrc[TQ];
  {
    int mrow[TQ], br[TQ], orw[TQ];
    bool v[TQ];
#pragma unroll
    for (int e = 0; e < TQ; ++e) mrow[e] = m0 + 8 * e + crow;
    token_rows<MOE, TQ>(p, mrow, br, orw, v);
#pragma unroll
    for (int e = 0; e < TQ; ++e) tsrc[e] = p.a + (int64_t)br[e] * p.lda + 16 * ((lane & 7) ^ lds_swz(8 * e + crow));
  }
  // Scale copy: lanes 0..SAL-1 the token rows' activation scales, lanes
  // SAL.. the weight scales (fp8: one per subtile of the block; int8 group:
  // one per row).
  const float* ssrc = nullptr;
  int64_t sstride = 0;
  if constexpr (SCALES) {
    int br, orw;
    bool v;
    if (lane < SAL) {
      token_row<MOE>(p, m0 + lane, br, orw, v);
      ssrc = p.sa + (int64_t)br * p.sa_rs;
      sstride = p.sa_ks;
    } else {
      const float* swb = p.sw + (int64_t)expert * p.sw_es;
      int wr;
      if constexpr (KIND == kFp8Block) {
        const int j = min(lane - SAL, NW * NT - 1);  // subtile j of the block
        const int jw = j / NT, js = j % NT;           // its wave and slot
        const int n0 = (blockIdx.x * NW + jw) * (16 * NTH);
        const int r0 = GATED ? (js < NTH ? n0 + 16 * js : p.gate_off + n0 + 16 * (js - NTH)) : n0 + 16 * js;
        wr = min(r0, p.N - 1) >> 7;
      } else {
        const int j = min(lane - SAL, 16 * NT - 1);
        wr = min(wrow0[j >> 4] + (j & 15), p.N - 1);
      }
      ssrc = swb + (int64_t)wr * p.sw_ns;
      sstride = p.sw_ks;
    }
  }
  auto issue = [&](int kb, int slot) {
    uint8_t* st = ring + slot * SLOT;
    const int64_t ko = (int64_t)kb * 128, kw = (int64_t)kb * p.w_kbs;
#pragma unroll
    for (int q = 0; q < WQ; ++q) g2l_b128(wsrc[q] + kw, st + wave * NT * 2048 + q * 1024);
    for (int e = e0; e < e0 + ne; ++e) {
      if (e < TQ) g2l_b128(tsrc[e] + ko, st + TOK_OFF + e * 1024);
      else if constexpr (SCALES) g2l_b32(ssrc + (int64_t)kb * sstride, st + SC_OFF);
    }
  };

  const uint32_t frag0 = (uint32_t)r16 * 128 + 16 * (g4 ^ lds_swz(r16));
  const uint32_t frag1 = (uint32_t)r16 * 128 + 16 * ((4 + g4) ^ lds_swz(r16));
  const int tr = (TQ == 1 && r16 >= 8) ? 0 : r16;  // token row this lane reads
  const uint32_t tfrag0 = (uint32_t)tr * 128 + 16 * (g4 ^ lds_swz(tr));
  const uint32_t tfrag1 = (uint32_t)tr * 128 + 16 * ((4 + g4) ^ lds_swz(tr));
  v4f acc[NT][MT];
  v4i acci[NT][MT];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      acc[s][t] = v4f{0.f, 0.f, 0.f, 0.f};
      acci[s][t] = v4i{0, 0, 0, 0};
    }

  const int nks_all = p.K >> 7;
  const int kb0 = KS == 1 ? 0 : kw * nks_all / KS;
  const int nks = KS == 1 ? nks_all : (kw + 1) * nks_all / KS;  // this wave's steps end here
#pragma unroll
  for (int s0 = 0; s0 < R - 1; ++s0)
    if (kb0 + s0 < nks) issue(kb0 + s0, s0);
  int slot = 0;
  for (int kb = kb0; kb < nks; ++kb) {
    constexpr int AHEAD = R - 2;  // slots issued after slot kb, in steady state
    if (kb + AHEAD <= nks - 1) {
      if (ne == E_HI) wait_vmcnt<AHEAD * (WQ + E_HI)>(); else wait_vmcnt<AHEAD * WQ>();
    } else {
      wait_vmcnt<0>();
    }
    if constexpr (NW > 1) lds_barrier();  // shared token and scale copies of other waves
    const uint8_t* st = ring + slot * SLOT;
    v8i bf[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
      bf[t] = cat8(lds128(st + TOK_OFF + t * 2048 + tfrag0), lds128(st + TOK_OFF + t * 2048 + tfrag1));
    v8i af[NT];
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      const uint8_t* sub = st + (wave * NT + s) * 2048;
      af[s] = cat8(lds128(sub + frag0), lds128(sub + frag1));
      if constexpr (WX128) af[s] = flip80(af[s]);
    }
    float sa[MT], sw[NT][4];
    if constexpr (SCALES) {
      const float* sl = reinterpret_cast<const float*>(st + SC_OFF);
#pragma unroll
      for (int t = 0; t < MT; ++t) sa[t] = sl[16 * t + r16];
#pragma unroll
      for (int s = 0; s < NT; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sw[s][i] = KIND == kFp8Block ? sl[SAL + wave * NT + s] : sl[SAL + 16 * s + 4 * g4 + i];
    }
    // The slot consumed last step is free: every wave has passed this step's
    // barrier, so its fragments are in registers.
    const int next = kb + R - 1;
    if (next < nks) issue(next, slot == 0 ? R - 1 : slot - 1);
#pragma unroll
    for (int s = 0; s < NT; ++s)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if constexpr (KIND == kFp8Block) {
          const v4f part = mfma_fp8(af[s], bf[t], v4f{0.f, 0.f, 0.f, 0.f});
          const float c = sw[s][0] * sa[t];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[s][t][i] = fmaf(part[i], c, acc[s][t][i]);
        } else if constexpr (KIND == kI8Token) {
          acci[s][t] = mfma_i8(lo4(af[s]), lo4(bf[t]), acci[s][t]);
          acci[s][t] = mfma_i8(hi4(af[s]), hi4(bf[t]), acci[s][t]);
        } else {
          v4i part = mfma_i8(lo4(af[s]), lo4(bf[t]), v4i{0, 0, 0, 0});
          part = mfma_i8(hi4(af[s]), hi4(bf[t]), part);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[s][t][i] = fmaf((float)part[i], sw[s][i] * sa[t], acc[s][t][i]);
        }
      }
    slot = slot == R - 1 ? 0 : slot + 1;
  }

  if constexpr (KS > 1) {
    // Partial sums through each wave's own (drained) ring; wave 0 adds them.
    wait_vmcnt<0>();
    float* red = reinterpret_cast<float*>(ring);
#pragma unroll
    for (int s2 = 0; s2 < NT; ++s2)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[((s2 * MT + t) * 4 + i) * 64 + lane] = INT_ACC ? __int_as_float(acci[s2][t][i]) : acc[s2][t][i];
    __syncthreads();
    if (kw != 0) return;
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      const float* rw = reinterpret_cast<const float*>(ring_all + w * (R * SLOT));
#pragma unroll
      for (int s2 = 0; s2 < NT; ++s2)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float v = rw[((s2 * MT + t) * 4 + i) * 64 + lane];
            if constexpr (INT_ACC) acci[s2][t][i] += __float_as_int(v);
            else acc[s2][t][i] += v;
          }
    }
  }

  if (nout0 >= p.n_out) return;
  int ebrow[MT], eorow[MT];
  bool ebval[MT];
  {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) mrow[t] = m0 + 16 * t + r16;
    token_rows<MOE, MT>(p, mrow, ebrow, eorow, ebval);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int brow = ebrow[t], orow = eorow[t];
    const bool bval = ebval[t];
#pragma unroll
    for (int so = 0; so < NTH; ++so) {
      float g[4], u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[i] = INT_ACC ? __int_as_float(acci[so][t][i]) : acc[so][t][i];
        if constexpr (GATED) u[i] = INT_ACC ? __int_as_float(acci[so + NTH][t][i]) : acc[so + NTH][t][i];
        else u[i] = 0.f;
      }
      finish4<KIND, EPI, ACT, MOE>(p, orow, brow, bval, nout0 + 16 * so + 4 * g4, g, u);
    }
  }
}

// ============================================================ int4 widening (W4A8)
// 1/16 for W4 weights: their MFMA operands are 16 * (q - 8), so the int32
// partial is 16 times the group sum (exact: |partial| < 2^24) and this
// power-of-two factor restores it exactly.
template <int W4>
constexpr float kW4Unit = W4 ? 0.0625f : 1.0f;

// One packed word of 8 4-bit values -> two words of int8 16 * (q - 8) in
// ascending k. W4 == 1: nibble j of the word is k j (byte b: k 2b low, 2b+1
// high). W4 == 2 (RDNAHybridW4A16): low nibbles of bytes 0..3 are k 0 4 1 5,
// high nibbles k 2 6 3 7.
template <int W4>
__device__ __forceinline__ void widen_word(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t L = ((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u;  // low nibbles, as 16 * (q - 8)
  const uint32_t H = (w & 0xF0F0F0F0u) ^ 0x80808080u;         // high nibbles
  if constexpr (W4 == 1) {
    lo = __builtin_amdgcn_perm(H, L, 0x05010400u);  // L0 H0 L1 H1: k 0 1 2 3
    hi = __builtin_amdgcn_perm(H, L, 0x07030602u);  // L2 H2 L3 H3: k 4 5 6 7
  } else {
    lo = __builtin_amdgcn_perm(H, L, 0x06040200u);  // L0 L2 H0 H2: k 0 1 2 3
    hi = __builtin_amdgcn_perm(H, L, 0x07050301u);  // L1 L3 H1 H3: k 4 5 6 7
  }
}
// The 16 packed bytes of a lane's fragment (8 per 64-K half) -> the 32-byte
// int8 fragment of the two 16x16x64 MFMAs.
template <int W4>
__device__ __forceinline__ v8i widen_int4(const uint2& h0, const uint2& h1) {
  v8i r;
  uint32_t a, b;
  widen_word<W4>(h0.x, a, b); r[0] = (int)a; r[1] = (int)b;
  widen_word<W4>(h0.y, a, b); r[2] = (int)a; r[3] = (int)b;
  widen_word<W4>(h1.x, a, b); r[4] = (int)a; r[5] = (int)b;
  widen_word<W4>(h1.y, a, b); r[6] = (int)a; r[7] = (int)b;
  return r;
}

// ============================================================ tiled8
// LDS stage: operand rows of 128 bytes (the stage's 128-K block), weight
// rows 0..BN-1 then token rows, each row's 16-byte chunks XOR-swizzled
// (lds_swz). Subtile j = 16 consecutive rows = 2 KiB. After them each
// stage keeps the scales of its 128-K block: BM activation scales, then the
// weight scales (fp8: one per weight subtile; int8 group: one per weight row).
// Every byte of a stage, scales included, arrives by direct global->LDS copy,
// so a wave's outstanding copies retire strictly in issue order and
// `s_waitcnt vmcnt(n)` with n = copies issued for later stages waits for
// exactly one stage.
template <int KIND, int BM, int BN, int WM, int WN, int STAGES, bool MOE, int EPI, int ACT, bool WX128, int W4 = 0>
__global__ void __launch_bounds__(WM * WN * 64) tiled8_kernel(G8 p, int tiles_m, int tiles_n, int group_m) {
  constexpr int W = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int MT = TM / 16, NT = TN / 16;
  constexpr int SA = BN / 16, SB = BM / 16;
  // W4 (int8 group kind only): 4-bit weights, 1 plain (low nibble = even k,
  // value q - 8) or 2 RDNAHybridW4A16 word order. A stage then holds each
  // weight row's 128-K block as 64 packed bytes (16 rows per 1 KiB copy,
  // 16-byte chunks XOR-swizzled by (row >> 2) & 3); the fragment read widens
  // the nibbles to int8 16 * (q - 8), exact, and the fold divides by 16.
  static_assert(W4 == 0 || (KIND == kI8Group && !WX128), "int4 weights: int8 group kind only");
  constexpr int WCOPIES = W4 ? SA : 2 * SA;          // 1 KiB weight copies per stage
  constexpr int TOK_BASE = WCOPIES * 1024;           // token rows start here in a stage
  constexpr int NQ = WCOPIES + 2 * SB;  // 1 KiB operand copies per stage (8 token rows each)
  static_assert(NQ % W == 0, "operand copies split evenly over the waves");
  constexpr int QPW = NQ / W;
  constexpr bool HAS_SA = (KIND != kI8Token);
  constexpr int SA_COPIES = HAS_SA ? BM / 64 : 0;
  constexpr int SW_COPIES = (KIND == kFp8Block) ? 1 : (KIND == kI8Group ? BN / 64 : 0);
  constexpr int EXTRA = SA_COPIES + SW_COPIES;  // wave w < EXTRA issues one more copy
  static_assert(EXTRA <= W, "at most one scale copy per wave");
  static_assert(!HAS_SA || BM % 64 == 0, "scale copies move 64 rows");
  static_assert(KIND != kI8Group || BN % 64 == 0, "int8 group weight scales move 64 rows");
  constexpr int SA_OFF = NQ * 1024;
  constexpr int SW_OFF = SA_OFF + (HAS_SA ? BM * 4 : 0);
  constexpr int STAGE = SW_OFF + (KIND == kFp8Block ? 256 : (KIND == kI8Group ? BN * 4 : 0));
  constexpr bool GATED = (EPI == kEpiGated);
  constexpr int NTH = GATED ? NT / 2 : NT;
  constexpr bool INT_ACC = (KIND == kI8Token);
  // One weight-scale value per wave and K block when the wave's rows sit in one 128-row block.
  constexpr bool ONE_SW = !GATED && TN <= 128 && (128 % TN == 0);
  static_assert(!GATED || (NT % 2 == 0), "gated wave tiles pair gate and up subtiles");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int wm = wave % WM, wn = wave / WM;

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
  // MoE: a wave whose TM token rows are all padding (in an expert's last,
  // partly filled row tile) skips its fragment reads, MFMAs and folds; it
  // still issues its copies and takes every barrier.
  // The epilogue rows (MoE), loaded before the K loop (dense rows are
  // arithmetic), cover the wave's TM rows and so also decide this.
  bool rows_live = true;
  EpiRow erow[MOE ? MT : 1];
  if constexpr (MOE) {
    int mrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) mrow[t] = m0 + wm * TM + 16 * t + r16;
    epi_rows<MOE, MT>(p, mrow, erow);
    bool any = false;
#pragma unroll
    for (int t = 0; t < MT; ++t) any = any || erow[t].valid;
    rows_live = __ballot(any) != 0;
  }
  auto wrow_of = [&](int j) -> int {  // first weight row of LDS weight subtile j
    if constexpr (GATED) {
      const int base = tn * (BN / 2);
      return j < SA / 2 ? base + 16 * j : p.gate_off + base + 16 * (j - SA / 2);
    } else {
      return tn * BN + 16 * j;
    }
  };

  // Copy slots: a uniform base pointer plus a fixed 32-bit per-lane offset.
  // Copy q moves 8 operand rows x 128 contiguous bytes (8 whole cache
  // lines): lane l takes row 8q + l/8 and stores to LDS slot l%8 the 16-byte
  // chunk (l%8) ^ swz(row) of that row.
  uint32_t qoff[QPW];
  bool qis_w[QPW];
  int qbr[QPW];   // activation rows of the token copies (one batch of lookups)
  {
    int mrow[QPW], orw[QPW];
    bool v[QPW];
#pragma unroll
    for (int j = 0; j < QPW; ++j) mrow[j] = m0 + 8 * (wave + W * j - WCOPIES) + (lane >> 3);
    token_rows<MOE, QPW>(p, mrow, qbr, orw, v);
  }
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int q = wave + W * j;           // wave-uniform (a copy holds weight rows only
    const bool is_w = q < WCOPIES;        // or token rows only)
    uint32_t off;
    if (is_w && W4) {
      const int row = 16 * q + (lane >> 2);  // 64-byte packed rows
      const int r = min(wrow_of(row >> 4) + (row & 15), p.N - 1);
      off = (uint32_t)r * (uint32_t)p.ldw + 16 * ((lane & 3) ^ ((row >> 2) & 3));
    } else if (is_w) {
      const int row = 8 * q + (lane >> 3);
      const int r = min(wrow_of(row >> 4) + (row & 15), p.N - 1);
      off = (uint32_t)r * (uint32_t)p.ldw + 16 * ((lane & 7) ^ lds_swz(row));
    } else {
      const int trow = 8 * (q - WCOPIES) + (lane >> 3);  // token row of the block
      off = (uint32_t)qbr[j] * (uint32_t)p.lda + 16 * ((lane & 7) ^ lds_swz(trow));
    }
    qis_w[j] = is_w;
    qoff[j] = off;
    // Keep the offset a 32-bit register: the copy adds it to a scalar base
    // (saddr form), so no 64-bit per-lane address stays live across the loop.
    asm("" : "+v"(qoff[j]));
  }
  if constexpr (MOE) {
    if (expert < 0) return;
  }
  const uint8_t* wbase = p.w + (int64_t)expert * p.w_es;
  // Fragment reads: lane l reads row 16*subtile + l%16, chunks l/16 (half 0)
  // and 4 + l/16 (half 1), at their swizzled slots.
  const uint32_t frag0 = (uint32_t)r16 * 128 + 16 * ((g4) ^ lds_swz(r16));
  const uint32_t frag1 = (uint32_t)r16 * 128 + 16 * ((4 + g4) ^ lds_swz(r16));
  // Scale copy slot of this wave (if any): a per-lane pointer advanced by K block.
  const float* xptr = nullptr;
  int64_t xstride = 0;
  const bool has_extra = wave < EXTRA;
  if (has_extra) {
    if (wave < SA_COPIES) {
      int br, orw;
      bool v;
      token_row<MOE>(p, m0 + 64 * wave + lane, br, orw, v);
      xptr = p.sa + (int64_t)br * p.sa_rs;
      xstride = p.sa_ks;
    } else if constexpr (KIND == kFp8Block) {
      const int j = lane < SA ? lane : 0;
      xptr = p.sw + (int64_t)expert * p.sw_es + (int64_t)(wrow_of(j) >> 7) * p.sw_ns;
      xstride = p.sw_ks;
    } else if constexpr (KIND == kI8Group) {
      const int r = 64 * (wave - SA_COPIES) + lane;  // weight row within the block
      const int row = min(wrow_of(r >> 4) + (r & 15), p.N - 1);
      xptr = p.sw + (int64_t)expert * p.sw_es + (int64_t)row * p.sw_ns;
      xstride = p.sw_ks;
    }
  }

  auto issue = [&](int kb, int buf) {
    uint8_t* st = smem + buf * STAGE;
    const uint8_t* wb = wbase + (int64_t)kb * p.w_kbs;
    const uint8_t* ab = p.a + (int64_t)kb * 128;
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
      // Re-pinned at each use so the compiler neither hoists a 64-bit
      // zero-extended copy of the offset out of the loop (live registers)
      // nor builds the address per lane: scalar base + 32-bit offset.
      uint32_t o = qoff[j];
      asm volatile("" : "+v"(o));
      g2l_b128((qis_w[j] ? wb : ab) + o, st + (wave + W * j) * 1024);
    }
    if (has_extra) {
      uint8_t* dst = wave < SA_COPIES ? st + SA_OFF + wave * 256 : st + SW_OFF + (wave - SA_COPIES) * 256;
      g2l_b32(xptr + (int64_t)kb * xstride, dst);
    }
  };

  int aidx[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    if constexpr (GATED)
      aidx[s] = s < NTH ? wn * NTH + s : SA / 2 + wn * NTH + (s - NTH);
    else
      aidx[s] = wn * NT + s;
  }

  v4f acc[NT][MT];
  v4i acci[NT][MT];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      acc[s][t] = v4f{0.f, 0.f, 0.f, 0.f};
      acci[s][t] = v4i{0, 0, 0, 0};
    }

  const int nkb = p.K >> 7;
#pragma unroll
  for (int s0 = 0; s0 < STAGES - 1; ++s0)
    if (s0 < nkb) issue(s0, s0);
  // The last subtile's partial products of a K block are folded at the start
  // of the next block (under its first MFMAs) instead of at the end of their
  // own, and once more after the loop. acc[NT-1] receives the same additions
  // in the same order, so the result is unchanged; before the first block the
  // carried values are zeros and their fold adds exactly nothing.
  v4f prev_f[MT];
  v4i prev_i[MT];
  float prev_sw[4] = {0.f, 0.f, 0.f, 0.f};  // weight scale(s) of the previous subtile
  float prev_sa[MT], prev_c1[MT];             // the carried subtile's activation scales / products
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    prev_f[t] = v4f{0.f, 0.f, 0.f, 0.f};
    prev_i[t] = v4i{0, 0, 0, 0};
    prev_sa[t] = 0.f;
    prev_c1[t] = 0.f;
  }

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb % STAGES;
    // Copies issued after stage kb: STAGES-2 stages in steady state.
    constexpr int AHEAD = STAGES - 2;
    if (kb + AHEAD <= nkb - 1) {
      if (has_extra) wait_vmcnt<AHEAD * (QPW + 1)>(); else wait_vmcnt<AHEAD * QPW>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if (kb + STAGES - 1 < nkb) issue(kb + STAGES - 1, (kb + STAGES - 1) % STAGES);

    if (rows_live) {  // the K block's fragment reads, MFMAs and folds
      const uint8_t* st = smem + buf * STAGE;
      v8i bf[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const uint8_t* sub = st + TOK_BASE + (wm * MT + t) * 2048;
        bf[t] = cat8(lds128(sub + frag0), lds128(sub + frag1));
      }
      float sa_t[MT];
      if constexpr (HAS_SA) {
        const float* sl = reinterpret_cast<const float*>(st + SA_OFF);
#pragma unroll
        for (int t = 0; t < MT; ++t) sa_t[t] = sl[wm * TM + 16 * t + r16];
      }
      const float* swl = reinterpret_cast<const float*>(st + SW_OFF);
      float c1[MT];
      if constexpr (KIND == kFp8Block && ONE_SW) {
        const float sw = swl[aidx[0]];
#pragma unroll
        for (int t = 0; t < MT; ++t) c1[t] = sw * sa_t[t];
      }
      auto afrag = [&](int s) -> v8i {
        if constexpr (W4) {
          // Lane (r16, g4) needs k 16*g4 + [0,16) of each 64-K half: 8 packed
          // bytes at 32*h + 8*g4, i.e. chunk 2h + g4/2 at offset 8*(g4 & 1).
          const uint8_t* row = st + aidx[s] * 1024 + r16 * 64 + 8 * (g4 & 1);
          const int sw4 = (r16 >> 2) & 3;
          const uint2 h0 = *reinterpret_cast<const uint2*>(row + 16 * ((g4 >> 1) ^ sw4));
          const uint2 h1 = *reinterpret_cast<const uint2*>(row + 16 * ((2 + (g4 >> 1)) ^ sw4));
          return widen_int4<W4>(h0, h1);
        } else {
          const uint8_t* sub = st + aidx[s] * 2048;
          return cat8(lds128(sub + frag0), lds128(sub + frag1));
        }
      };
      // Software pipeline over the weight subtiles: the fragment of subtile
      // s+1 is read while subtile s runs its MFMAs, and the block-scale fold
      // of subtile s-1 is issued between them, so no fold waits on the MFMA
      // that produced its operand. sched_barrier keeps each step's
      // instructions in that step; the group barriers interleave one MFMA with
      // the fold of one earlier result.
      v8i afc = afrag(0);
#pragma unroll
      for (int s = 0; s < NT; ++s) {
        v8i afn;
        if (s + 1 < NT) afn = afrag(s + 1);
        v8i af = afc;
        if constexpr (WX128) af = flip80(af);
        v4f part_f[MT];
        v4i part_i[MT];
        float cur_sw[4];
        if constexpr (KIND == kFp8Block) {
          cur_sw[0] = ONE_SW ? 0.f : swl[aidx[s]];
#pragma unroll
          for (int t = 0; t < MT; ++t) part_f[t] = mfma_fp8(af, bf[t], v4f{0.f, 0.f, 0.f, 0.f});
        } else if constexpr (KIND == kI8Token) {
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            acci[s][t] = mfma_i8(lo4(af), lo4(bf[t]), acci[s][t]);
            acci[s][t] = mfma_i8(hi4(af), hi4(bf[t]), acci[s][t]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) cur_sw[i] = swl[16 * aidx[s] + 4 * g4 + i];
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            part_i[t] = mfma_i8(lo4(af), lo4(bf[t]), v4i{0, 0, 0, 0});
            part_i[t] = mfma_i8(hi4(af), hi4(bf[t]), part_i[t]);
          }
        }
        // The fold's scale of subtile s' and token subtile t, row i of the lane's four.
        auto fold_c = [&](const float* sw, int t, int i) -> float {
          if constexpr (KIND == kFp8Block) return ONE_SW ? c1[t] : sw[0] * sa_t[t];
          else return sw[i] * sa_t[t];
        };
        if constexpr (!INT_ACC) {
          if (s > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float v = (KIND == kFp8Block) ? prev_f[t][i] : (float)prev_i[t][i] * kW4Unit<W4>;
                acc[s - 1][t][i] = fmaf(v, fold_c(prev_sw, t, i), acc[s - 1][t][i]);
              }
          } else {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float v = (KIND == kFp8Block) ? prev_f[t][i] : (float)prev_i[t][i] * kW4Unit<W4>;
                const float c = (KIND == kFp8Block) ? (ONE_SW ? prev_c1[t] : prev_sw[0] * prev_sa[t])
                                                    : prev_sw[i] * prev_sa[t];
                acc[NT - 1][t][i] = fmaf(v, c, acc[NT - 1][t][i]);
              }
          }
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            prev_f[t] = part_f[t];
            prev_i[t] = part_i[t];
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) prev_sw[i] = cur_sw[i];
          // The next fragment's reads go out after this subtile's first MFMA:
          // the wait for them then comes one subtile later, never right after
          // they are issued.
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, KIND == kFp8Block ? 1 : 2, 0);
            if (t == 0 && s + 1 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, KIND == kFp8Block ? 4 : 8, 0);
          }
        }
        if (s + 1 < NT) afc = afn;
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (!INT_ACC) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          prev_sa[t] = sa_t[t];
          if constexpr (KIND == kFp8Block && ONE_SW) prev_c1[t] = c1[t];
        }
      }
    }  // rows_live
  }
  if constexpr (!INT_ACC) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = (KIND == kFp8Block) ? prev_f[t][i] : (float)prev_i[t][i] * kW4Unit<W4>;
        const float c = (KIND == kFp8Block) ? (ONE_SW ? prev_c1[t] : prev_sw[0] * prev_sa[t]) : prev_sw[i] * prev_sa[t];
        acc[NT - 1][t][i] = fmaf(v, c, acc[NT - 1][t][i]);
      }
  }

  // Epilogue straight from registers.
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const EpiRow e = MOE ? erow[MOE ? t : 0] : epi_row<MOE>(p, m0 + wm * TM + 16 * t + r16);
    const int br = e.brow, orw = e.orow;
    const bool v = e.valid;
#pragma unroll
    for (int so = 0; so < NTH; ++so) {
      float g[4], u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[i] = INT_ACC ? __int_as_float(acci[so][t][i]) : acc[so][t][i];
        if constexpr (GATED) u[i] = acc[so + NTH][t][i];
        else u[i] = 0.f;
      }
      const int col0 = GATED ? (tn * (BN / 2) + 16 * (wn * NTH + so) + 4 * g4)
                             : (tn * BN + 16 * (wn * NT + so) + 4 * g4);
      finish4_tw<KIND, EPI, ACT, MOE>(p, orw, br, v, col0, g, u, e.tw);
    }
  }
}

// ============================================================ launchers
// Token rows go to LDS when one 16-row subtile of them fits next to a second
// block on the CU (16 x K bytes <= 80 KiB); otherwise they stream with the weights.
constexpr int64_t kTokLdsMax = 80 * 1024;

template <int KIND, int NT, int MT, int KS, bool MOE, int EPI, int ACT, int U, bool WX128>
int launch_stream(const G8& p, int grid_y, hipStream_t st, const char* op) {
  constexpr int NTH = (EPI == kEpiGated) ? NT / 2 : NT;
  constexpr int NS = 4 / KS;
  const int groups = (p.n_out + 16 * NTH - 1) / (16 * NTH);
  const int grid_x = (groups + NS - 1) / NS;
  const int64_t tok_bytes = 16 * (int64_t)p.K;
  if (MT == 1 && tok_bytes <= kTokLdsMax) {
    hipLaunchKernelGGL((stream8_kernel<KIND, NT, MT, KS, MOE, EPI, ACT, U, WX128, MT == 1>), dim3(grid_x, grid_y),
                       dim3(256), (size_t)tok_bytes, st, p);
  } else {
    hipLaunchKernelGGL((stream8_kernel<KIND, NT, MT, KS, MOE, EPI, ACT, U, WX128, false>), dim3(grid_x, grid_y),
                       dim3(256), 0, st, p);
  }
  return check_launch(op);
}

// K-split factor of the ring kernel. Below four output waves per CU, four
// waves split K (two if K is too short for four steps each); from four per
// CU up a split only adds ring fills and a reduction (measured on MI355X:
// INT8 N=K=5120 at M=1 9.1 -> 7.6 us with the split, FP8 N=17408 K=5120 at
// M=1 20.2 -> 22.1 us with a two-way split).
//
// With one or four token copies per step (M <= 8, M 17..32) the split is
// taken while every block stays resident in one round (160 KiB of LDS per
// CU). With two token copies (M 9..16) it pays only on short K (measured: INT8 N=K=5120 at M=32 10.9 ->
// 10.1 us with four waves; FP8 N=5120 K=17408 at M=16 28 -> 32-36 us with two
// or four), so there it needs K <= 8192.
inline int ring_ksplit(const G8& p, int64_t waves, int64_t blocks, int64_t ring_bytes, int tq) {
  const int nks = p.K >> 7;
  const int64_t cus = cu_count();
  if (waves >= 4 * cus) return 1;
  const int top = nks >= 16 ? 4 : nks >= 8 ? 2 : 1;
  if (tq == 2) return nks <= 64 ? top : 1;
  const int64_t per_cu = (blocks + cus - 1) / cus;
  for (int ks = top; ks > 1; ks /= 2)
    if (per_cu * ks * ring_bytes <= 160 * 1024) return ks;
  return 1;
}

// T32: dense blocks of 17..32 token rows take two token subtiles per wave
// (weights streamed once); otherwise a block covers 16 rows (grid_y given).
template <int KIND, int NT, bool MOE, int EPI, int ACT, int R, bool WX128, int NW, bool SPLIT = false,
          bool T32 = false>
int launch_ring(const G8& p, int grid_y, hipStream_t st, const char* op) {
  constexpr int NTH = (EPI == kEpiGated) ? NT / 2 : NT;
  const int groups = (p.n_out + 16 * NTH - 1) / (16 * NTH);
  const int grid_x = (groups + NW - 1) / NW;
  // 32-row token subtiles pay when the columns alone give four waves per CU;
  // below that, two 16-row groups with the K split run faster (measured:
  // INT8 N=K=5120 at M=32 10.1 vs 11.8 us; FP8 N=17408 K=5120 at M=32 35 vs
  // 31 us the other way).
  const bool t32 = T32 && !MOE && NW == 1 && p.M > 16 && (int64_t)grid_x * ((p.M + 31) / 32) >= 4LL * cu_count();
  const int tq = (!MOE && p.M <= 8) ? 1 : (t32 ? 4 : 2);
  if (tq == 4) grid_y = (p.M + 31) / 32;
  int ks = 1;
  if constexpr (SPLIT && NW == 1) {
    constexpr bool SCALES = (KIND != kI8Token);
    const int64_t ring_bytes = (int64_t)R * (NT * 2048 + tq * 1024 + (SCALES ? 256 : 0));
    ks = ring_ksplit(p, (int64_t)grid_x * grid_y, (int64_t)grid_x * grid_y, ring_bytes, tq);
  }
  auto go = [&](auto tq_tag, auto ks_tag) {
    constexpr int TQ_ = decltype(tq_tag)::value;
    constexpr int KS_ = decltype(ks_tag)::value;
    hipLaunchKernelGGL((ring8_kernel<KIND, NT, MOE, EPI, ACT, R, WX128, TQ_, NW, KS_>), dim3(grid_x, grid_y),
                       dim3(64 * NW * KS_), 0, st, p);
  };
  auto with_tq = [&](auto ks_tag) {
    if (tq == 1) go(std::integral_constant<int, 1>{}, ks_tag);
    else if constexpr (T32 && !MOE && NW == 1) {
      if (tq == 4) go(std::integral_constant<int, 4>{}, ks_tag);
      else go(std::integral_constant<int, 2>{}, ks_tag);
    } else {
      go(std::integral_constant<int, 2>{}, ks_tag);
    }
  };
  if constexpr (SPLIT && NW == 1) {
    if (ks == 4) with_tq(std::integral_constant<int, 4>{});
    else if (ks == 2) with_tq(std::integral_constant<int, 2>{});
    else with_tq(std::integral_constant<int, 1>{});
  } else {
    with_tq(std::integral_constant<int, 1>{});
  }
  return check_launch(op);
}

// Dense decode ring (the automatic config up to 32 rows and wherever the
// weights stream): the ring depth and K split set the weight bytes in flight
// and how compact the window of concurrent reads is. A sweep on MI355X
// (K-block-major FP8, N x K from 2048 x 7168 to 17408 x 5120, M 1..32) found
// a three-slot ring with the K split sized to about five waves per CU best or
// near it almost everywhere (N=17408 K=5120: M=16 22.0 -> 18.5 us, M=32 28.6
// -> 26.6; N=5120 K=5120 M=32 14.4 -> 9.4; N=5120 K=17408 M=1 21.7 -> 19.1),
// except two token copies with long K (N=5120 K=17408 at M=16: 27 us unsplit
// with five slots, 40 with three) and int8 tokens with two copies (config 1,
// M=32: 10.7 vs 11.1 us), which keep the five-slot ring and its split rule.
template <int KIND, int EPI, bool WX128>
int launch_ring_dense(const G8& p, hipStream_t st, const char* op) {
  const int64_t cus = cu_count();
  const int grid_x = (p.n_out + 15) / 16;
  const bool t32 = p.M > 16 && (int64_t)grid_x * ((p.M + 31) / 32) >= 4 * cus;
  const int tq = p.M <= 8 ? 1 : (t32 ? 4 : 2);
  const int nks = p.K >> 7;
  if (tq == 2 && (KIND == kI8Token || nks > 64))
    return launch_ring<KIND, 1, false, EPI, kActSilu, 5, WX128, 1, true, true>(p, (p.M + 15) / 16, st, op);
  const int grid_y = tq == 4 ? (p.M + 31) / 32 : (p.M + 15) / 16;
  const double per_cu = (double)grid_x * grid_y / (double)cus;  // waves per CU without a split
  int ks = 1;
  for (int c : {2, 4})
    if (nks >= 4 * c && std::fabs(per_cu * c - 5.0) < std::fabs(per_cu * ks - 5.0)) ks = c;
  auto go = [&](auto tq_tag, auto ks_tag, auto r_tag) {
    constexpr int TQ_ = decltype(tq_tag)::value;
    constexpr int KS_ = decltype(ks_tag)::value;
    constexpr int R_ = decltype(r_tag)::value;
    hipLaunchKernelGGL((ring8_kernel<KIND, 1, false, EPI, kActSilu, R_, WX128, TQ_, 1, KS_>), dim3(grid_x, grid_y),
                       dim3(64 * KS_), 0, st, p);
  };
  auto with_ks = [&](auto tq_tag) {
    constexpr std::integral_constant<int, 3> r3{};
    if (ks == 4) go(tq_tag, std::integral_constant<int, 4>{}, r3);
    else if (ks == 2) go(tq_tag, std::integral_constant<int, 2>{}, r3);
    else go(tq_tag, std::integral_constant<int, 1>{}, r3);
  };
  // Up to 8 token rows without a split a fourth slot pays (N=17408 K=5120 at
  // M=1: 18.3 -> 17.2 us); with a split, or more token rows, three are better.
  if (tq == 1 && ks == 1)
    go(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 4>{});
  else if (tq == 1) with_ks(std::integral_constant<int, 1>{});
  else if (tq == 2) with_ks(std::integral_constant<int, 2>{});
  else with_ks(std::integral_constant<int, 4>{});
  return check_launch(op);
}

template <int KIND, int BM, int BN, int WM, int WN, int STAGES, bool MOE, int EPI, int ACT, bool WX128, int W4 = 0>
int launch_tiled(const G8& p, int grid_y_moe, hipStream_t st, const char* op) {
  constexpr int COLS = (EPI == kEpiGated) ? BN / 2 : BN;
  const int tiles_n = (p.n_out + COLS - 1) / COLS;
  if constexpr (MOE) {
    hipLaunchKernelGGL((tiled8_kernel<KIND, BM, BN, WM, WN, STAGES, MOE, EPI, ACT, WX128, W4>),
                       dim3(tiles_n, grid_y_moe), dim3(WM * WN * 64), 0, st, p, 0, tiles_n, 0);
  } else {
    const int tiles_m = (p.M + BM - 1) / BM;
    hipLaunchKernelGGL((tiled8_kernel<KIND, BM, BN, WM, WN, STAGES, MOE, EPI, ACT, WX128, W4>),
                       dim3(tiles_m * tiles_n), dim3(WM * WN * 64), 0, st, p, tiles_m, tiles_n, 8);
  }
  return check_launch(op);
}

// The same dense GEMM restricted to output columns [n0, N): weights, weight
// scales and output start n0 columns later.
template <int KIND, int EPI>
G8 dense_columns_from(const G8& p, int n0) {
  G8 q = p;
  q.w = p.w + (int64_t)n0 * p.ldw;
  q.sw = p.sw + (KIND == kFp8Block ? (int64_t)(n0 / 128) * p.sw_ns : (int64_t)n0 * p.sw_ns);
  q.out = static_cast<uint8_t*>(p.out) + (int64_t)n0 * (EPI == kEpiI32 ? 4 : 2);
  q.N = p.N - n0;
  q.n_out = p.n_out - n0;
  return q;
}

// 256x256 tiles, one block per CU. When the tile count leaves a last round
// less than half full, the whole rounds take the first columns and 128x128
// tiles (a quarter of the work each) finish the remaining columns, so the
// tail runs on every CU instead of a few.
template <int KIND, int EPI, bool WX128>
int launch_dense_256(const G8& p, hipStream_t st, const char* op) {
  const int cus = cu_count();
  const int tm = (p.M + 255) / 256, tn = (p.n_out + 255) / 256;
  const int64_t tiles = (int64_t)tm * tn;
  const int64_t rounds = tiles / cus, rem = tiles % cus;
  if (rounds >= 1 && rem > 0 && 2 * rem <= cus) {
    const int nb = (int)((rounds * cus) / tm);  // 256-column tiles run at full size
    if (nb >= 1 && nb < tn) {
      G8 big = p;
      big.N = big.n_out = 256 * nb;
      int rc = launch_tiled<KIND, 256, 256, 4, 2, 2, false, EPI, kActSilu, WX128>(big, 0, st, op);
      if (rc) return rc;
      return launch_tiled<KIND, 128, 128, 2, 2, 4, false, EPI, kActSilu, WX128>(
          dense_columns_from<KIND, EPI>(p, 256 * nb), 0, st, op);
    }
  }
  return launch_tiled<KIND, 256, 256, 4, 2, 2, false, EPI, kActSilu, WX128>(p, 0, st, op);
}

// Automatic config of the dense 8-bit GEMM: up to 32 rows the weight ring;
// above, the cheapest of four priced candidates (the wider tile on a tie).
//  - ring: one weight stream per 32 token rows, N*K bytes at 5 TB/s each,
//    plus 3 us;
//  - 128x128, 128x160, 128x256, 256x256 tiles: (rounds of tiles over the
//    CUs) x (one tile at the shape's per-CU rate + 4 us), the rates measured
//    on MI355X over one full round of FP8-block tiles (5.9, 5.6, 7.6, 9.1
//    TFLOP/s per CU); 256x256 adds its 128x128 column strip when it uses one.
// Fitted on a sweep of six shapes (N x K from 2048 x 7168 to 17408 x 5120,
// M 48..2048), this picks the fastest config, or one within 5 % of it, on
// every point; the fixed rule it replaces lost up to 2x (N=5120 K=17408:
// M=64 96 -> 46 us, M=256 149 -> 97 us; N=17408 K=5120 M=512 101 -> 74 us).
// int8 group weights keep the fixed rule (their 128x256 config is 128x128).
inline int dense_auto_cfg(int64_t M, int64_t n_out, int64_t K, bool group) {
  if (M <= 32) return 0;
  const int64_t cus = cu_count();
  auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((n_out + bn - 1) / bn); };
  auto rounds = [&](int64_t t) { return (double)((t + cus - 1) / cus); };
  const int64_t t256 = tiles(256, 256);
  if (group) return M <= 128 ? 3 : (t256 >= cus ? 5 : 6);
  const double flop = 2.0 * (double)K;  // per output element of a tile
  const double T3 = 128.0 * 128.0 * flop / 5.9e6 + 4.0;  // us
  const double T6 = 128.0 * 256.0 * flop / 7.6e6 + 4.0;
  const double T5 = 256.0 * 256.0 * flop / 9.1e6 + 4.0;
  const double T12 = 128.0 * 160.0 * flop / 5.6e6 + 4.0;
  const double e0 = (double)((M + 31) / 32) * (double)n_out * (double)K / 5e6 + 3.0;
  const double e3 = rounds(tiles(128, 128)) * T3, e6 = rounds(tiles(128, 256)) * T6;
  const double e12 = rounds(tiles(128, 160)) * T12;
  const int64_t r5 = t256 / cus, rem = t256 % cus;
  const double e5 = (r5 >= 1 && rem > 0 && 2 * rem <= cus) ? (double)r5 * T5 + rounds(4 * rem) * T3
                                                          : rounds(t256) * T5;
  // Candidates from the widest tile down; the first strictly cheaper wins.
  int best = 5;
  double eb = e5;
  const std::pair<int, double> rest[] = {{6, e6}, {12, e12}, {3, e3}, {0, e0}};
  for (const auto& c : rest)
    if (c.second < eb) { best = c.first; eb = c.second; }
  return best;
}

// Dense dispatch by M. cfg >= 0 pins one tile config (tile sweeps).
template <int KIND, int EPI, bool WX128>
int dense_dispatch(const G8& p, hipStream_t st, const char* op, int cfg) {
  const int M = p.M;
  if (cfg < 0) cfg = dense_auto_cfg(M, p.n_out, p.K, KIND == kI8Group);
  switch (cfg) {
    case 0: return launch_ring_dense<KIND, EPI, WX128>(p, st, op);
    case 1: return launch_stream<KIND, 1, 2, 4, false, EPI, kActSilu, 4, WX128>(p, (M + 31) / 32, st, op);
    case 2: return launch_stream<KIND, 1, 4, 4, false, EPI, kActSilu, 2, WX128>(p, (M + 63) / 64, st, op);
    case 3: return launch_tiled<KIND, 128, 128, 2, 2, 4, false, EPI, kActSilu, WX128>(p, 0, st, op);
    case 4: return launch_tiled<KIND, 256, 64, 4, 2, 3, false, EPI, kActSilu, WX128>(p, 0, st, op);
    case 5: return launch_dense_256<KIND, EPI, WX128>(p, st, op);
    case 6:
      // int8 group scales need one copy per 64 weight rows: 4 waves cannot carry 256 rows of them.
      if constexpr (KIND == kI8Group) return launch_tiled<KIND, 128, 128, 2, 2, 4, false, EPI, kActSilu, WX128>(p, 0, st, op);
      else return launch_tiled<KIND, 128, 256, 2, 2, 3, false, EPI, kActSilu, WX128>(p, 0, st, op);
    // Decode sweep points (token rows per wave, waves splitting K, K-steps per batch).
    case 7: return launch_stream<KIND, 1, 1, 2, false, EPI, kActSilu, 4, WX128>(p, (M + 15) / 16, st, op);
    case 8: return launch_stream<KIND, 1, 1, 4, false, EPI, kActSilu, 4, WX128>(p, (M + 15) / 16, st, op);
    case 9: return launch_ring<KIND, 1, false, EPI, kActSilu, 7, WX128, KIND == kI8Group ? 1 : 4>(p, (M + 15) / 16, st, op);
    case 10: return launch_ring<KIND, 1, false, EPI, kActSilu, 7, WX128, 1>(p, (M + 15) / 16, st, op);
    case 11: return launch_ring<KIND, 1, false, EPI, kActSilu, 6, WX128, KIND == kI8Group ? 1 : 4>(p, (M + 15) / 16, st, op);
    // 128x160: a round that 128x256 fills only half, filled to 85 % (17408
    // columns in 109 tiles per 128 rows: config 2 at M=256 54.4 -> 42.4 us).
    // int8 group scales need 64-row multiples: 128x128 there.
    case 12:
      if constexpr (KIND == kI8Group) return launch_tiled<KIND, 128, 128, 2, 2, 4, false, EPI, kActSilu, WX128>(p, 0, st, op);
      else return launch_tiled<KIND, 128, 160, 2, 2, 3, false, EPI, kActSilu, WX128>(p, 0, st, op);
    default: return set_error(STRIX_ERR_INVALID, "%s: cfg must be in 0..12, got %d", op, cfg);
  }
}

// MoE dispatch by block_m (the sorted-id granularity).
template <int KIND, int EPI, int ACT>
int moe_dispatch(const G8& p, int block_m, int num_blocks, hipStream_t st, const char* op) {
  constexpr int NTS = (EPI == kEpiGated) ? 2 : 1;
  switch (block_m) {
    // No K split here: measured slower at T=1 (29 -> 32 us for config 3).
    // Two 16-row weight subtiles per wave for both GEMMs: the short-K down
    // projection keeps twice the bytes in flight per wave (config 3 T=64
    // 145 -> 140 us). Three ring slots once the live blocks (at most one per
    // routed slot) give four waves per CU, five below (config 3: T=64 140 ->
    // 134 us with three, T=1 31 -> 33 us).
    case 16: {
      constexpr int COLS = (EPI == kEpiGated) ? 16 : 32;  // output columns per wave
      const int64_t live = std::min<int64_t>(num_blocks, p.num_slots);
      if ((int64_t)((p.n_out + COLS - 1) / COLS) * live >= 4LL * cu_count())
        return launch_ring<KIND, 2, true, EPI, ACT, 3, false, 1>(p, num_blocks, st, op);
      return launch_ring<KIND, 2, true, EPI, ACT, 5, false, 1>(p, num_blocks, st, op);
    }
    case 32: return launch_stream<KIND, NTS, 2, 2, true, EPI, ACT, 4, false>(p, num_blocks, st, op);
    case 64: return launch_tiled<KIND, 64, 128, 1, 4, 4, true, EPI, ACT, false>(p, num_blocks, st, op);
    case 128: return launch_tiled<KIND, 128, 128, 2, 2, 4, true, EPI, ACT, false>(p, num_blocks, st, op);
    // The dense headline's 256x256 tile: 571 -> 505 us for config 3 at T=4096 against 256x128.
    case 256: return launch_tiled<KIND, 256, 256, 4, 2, 2, true, EPI, ACT, false>(p, num_blocks, st, op);
    default: return set_error(STRIX_ERR_INVALID, "%s: block_m must be 16, 32, 64, 128 or 256, got %d", op, block_m);
  }
}

// Row-major 8-bit weights [E][N][ldw] -> K-block-major [E][K/128][N][128]:
// every 128-K block of all N rows is one contiguous run. The decode and
// prefill kernels read weights 128 K at a time, and in this order the blocks
// all waves read at one moment lie close together in memory instead of one
// per row group across the whole matrix, which DRAM serves faster. One
// thread per 16-byte chunk, in output order.
__global__ void __launch_bounds__(256)
    weight_kmajor_kernel(const uint8_t* __restrict__ w, int64_t ldw, int64_t N, int64_t kbs,
                         int64_t chunks, uint8_t* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int64_t j = c & 7, row = c >> 3;   // 16-byte chunk within the 128-byte block, global block row
  const int64_t n = row % N, ekb = row / N;
  const int64_t e = ekb / kbs, kb = ekb % kbs;
  const u32x4 v = *reinterpret_cast<const u32x4*>(w + (e * N + n) * ldw + kb * 128 + j * 16);
  *reinterpret_cast<u32x4*>(out + c * 16) = v;
}

int check_common(const char* op, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw,
                 const void* a, const void* w) {
  STRIX_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size", op);
  STRIX_REQUIRE(K % 128 == 0, "%s: K must be a multiple of 128, got K=%lld", op, (long long)K);
  STRIX_REQUIRE(ldw >= K && ldw % 16 == 0, "%s: weight row stride (%lld bytes) must be >= K and a multiple of 16",
                op, (long long)ldw);
  STRIX_REQUIRE(lda >= K && lda % 16 == 0, "%s: activation row stride must be >= K and a multiple of 16", op);
  STRIX_REQUIRE(aligned(a, 16) && aligned(w, 16), "%s: operands must be 16-byte aligned", op);
  STRIX_REQUIRE(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, "%s: sizes overflow 32-bit indexing", op);
  STRIX_REQUIRE(fits_u32_rows(M, lda, K) && fits_u32_rows(N, ldw, K),
                "%s: an operand spans more than 4 GiB (the kernels use 32-bit row offsets); split the call", op);
  return STRIX_OK;
}

}  // namespace
}  // namespace strix

using namespace strix;

extern "C" {

int strix_fp8_w8a8_block_gemm(const uint8_t* qa, int64_t lda, const float* sa, int64_t sa_ld,
                              const uint8_t* w, int64_t ldw, const float* sw, int64_t sw_ld,
                              void* out, int64_t ldo, int out_dtype, int64_t M, int64_t N,
                              int64_t K, int cfg, void* stream) {
  const char* op = "fp8_w8a8_block_gemm";
  int rc = check_common(op, M, N, K, lda, ldw, qa, w);
  if (rc) return rc;
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(sa_ld >= K / 128 && sw_ld >= K / 128, "%s: scale row strides must be >= K/128", op);
  STRIX_REQUIRE(ldo >= N && ldo % 4 == 0 && aligned(out, 8), "%s: output rows must be >= N, 8-byte aligned", op);
  if (M == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = w; p.ldw = ldw; p.w_es = 0;
  p.sw = sw; p.sw_es = 0; p.sw_ns = sw_ld; p.sw_ks = 1;
  p.a = qa; p.lda = lda; p.sa = sa; p.sa_rs = sa_ld; p.sa_ks = 1;
  p.out = out; p.ldo = ldo; p.out_f16 = out_dtype == STRIX_F16;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.n_out = (int)N;
  return dense_dispatch<kFp8Block, kEpiStore, false>(p, as_stream(stream), op, cfg);
}

int strix_weight8_kmajor(const uint8_t* w, int64_t ldw, int64_t E, int64_t N, int64_t K, uint8_t* out,
                         void* stream) {
  const char* op = "weight8_kmajor";
  STRIX_REQUIRE(E >= 1 && N >= 0 && K >= 0, "%s: bad sizes", op);
  STRIX_REQUIRE(K % 128 == 0, "%s: K must be a multiple of 128, got K=%lld", op, (long long)K);
  STRIX_REQUIRE(ldw >= K && ldw % 16 == 0, "%s: weight row stride must be >= K and a multiple of 16", op);
  STRIX_REQUIRE(aligned(w, 16) && aligned(out, 16), "%s: weights must be 16-byte aligned", op);
  if (N == 0 || K == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  const int64_t chunks = E * N * (K / 16);
  hipLaunchKernelGGL(weight_kmajor_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, as_stream(stream),
                     w, ldw, N, K / 128, chunks, out);
  return check_launch(op);
}

int strix_fp8_w8a8_block_gemm_kmajor(const uint8_t* qa, int64_t lda, const float* sa, int64_t sa_ld,
                                     const uint8_t* w_kmajor, const float* sw, int64_t sw_ld, void* out,
                                     int64_t ldo, int out_dtype, int64_t M, int64_t N, int64_t K, int cfg,
                                     void* stream) {
  const char* op = "fp8_w8a8_block_gemm_kmajor";
  int rc = check_common(op, M, N, K, lda, K, qa, w_kmajor);
  if (rc) return rc;
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(sa_ld >= K / 128 && sw_ld >= K / 128, "%s: scale row strides must be >= K/128", op);
  STRIX_REQUIRE(ldo >= N && ldo % 4 == 0 && aligned(out, 8), "%s: output rows must be >= N, 8-byte aligned", op);
  if (M == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = w_kmajor; p.ldw = 128; p.w_kbs = 128 * N; p.w_es = 0;
  p.sw = sw; p.sw_es = 0; p.sw_ns = sw_ld; p.sw_ks = 1;
  p.a = qa; p.lda = lda; p.sa = sa; p.sa_rs = sa_ld; p.sa_ks = 1;
  p.out = out; p.ldo = ldo; p.out_f16 = out_dtype == STRIX_F16;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.n_out = (int)N;
  return dense_dispatch<kFp8Block, kEpiStore, false>(p, as_stream(stream), op, cfg);
}

int strix_w8a8_int8_gemm(const int8_t* qa, int64_t lda, const float* sa, const int8_t* w, int64_t ldw,
                         const float* sw, void* out, int64_t ldo, int out_dtype, int64_t M, int64_t N,
                         int64_t K, int cfg, void* stream) {
  const char* op = "w8a8_scaled_mm";
  int rc = check_common(op, M, N, K, lda, ldw, qa, w);
  if (rc) return rc;
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16 || out_dtype == STRIX_I32,
                "%s: output must be bfloat16, float16 or int32", op);
  STRIX_REQUIRE(ldo >= N && ldo % 4 == 0 && aligned(out, 16), "%s: output rows must be >= N, 16-byte aligned", op);
  if (M == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = reinterpret_cast<const uint8_t*>(w); p.ldw = ldw;
  p.sw = sw; p.sw_ns = 1;
  p.a = reinterpret_cast<const uint8_t*>(qa); p.lda = lda; p.sa = sa; p.sa_rs = 1; p.sa_ks = 0;
  p.out = out; p.ldo = ldo; p.out_f16 = out_dtype == STRIX_F16;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.n_out = (int)N;
  if (out_dtype == STRIX_I32) return dense_dispatch<kI8Token, kEpiI32, false>(p, as_stream(stream), op, cfg);
  STRIX_REQUIRE(sa != nullptr && sw != nullptr, "%s: scales are required for a float output", op);
  return dense_dispatch<kI8Token, kEpiStore, false>(p, as_stream(stream), op, cfg);
}

int strix_w8a8_int8_group_gemm(const int8_t* qa, int64_t lda, const float* sa, int64_t sa_ld,
                               const uint8_t* w, int64_t ldw, int w_excess128, const float* sw,
                               int64_t sw_ns, int64_t sw_gs, void* out, int64_t ldo, int out_dtype,
                               int64_t M, int64_t N, int64_t K, int cfg, void* stream) {
  const char* op = "w8a8_wmma_gemm";
  int rc = check_common(op, M, N, K, lda, ldw, qa, w);
  if (rc) return rc;
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(ldo >= N && ldo % 4 == 0 && aligned(out, 8), "%s: output rows must be >= N, 8-byte aligned", op);
  if (M == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = w; p.ldw = ldw;
  p.sw = sw; p.sw_ns = sw_ns; p.sw_ks = sw_gs;
  p.a = reinterpret_cast<const uint8_t*>(qa); p.lda = lda; p.sa = sa; p.sa_rs = sa_ld; p.sa_ks = 1;
  p.out = out; p.ldo = ldo; p.out_f16 = out_dtype == STRIX_F16;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.n_out = (int)N;
  if (w_excess128) return dense_dispatch<kI8Group, kEpiStore, true>(p, as_stream(stream), op, cfg);
  return dense_dispatch<kI8Group, kEpiStore, false>(p, as_stream(stream), op, cfg);
}

}  // extern "C"

namespace strix {
namespace {

// Checks shared by the W4A8 entry points: int8 activations [rows, lda >= K],
// packed 4-bit weight rows of K/2 bytes (16-byte aligned strides).
int check_w4a8(const char* op, int64_t rows, int64_t N, int64_t K, int64_t lda, int64_t ldw, const void* a,
               const void* w) {
  STRIX_REQUIRE(rows >= 0 && N >= 0 && K >= 0, "%s: negative size", op);
  STRIX_REQUIRE(K % 128 == 0, "%s: K must be a multiple of 128, got K=%lld", op, (long long)K);
  STRIX_REQUIRE(ldw * 2 >= K && ldw % 16 == 0, "%s: weight rows must hold K/2 bytes at a 16-byte multiple stride", op);
  STRIX_REQUIRE(lda >= K && lda % 16 == 0, "%s: activation row stride must be >= K and a multiple of 16", op);
  STRIX_REQUIRE(aligned(a, 16) && aligned(w, 16), "%s: operands must be 16-byte aligned", op);
  STRIX_REQUIRE(rows <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, "%s: sizes overflow 32-bit indexing", op);
  STRIX_REQUIRE(fits_u32_rows(rows, lda, K) && fits_u32_rows(N, ldw, K / 2),
                "%s: an operand spans more than 4 GiB (the kernels use 32-bit row offsets); split the call", op);
  return STRIX_OK;
}

template <int W4>
int w4a8_dense(const G8& p, hipStream_t st, const char* op) {
  if (p.M <= 128) return launch_tiled<kI8Group, 128, 128, 2, 2, 3, false, kEpiStore, kActSilu, false, W4>(p, 0, st, op);
  return launch_tiled<kI8Group, 256, 256, 4, 2, 2, false, kEpiStore, kActSilu, false, W4>(p, 0, st, op);
}

template <int EPI, int ACT>
int w4a8_moe(const G8& p, int block_m, int num_blocks, hipStream_t st, const char* op) {
  switch (block_m) {
    case 64: return launch_tiled<kI8Group, 64, 128, 1, 4, 4, true, EPI, ACT, false, 1>(p, num_blocks, st, op);
    case 128: return launch_tiled<kI8Group, 128, 128, 2, 2, 3, true, EPI, ACT, false, 1>(p, num_blocks, st, op);
    case 256: return launch_tiled<kI8Group, 256, 256, 4, 2, 2, true, EPI, ACT, false, 1>(p, num_blocks, st, op);
    default: return set_error(STRIX_ERR_INVALID, "%s: block_m must be 64, 128 or 256, got %d", op, block_m);
  }
}

}  // namespace
}  // namespace strix

extern "C" {

int strix_w4a8_gemm(const int8_t* qa, int64_t lda, const float* sa, int64_t sa_ld, const uint8_t* w4, int64_t ldw,
                    int order, const float* sw, int64_t sw_ns, int64_t sw_gs, void* out, int64_t ldo, int out_dtype,
                    int64_t M, int64_t N, int64_t K, void* stream) {
  const char* op = "w4a8_wmma_gemm";
  int rc = check_w4a8(op, M, N, K, lda, ldw, qa, w4);
  if (rc) return rc;
  STRIX_REQUIRE(order == 1 || order == 2, "%s: nibble order must be 1 (plain) or 2 (RDNAHybridW4A16), got %d", op,
                order);
  STRIX_REQUIRE(out_dtype == STRIX_BF16 || out_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(ldo >= N && ldo % 4 == 0 && aligned(out, 8), "%s: output rows must be >= N, 8-byte aligned", op);
  STRIX_REQUIRE(sa != nullptr && sw != nullptr, "%s: scales are required", op);
  if (M == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = w4; p.ldw = ldw; p.w_kbs = 64;
  p.sw = sw; p.sw_ns = sw_ns; p.sw_ks = sw_gs;
  p.a = reinterpret_cast<const uint8_t*>(qa); p.lda = lda; p.sa = sa; p.sa_rs = sa_ld; p.sa_ks = 1;
  p.out = out; p.ldo = ldo; p.out_f16 = out_dtype == STRIX_F16;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.n_out = (int)N;
  return order == 2 ? w4a8_dense<2>(p, as_stream(stream), op) : w4a8_dense<1>(p, as_stream(stream), op);
}

int strix_moe_gemm_w4a8(void* c, int64_t ldc, int c_dtype, const int8_t* qa, int64_t lda, const float* sa,
                        int64_t sa_ld, const uint8_t* w4, int64_t w_es, int64_t ldw, const float* sw, int64_t sw_es,
                        int64_t sw_ns, const int32_t* sorted_ids, int64_t sorted_len, const int32_t* expert_ids,
                        int64_t num_blocks, const int32_t* num_post, const float* topk_weights, int64_t num_slots,
                        int64_t top_k, int64_t block_m, int silu_mul, int activation, int64_t N, int64_t K,
                        void* stream) {
  const char* op = "moe_gemm_w4a8";
  int rc = check_w4a8(op, num_slots, N, K, lda, ldw, qa, w4);
  if (rc) return rc;
  STRIX_REQUIRE(c_dtype == STRIX_BF16 || c_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(top_k >= 1, "%s: top_k must be >= 1", op);
  STRIX_REQUIRE(w_es % 16 == 0, "%s: the expert stride of the weights must be a multiple of 16 bytes", op);
  STRIX_REQUIRE(num_blocks * block_m >= sorted_len, "%s: expert_ids.numel() * block_m must cover sorted_ids", op);
  STRIX_REQUIRE(N % 16 == 0, "%s: N must be a multiple of 16", op);
  STRIX_REQUIRE(activation == kActSilu || activation == kActGeluTanh, "%s: unknown activation", op);
  const int64_t n_out = silu_mul ? N / 2 : N;
  STRIX_REQUIRE(ldc >= n_out && ldc % 4 == 0 && aligned(c, 8), "%s: output rows must be >= %lld, 8-byte aligned",
                op, (long long)n_out);
  // A gated tile holds BN/2 gate and BN/2 up rows: 64 each (block_m 64, 128), 128 (block_m 256).
  const int64_t half_tile = block_m == 256 ? 128 : 64;
  STRIX_REQUIRE(!silu_mul || (N / 2) % half_tile == 0, "%s: gated N/2 must be a multiple of %lld at block_m %lld",
                op, (long long)half_tile, (long long)block_m);
  if (num_blocks == 0 || sorted_len == 0 || num_slots == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = w4; p.ldw = ldw; p.w_es = w_es; p.w_kbs = 64;
  p.sw = sw; p.sw_es = sw_es; p.sw_ns = sw_ns; p.sw_ks = 1;
  p.a = reinterpret_cast<const uint8_t*>(qa); p.lda = lda; p.sa = sa; p.sa_rs = sa_ld; p.sa_ks = 1;
  p.out = c; p.ldo = ldc; p.out_f16 = c_dtype == STRIX_F16;
  p.M = (int)num_slots; p.N = (int)N; p.K = (int)K; p.n_out = (int)n_out; p.gate_off = (int)(N / 2);
  p.sorted_ids = sorted_ids; p.sorted_len = sorted_len; p.expert_ids = expert_ids; p.num_post = num_post;
  p.num_slots = (int)num_slots; p.top_k = (int)top_k; p.topk_w = topk_weights;
  hipStream_t st = as_stream(stream);
  const int nb = (int)num_blocks, bm = (int)block_m;
  if (silu_mul) {
    if (activation == kActGeluTanh) return w4a8_moe<kEpiGated, kActGeluTanh>(p, bm, nb, st, op);
    return w4a8_moe<kEpiGated, kActSilu>(p, bm, nb, st, op);
  }
  return w4a8_moe<kEpiStore, kActSilu>(p, bm, nb, st, op);
}

}  // extern "C"

namespace strix {
namespace {

// The FP8-block expert GEMM over row-major weights [E][N][ldw] (w_es bytes
// per expert) or, with kmajor, K-block-major ones [E][K/128][N][128].
int moe_gemm_fp8(const char* op, void* c, int64_t ldc, int c_dtype, const uint8_t* qa, int64_t lda,
                 const float* sa, int64_t sa_ld, const uint8_t* w, int64_t w_es, int64_t ldw, bool kmajor,
                 const float* sw, int64_t sw_es, int64_t sw_ns, const int32_t* sorted_ids, int64_t sorted_len,
                 const int32_t* expert_ids, int64_t num_blocks, const int32_t* num_post,
                 const float* topk_weights, int64_t num_slots, int64_t top_k, int64_t block_m, int silu_mul,
                 int activation, int64_t N, int64_t K, void* stream) {
  int rc = check_common(op, num_slots, N, K, lda, kmajor ? K : ldw, qa, w);
  if (rc) return rc;
  STRIX_REQUIRE(c_dtype == STRIX_BF16 || c_dtype == STRIX_F16, "%s: output must be bfloat16 or float16", op);
  STRIX_REQUIRE(top_k >= 1, "%s: top_k must be >= 1", op);
  STRIX_REQUIRE(num_blocks * block_m >= sorted_len, "%s: expert_ids.numel() * block_m must cover sorted_ids", op);
  STRIX_REQUIRE(!silu_mul || N % 32 == 0, "%s: gated N must be a multiple of 32", op);
  STRIX_REQUIRE(N % 16 == 0, "%s: N must be a multiple of 16", op);
  STRIX_REQUIRE(activation == kActSilu || activation == kActGeluTanh, "%s: unknown activation", op);
  const int64_t n_out = silu_mul ? N / 2 : N;
  STRIX_REQUIRE(ldc >= n_out && ldc % 4 == 0 && aligned(c, 8), "%s: output rows must be >= %lld, 8-byte aligned",
                op, (long long)n_out);
  STRIX_REQUIRE(!silu_mul || (N / 2) % 128 == 0, "%s: gated FP8-block N/2 must be a multiple of 128", op);
  if (num_blocks == 0 || sorted_len == 0 || num_slots == 0 || N == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  G8 p = {};
  p.w = w;
  if (kmajor) {
    p.ldw = 128; p.w_es = N * K; p.w_kbs = 128 * N;
  } else {
    p.ldw = ldw; p.w_es = w_es;
  }
  p.sw = sw; p.sw_es = sw_es; p.sw_ns = sw_ns; p.sw_ks = 1;
  p.a = qa; p.lda = lda; p.sa = sa; p.sa_rs = sa_ld; p.sa_ks = 1;
  p.out = c; p.ldo = ldc; p.out_f16 = c_dtype == STRIX_F16;
  p.M = (int)num_slots; p.N = (int)N; p.K = (int)K; p.n_out = (int)n_out; p.gate_off = (int)(N / 2);
  p.sorted_ids = sorted_ids; p.sorted_len = sorted_len; p.expert_ids = expert_ids; p.num_post = num_post;
  p.num_slots = (int)num_slots; p.top_k = (int)top_k; p.topk_w = topk_weights;
  hipStream_t st = as_stream(stream);
  const int nb = (int)num_blocks, bm = (int)block_m;
  if (silu_mul) {
    if (activation == kActGeluTanh) return moe_dispatch<kFp8Block, kEpiGated, kActGeluTanh>(p, bm, nb, st, op);
    return moe_dispatch<kFp8Block, kEpiGated, kActSilu>(p, bm, nb, st, op);
  }
  return moe_dispatch<kFp8Block, kEpiStore, kActSilu>(p, bm, nb, st, op);
}

}  // namespace
}  // namespace strix

extern "C" {

int strix_moe_gemm_fp8_w8a8(void* c, int64_t ldc, int c_dtype, const uint8_t* qa, int64_t lda,
                            const float* sa, int64_t sa_ld, const uint8_t* w, int64_t w_es, int64_t ldw,
                            const float* sw, int64_t sw_es, int64_t sw_ns, const int32_t* sorted_ids,
                            int64_t sorted_len, const int32_t* expert_ids, int64_t num_blocks,
                            const int32_t* num_post, const float* topk_weights, int64_t num_slots,
                            int64_t top_k, int64_t block_m, int silu_mul, int activation, int64_t N,
                            int64_t K, void* stream) {
  return moe_gemm_fp8("moe_gemm_fp8_w8a8", c, ldc, c_dtype, qa, lda, sa, sa_ld, w, w_es, ldw, false, sw, sw_es,
                      sw_ns, sorted_ids, sorted_len, expert_ids, num_blocks, num_post, topk_weights, num_slots,
                      top_k, block_m, silu_mul, activation, N, K, stream);
}

int strix_moe_gemm_fp8_w8a8_kmajor(void* c, int64_t ldc, int c_dtype, const uint8_t* qa, int64_t lda,
                                   const float* sa, int64_t sa_ld, const uint8_t* w_kmajor, const float* sw,
                                   int64_t sw_es, int64_t sw_ns, const int32_t* sorted_ids, int64_t sorted_len,
                                   const int32_t* expert_ids, int64_t num_blocks, const int32_t* num_post,
                                   const float* topk_weights, int64_t num_slots, int64_t top_k, int64_t block_m,
                                   int silu_mul, int activation, int64_t N, int64_t K, void* stream) {
  return moe_gemm_fp8("moe_gemm_fp8_w8a8_kmajor", c, ldc, c_dtype, qa, lda, sa, sa_ld, w_kmajor, 0, 0, true,
                      sw, sw_es, sw_ns, sorted_ids, sorted_len, expert_ids, num_blocks, num_post,
                      topk_weights, num_slots, top_k, block_m, silu_mul, activation, N, K, stream);
}

}  // extern "C"
