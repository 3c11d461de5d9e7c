// SPDX-License-Identifier: MIT
// Pieces shared by the 8-bit (gemm8.hip) and 16-bit (gemm16.hip) GEMM
// kernels: raw vector moves, the dense/MoE token-row mapping, the swizzled LDS
// row layout and the epilogue (gated act*mul, top-k weight, bf16/fp16 store).
//
// MoE contract (reference: csrc/moe/moe_gemm_w8a16.hip:76-404,
// tests/test_moe_gemm.py:9-42): sorted_ids groups slot ids by expert; a slot
// id >= num_slots is padding; the A row of slot s is s / top_k; a block whose
// first sorted position is >= num_post_padded, or whose expert id is < 0,
// does nothing.
#pragma once

#include "strix_common.h"

namespace strix {

enum Epi : int { kEpiStore = 0, kEpiGated = 1, kEpiI32 = 2 };

__device__ __forceinline__ u32x4 ldg128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 lds128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ v8i cat8(const u32x4& lo, const u32x4& hi) {
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}
__device__ __forceinline__ v4i lo4(const v8i& x) { v4i r; r[0] = x[0]; r[1] = x[1]; r[2] = x[2]; r[3] = x[3]; return r; }
__device__ __forceinline__ v4i hi4(const v8i& x) { v4i r; r[0] = x[4]; r[1] = x[5]; r[2] = x[6]; r[3] = x[7]; return r; }

// LDS operand rows are 128 bytes (8 chunks of 16 B). Chunk c of row r sits at
// slot c ^ lds_swz(r), so the 16 lanes of one ds_read_b128 group (16
// consecutive rows, one chunk index) hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_swz(int row) { return (row >> 1) & 7; }

// Waits until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  // gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Makes x a value the compiler must have in a register here. Applied to
// loaded values after all loads of a batch are issued, it keeps the compiler
// from turning a select of a loaded value into a branch around the load
// (which it does otherwise, with a wait right after each such load).
template <class T>
__device__ __forceinline__ T settle(T x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Token rows of MFMA columns m[i] (block-relative index already added):
// brow is the activation row to read (a valid row even for padding), orow
// the output row, valid whether the result is stored. The MoE lookups of a
// batch go out together, without branches (an index past sorted_ids reads
// entry 0 and is then discarded; the launchers return before any kernel when
// sorted_ids is empty): one memory round trip for the batch.
template <bool MOE, int N, class P>
__device__ __forceinline__ void token_rows(const P& p, const int (&m)[N], int (&brow)[N], int (&orow)[N],
                                           bool (&valid)[N]) {
  if constexpr (MOE) {
    int raw[N];
#pragma unroll
    for (int i = 0; i < N; ++i) raw[i] = p.sorted_ids[(m[i] >= 0 && m[i] < p.sorted_len) ? m[i] : 0];
#pragma unroll
    for (int i = 0; i < N; ++i) raw[i] = settle(raw[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int sid = (m[i] >= 0 && m[i] < p.sorted_len) ? raw[i] : p.num_slots;
      valid[i] = sid >= 0 && sid < p.num_slots;
      brow[i] = valid[i] ? (int)((uint32_t)sid / (uint32_t)max(p.top_k, 1)) : 0;
      orow[i] = sid;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      valid[i] = m[i] >= 0 && m[i] < p.M;
      brow[i] = valid[i] ? m[i] : 0;
      orow[i] = m[i];
    }
  }
}
template <bool MOE, class P>
__device__ __forceinline__ void token_row(const P& p, int m, int& brow, int& orow, bool& valid) {
  const int mm[1] = {m};
  int br[1], orw[1];
  bool v[1];
  token_rows<MOE, 1>(p, mm, br, orw, v);
  brow = br[0];
  orow = orw[0];
  valid = v[0];
}

// Stores four consecutive output columns col0..col0+3 of row orow.
template <class P>
__device__ __forceinline__ void store4(const P& p, int orow, int col0, const float v[4]) {
  uint16_t* o = static_cast<uint16_t*>(p.out) + (int64_t)orow * p.ldo + col0;
  if (p.out_f16) {
    if (col0 + 3 < p.n_out) {
      *reinterpret_cast<uint2*>(o) = make_uint2(f32_to_f16_bits(v[0]) | (f32_to_f16_bits(v[1]) << 16),
                                                f32_to_f16_bits(v[2]) | (f32_to_f16_bits(v[3]) << 16));
    } else {
      for (int i = 0; i < 4; ++i)
        if (col0 + i < p.n_out) o[i] = (uint16_t)f32_to_f16_bits(v[i]);
    }
  } else {
    if (col0 + 3 < p.n_out) {
      *reinterpret_cast<uint2*>(o) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
      for (int i = 0; i < 4; ++i)
        if (col0 + i < p.n_out) o[i] = (uint16_t)f32_to_bf16_bits(v[i]);
    }
  }
}

template <class P>
__device__ __forceinline__ void store4_i32(const P& p, int orow, int col0, const int v[4]) {
  int* o = static_cast<int*>(p.out) + (int64_t)orow * p.ldo + col0;
  if (col0 + 3 < p.n_out) {
    *reinterpret_cast<int4*>(o) = make_int4(v[0], v[1], v[2], v[3]);
  } else {
    for (int i = 0; i < 4; ++i)
      if (col0 + i < p.n_out) o[i] = v[i];
  }
}

// Float epilogue of one lane's four results: act(g)*u when gated, times the
// slot's top-k weight (MoE, when given), then the store.
template <int EPI, int ACT, bool MOE, class P>
__device__ __forceinline__ void finish_float4_tw(const P& p, int orow, int col0, const float g[4], const float u[4],
                                                 float tw) {
  float v[4];
  if constexpr (EPI == kEpiGated) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = gate_act<ACT>(g[i]) * u[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = g[i];
  }
  if constexpr (MOE) {
    if (p.topk_w) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] *= tw;
    }
  }
  store4(p, orow, col0, v);
}
template <int EPI, int ACT, bool MOE, class P>
__device__ __forceinline__ void finish_float4(const P& p, int orow, int col0, const float g[4], const float u[4]) {
  const float tw = (MOE && p.topk_w) ? p.topk_w[orow] : 1.f;
  finish_float4_tw<EPI, ACT, MOE>(p, orow, col0, g, u, tw);
}

// An epilogue row of a tiled kernel (MFMA column m): output row, whether it
// is stored, and its top-k weight (MoE with weights; else 1). The tiled
// kernels load these before their K loop: loaded in the epilogue they would
// come one 16-row subtile at a time behind the previous subtile's stores.
struct EpiRow {
  int brow, orow;
  int valid;
  float tw;
};
// Epilogue rows of MFMA columns m[i]: the row lookups, then the top-k
// weights (one more round trip), each as one batch.
template <bool MOE, int N, class P>
__device__ __forceinline__ void epi_rows(const P& p, const int (&m)[N], EpiRow (&e)[N]) {
  int br[N], orw[N];
  bool v[N];
  token_rows<MOE, N>(p, m, br, orw, v);
  float w[N];
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = 1.f;
  if constexpr (MOE) {
    if (p.topk_w) {   // uniform; the loads are unconditional (slot 0 for padding rows)
#pragma unroll
      for (int i = 0; i < N; ++i) w[i] = p.topk_w[v[i] ? orw[i] : 0];
#pragma unroll
      for (int i = 0; i < N; ++i) w[i] = settle(w[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    e[i].brow = br[i];
    e[i].orow = orw[i];
    e[i].valid = v[i];
    e[i].tw = v[i] ? w[i] : 1.f;
  }
}
template <bool MOE, class P>
__device__ __forceinline__ EpiRow epi_row(const P& p, int m) {
  const int mm[1] = {m};
  EpiRow e[1];
  epi_rows<MOE, 1>(p, mm, e);
  return e[0];
}

// The hardware deals the blocks of a launch to the eight XCDs round robin
// (linear block b runs on XCD b % 8), and each XCD has its own L2.
// xcd_remap turns b into a logical block id such that each XCD gets a
// contiguous run of logical ids, for any block count: XCDs below nblk % 8
// take one more. A bijection of [0, nblk).
__device__ __forceinline__ int xcd_remap(int b, int nblk) {
  const int q = nblk >> 3, r = nblk & 7;
  const int x = b & 7, j = b >> 3;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + j;
}

// Maps a dense block index to (tile_m, tile_n): each XCD gets a contiguous
// run of tiles, walked in group_m-tall columns (tiles sharing a weight
// column run back to back).
__device__ __forceinline__ void dense_tile(int bid, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int nblk = tiles_m * tiles_n;
  const int b = xcd_remap(bid, nblk);
  const int per_group = group_m * tiles_n;
  const int grp = b / per_group;
  const int first_m = grp * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int in = b - grp * per_group;
  tm = first_m + in % gm;
  tn = in / gm;
}

// Expert of a decode kernel's row block blockIdx.y (-1: no routed rows):
// num_post and the block's expert id are loaded together, with no branch
// between them (expert_ids holds one entry per block of the grid, so the
// load is in bounds for every block), one memory round trip before the
// weight addresses are known instead of two.
__device__ __forceinline__ int moe_block_expert(const int32_t* num_post, const int32_t* expert_ids, int m0) {
  const int np = *num_post;
  const int ex = expert_ids[blockIdx.y];
  return m0 < np ? ex : -1;
}

// MoE tile (tm, tn) of this block in a grid of (column tiles, row tiles):
// only the row tiles holding routed rows (num_post of them, in tiles of bm,
// at most gridDim.y) are dealt out; blocks past them return false. Each XCD
// gets a contiguous run of row-major tiles, so the column tiles of one row
// tile (which read the same gathered token rows) and the row tiles of one
// expert (which read the same weights) run under one L2.
__device__ __forceinline__ bool moe_tile(int num_post, int bm, int& tm, int& tn) {
  const int gx = (int)gridDim.x;
  const int rows = min((num_post + bm - 1) / bm, (int)gridDim.y);
  const int active = rows * gx;
  const int b = (int)blockIdx.x + (int)blockIdx.y * gx;
  if (b >= active) return false;
  const int lg = xcd_remap(b, active);
  tm = lg / gx;
  tn = lg - tm * gx;
  return true;
}

}  // namespace strix
