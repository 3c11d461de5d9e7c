// SPDX-License-Identifier: MIT
// MoE plumbing around the expert GEMMs: router top-k, token alignment and the
// top-k combine. In the reference these three steps are vLLM's
// (fused_topk, moe_align_block_size, moe_sum: python/strix_vllm/moe.py:181-184,
// 286-288, 328-330); their contract is pinned by the reference's test
// restatement `align()` (tests/test_moe_gemm.py:9-31).
//
// Determinism: every index output here is a pure function of the inputs.
//   route:  top-k by logit value, larger first, lower expert index first on
//           ties (softmax is monotone, so this is the top-k of the probs).
//   align:  stable counting sort of slot ids by expert: within an expert the
//           slots appear in ascending order, each expert's run is padded to a
//           multiple of block_m with the id S = T*top_k.
#include <mutex>

#include "capi_internal.h"
#include "quant_common.h"
#include "strix_common.h"

namespace strix {
namespace {

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024

// Per-wave LDS scratch of the router: the k selected entries.
struct RouteScratch {
  uint32_t key[64];
  int id[64];
  float val[64];
};

// Order-preserving unsigned key of a float (-0 is keyed as +0, so the two
// tie like the reference's sort does).
__device__ __forceinline__ uint32_t float_key(float x) {
  const uint32_t b = __float_as_uint(x + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Top-k of one token's logits by one wave. Lane r < k ends with the r-th
// selected expert (by logit, larger first, lower expert id first on ties) in
// `my_id` and its softmax weight as the return value.
//
// The k-th largest key comes from a 32-step bisection over the key bits,
// each step one ballot per lane slot; the entries above it and the first
// ties by expert id are compacted (in expert order) into LDS, ranked there,
// and permuted into rank order. No step is a k-round argmax.
//
// PER = logits per lane (E <= 64 * PER): the loops are unrolled to exactly
// that, which keeps the code small; a kernel this short is bound by its own
// instruction fetch more than by its arithmetic.
template <bool BF16_LOGITS, int PER>
__device__ __forceinline__ float route_token(const void* __restrict__ logits, int64_t ldl, int t, int E, int k,
                                             int renorm, int& my_id, RouteScratch& sc) {
  const int lane = threadIdx.x & 63;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));  // lanes below this one
  constexpr int kMaxExpertsPerLane = PER;
  float v[kMaxExpertsPerLane];
  uint32_t key[kMaxExpertsPerLane];
  const int per = PER;
#pragma unroll
  for (int j = 0; j < kMaxExpertsPerLane; ++j) {
    const int e = lane + 64 * j;
    float x = -INFINITY;
    const bool in = j < per && e < E;
    if (in) {
      if constexpr (BF16_LOGITS)
        x = bf16_bits_to_f32(static_cast<const uint16_t*>(logits)[(int64_t)t * ldl + e]);
      else
        x = static_cast<const float*>(logits)[(int64_t)t * ldl + e];
    }
    v[j] = x;
    key[j] = in ? float_key(x) : 0u;
  }
  // K = the k-th largest key: the largest K with #(key >= K) >= k.
  uint32_t K = 0;
#pragma unroll 1
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = K | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kMaxExpertsPerLane; ++j)
      if (j < per) cnt += __popcll(__ballot(key[j] >= cand));
    if (cnt >= k) K = cand;
  }
  int above = 0;
#pragma unroll
  for (int j = 0; j < kMaxExpertsPerLane; ++j)
    if (j < per) above += __popcll(__ballot(key[j] > K));
  // Selected: every key above K, then the first (k - above) keys equal to K
  // in expert order; compacted into LDS in expert order.
  int ties_before = 0, sel_before = 0;
#pragma unroll
  for (int j = 0; j < kMaxExpertsPerLane; ++j) {
    if (j < per) {
      const uint64_t tie = __ballot(key[j] == K && key[j] != 0u);
      const bool is_tie = (tie >> lane) & 1ull;
      const int tie_rank = ties_before + __popcll(tie & lt);
      const bool sel = key[j] > K || (is_tie && tie_rank < k - above);
      const uint64_t selm = __ballot(sel);
      if (sel) {
        const int pos = sel_before + __popcll(selm & lt);
        sc.key[pos] = key[j];
        sc.id[pos] = lane + 64 * j;
        sc.val[pos] = v[j];
      }
      ties_before += __popcll(tie);
      sel_before += __popcll(selm);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  uint32_t mk = 0;
  int mid = 0;
  float mv = 0.0f;
  int rank = 0;
  if (lane < k) {
    mk = sc.key[lane];
    mid = sc.id[lane];
    mv = sc.val[lane];
    for (int q = 0; q < k; ++q) {
      const uint32_t kq = sc.key[q];
      rank += (kq > mk) || (kq == mk && sc.id[q] < mid);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (lane < k) {
    sc.id[rank] = mid;
    sc.val[rank] = mv;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const float mx = sc.val[0];
  my_id = lane < k ? sc.id[lane] : 0;
  const float my_v = lane < k ? sc.val[lane] : -INFINITY;
  const float my_e = lane < k ? __expf(my_v - mx) : 0.0f;
  float denom;
  if (renorm) {
    denom = wave_sum(my_e);
  } else {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxExpertsPerLane; ++j)
      if (j < per && lane + 64 * j < E) s += __expf(v[j] - mx);
    denom = wave_sum(s);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();  // the scratch is reused by the wave's next token
  return my_e / denom;
}

// One wave per token.
template <bool BF16_LOGITS, int PER>
__global__ void __launch_bounds__(256)
    route_topk_kernel(const void* __restrict__ logits, int64_t ldl, int T, int E, int k, int renorm,
                      int32_t* __restrict__ ids, float* __restrict__ wts, int64_t ldo) {
  __shared__ RouteScratch scratch[4];
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  int my_id = 0;
  const float w = route_token<BF16_LOGITS, PER>(logits, ldl, t, E, k, renorm, my_id, scratch[threadIdx.x >> 6]);
  if (lane < k) {
    ids[(int64_t)t * ldo + lane] = my_id;
    wts[(int64_t)t * ldo + lane] = w;
  }
}

// ---- align, small case: every step in one block of 1024 threads, the slot
// ids in LDS. Used up to kAlignSmall slots (decode and small prefill), where
// the three-pass path below is all launch latency.
constexpr int kAlignSmall = 1024;

// Inclusive sum over the block of one value per thread (1024 threads).
__device__ __forceinline__ int block_inclusive_sum(int x, int* wave_tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  if (threadIdx.x < 16) {
    int v = wave_tot[threadIdx.x];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(v, o, kWave);
      if ((int)threadIdx.x >= o) v += y;
    }
    wave_tot[threadIdx.x] = v;
  }
  __syncthreads();
  return x + (wave > 0 ? wave_tot[wave - 1] : 0);
}

// Align the S slot ids held in LDS `ids` (S <= 1024, E <= 1024). Same outputs
// as the three-pass path: stable within an expert, runs padded with S.
__device__ void align_block(const int32_t* ids, int S, int E, int block_m, int32_t* __restrict__ sorted_ids,
                            int64_t sorted_cap, int32_t* __restrict__ expert_ids, int64_t blocks_cap,
                            int32_t* __restrict__ num_post, int* cnt, int* off, int* wave_tot) {
  const int tid = threadIdx.x;
  if (tid < E) cnt[tid] = 0;
  __syncthreads();
  if (tid < S) {
    const int e = ids[tid];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  const int c = tid < E ? cnt[tid] : 0;
  const int padded = (c + block_m - 1) / block_m * block_m;
  const int incl = block_inclusive_sum(padded, wave_tot);
  if (tid < E) off[tid] = incl - padded;
  const int total = wave_tot[15];
  if (tid == 0) num_post[0] = total;
  __syncthreads();
  // Padding: each expert's tail and everything past the last run.
  if (tid < E) {
    for (int i = c; i < padded; ++i) sorted_ids[off[tid] + i] = S;
  }
  for (int64_t i = total + tid; i < sorted_cap; i += 1024) sorted_ids[i] = S;
  for (int64_t b = tid; b < blocks_cap; b += 1024) {
    int ex = -1;
    const int64_t pos = b * block_m;
    if (pos < total) {
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= pos) lo = mid; else hi = mid - 1;
      }
      while (lo < E - 1 && off[lo + 1] == off[lo]) ++lo;  // skip experts with no slots
      ex = lo;
    }
    expert_ids[b] = ex;
  }
  // Stable scatter: rank = earlier slots of the same expert, counted four
  // ids per LDS read with independent reads in flight.
  if (tid < S) {
    const int e = ids[tid];
    if (e >= 0 && e < E) {
      int rank = 0;
      const int4* v4 = reinterpret_cast<const int4*>(ids);
      const int n4 = tid >> 2;
#pragma unroll 8
      for (int j = 0; j < n4; ++j) {
        const int4 q = v4[j];
        rank += (q.x == e) + (q.y == e) + (q.z == e) + (q.w == e);
      }
      for (int j = n4 * 4; j < tid; ++j) rank += (ids[j] == e);
      sorted_ids[off[e] + rank] = tid;
    }
  }
}

// The tokens' e4m3 1x128 quantization that the single-block align and router
// kernels may do on the side (x == nullptr: none): x [T, K] bf16/fp16 -> q [T, K] e4m3, s [T, K/128].
struct ActQuant {
  const uint16_t* x;
  int64_t ldx;
  uint8_t* q;
  int64_t ldq;
  float* s;
  int64_t lds;
  int K;
  int f16;
};

// Threads [0, nthreads) of the block (whole waves) quantize rows [0, M).
__device__ __forceinline__ void quant_rows(const ActQuant& a, int M, int tid, int nthreads) {
  const uint32_t gpr = (uint32_t)(a.K >> 7), total = (uint32_t)M * gpr;
  const uint32_t per_pass = (uint32_t)nthreads >> 3;
  for (uint32_t base = 0; base < total; base += per_pass) {  // the same trip count in every lane
    const uint32_t grp = base + ((uint32_t)tid >> 3);
    const bool live = grp < total;
    const uint32_t m = live ? grp / gpr : 0u, g = live ? grp - m * gpr : 0u;
    if (a.f16) quant128_lane<true, true>(a.x, a.ldx, a.q, a.ldq, a.s, a.lds, m, g, tid & 7, live);
    else quant128_lane<false, true>(a.x, a.ldx, a.q, a.ldq, a.s, a.lds, m, g, tid & 7, live);
  }
}

// With `act`, the block quantizes the T token rows after the align (T <= 64,
// checked on the host).
__global__ void __launch_bounds__(1024)
    align_small_kernel(const int32_t* __restrict__ topk_ids, int S, int E, int block_m,
                       int32_t* __restrict__ sorted_ids, int64_t sorted_cap, int32_t* __restrict__ expert_ids,
                       int64_t blocks_cap, int32_t* __restrict__ num_post, ActQuant act, int T) {
  __shared__ __align__(16) int32_t ids[kAlignSmall];
  __shared__ int cnt[1024], off[1024], wave_tot[16];
  if ((int)threadIdx.x < S) ids[threadIdx.x] = topk_ids[threadIdx.x];
  __syncthreads();
  align_block(ids, S, E, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post, cnt, off, wave_tot);
  if (act.x != nullptr) quant_rows(act, T, threadIdx.x, 1024);
}


// Router and align in one block: 16 waves route the T tokens (T * k <= 1024),
// then the block aligns the slot ids it just produced. With `act`, the block
// also quantizes the T token rows: waves past the last token do it while the
// router runs (all 16 waves after the align when T is 16).
template <bool BF16_LOGITS, int PER>
__global__ void __launch_bounds__(1024)
    route_align_small_kernel(const void* __restrict__ logits, int64_t ldl, int T, int E, int k, int renorm,
                             int32_t* __restrict__ topk_ids, float* __restrict__ topk_w, int block_m,
                             int32_t* __restrict__ sorted_ids, int64_t sorted_cap, int32_t* __restrict__ expert_ids,
                             int64_t blocks_cap, int32_t* __restrict__ num_post, ActQuant act) {
  __shared__ __align__(16) int32_t ids[kAlignSmall];
  __shared__ int cnt[1024], off[1024], wave_tot[16];
  __shared__ RouteScratch scratch[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (act.x != nullptr && T < 16 && wave >= T) quant_rows(act, T, threadIdx.x - 64 * T, 64 * (16 - T));
  for (int t = wave; t < T; t += 16) {
    int my_id = 0;
    const float w = route_token<BF16_LOGITS, PER>(logits, ldl, t, E, k, renorm, my_id, scratch[wave]);
    if (lane < k) {
      ids[t * k + lane] = my_id;
      topk_ids[(int64_t)t * k + lane] = my_id;
      topk_w[(int64_t)t * k + lane] = w;
    }
  }
  __syncthreads();
  align_block(ids, T * k, E, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post, cnt, off, wave_tot);
  if (act.x != nullptr && T >= 16) quant_rows(act, T, threadIdx.x, 1024);
}

// ---- align, pass 1: per-chunk histograms. Chunk c covers slots [256c, 256c+256).
__global__ void __launch_bounds__(256)
    align_hist_kernel(const int32_t* __restrict__ topk_ids, int S, int E, int32_t* __restrict__ hist) {
  extern __shared__ int32_t h[];
  for (int e = threadIdx.x; e < E; e += 256) h[e] = 0;
  __syncthreads();
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s < S) {
    const int e = topk_ids[s];
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) hist[(int64_t)blockIdx.x * E + e] = h[e];
}

// ---- align, pass 2 (one block): expert offsets, per-chunk bases (in place
// over hist), expert_ids, num_post_padded and the padding fill. Thread
// (part, e) owns expert e's chunks [part*cpp, (part+1)*cpp): its loads are
// independent and coalesced across e, and the only serial step is a block
// scan over the E padded counts.
__global__ void __launch_bounds__(1024)
    align_scan_kernel(int32_t* __restrict__ hist, int chunks, int S, int E, int block_m,
                      int32_t* __restrict__ sorted_ids, int64_t sorted_cap, int32_t* __restrict__ expert_ids,
                      int64_t blocks_cap, int32_t* __restrict__ num_post) {
  extern __shared__ int32_t sm[];  // [parts][E] partial counts, [E] offsets, [16] wave totals, [E] counts
  const int parts = max(1, 1024 / E);
  const int cpp = (chunks + parts - 1) / parts;
  int32_t* psum = sm;
  int32_t* off = sm + parts * E;
  int32_t* wave_tot = off + E;
  const int tid = threadIdx.x;
  const int e = tid % E, part = tid / E;
  const bool owner = part < parts && tid < parts * E;
  const int c0 = owner ? part * cpp : 0, c1 = owner ? min(chunks, c0 + cpp) : 0;
  // Experts beyond 1024 threads: one thread walks several (E > 1024 is rejected on the host).
  int local = 0;
  {
    int c = c0;
    for (; c + 8 <= c1; c += 8) {
      int h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = hist[(int64_t)(c + j) * E + e];
#pragma unroll
      for (int j = 0; j < 8; ++j) local += h[j];
    }
    for (; c < c1; ++c) local += hist[(int64_t)c * E + e];
  }
  if (owner) psum[part * E + e] = local;
  __syncthreads();
  int cnt = 0;
  if (tid < E)
    for (int q = 0; q < parts; ++q) cnt += psum[q * E + tid];
  const int padded = tid < E ? (cnt + block_m - 1) / block_m * block_m : 0;
  const int incl = block_inclusive_sum(padded, wave_tot);
  if (tid < E) off[tid] = incl - padded;
  const int total = wave_tot[15];
  if (tid == 0) num_post[0] = total;
  __syncthreads();
  // Padding fill: each expert's tail, `parts` threads per expert striding over
  // it, then everything past the last run (disjoint from the slots the scatter
  // pass writes). Counts go through LDS, since thread e owns count e.
  int32_t* cnt_l = wave_tot + 16;
  if (tid < E) cnt_l[tid] = cnt;
  __syncthreads();
  if (tid < parts * E) {
    const int pe = tid / parts, pq = tid - pe * parts;
    const int c2 = cnt_l[pe];
    const int pad2 = (c2 + block_m - 1) / block_m * block_m;
    for (int i = c2 + pq; i < pad2; i += parts) sorted_ids[off[pe] + i] = S;
  }
  for (int64_t i = total + tid; i < sorted_cap; i += 1024) sorted_ids[i] = S;
  for (int64_t b = tid; b < blocks_cap; b += 1024) {
    int ex = -1;
    const int64_t pos = b * block_m;
    if (pos < total) {  // binary search: last expert whose offset <= pos
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= pos) lo = mid; else hi = mid - 1;
      }
      while (lo < E - 1 && off[lo + 1] == off[lo]) ++lo;  // skip experts with no slots
      ex = lo;
    }
    expert_ids[b] = ex;
  }
  // Chunk bases: expert offset + this part's predecessors + running count.
  // Eight chunks' counts are loaded before any base is written back, so the
  // walk pays one memory latency per eight chunks.
  if (owner) {
    int run = off[e];
    for (int q = 0; q < part; ++q) run += psum[q * E + e];
    int c = c0;
    for (; c + 8 <= c1; c += 8) {
      int h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = hist[(int64_t)(c + j) * E + e];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        hist[(int64_t)(c + j) * E + e] = run;
        run += h[j];
      }
    }
    for (; c < c1; ++c) {
      const int64_t i = (int64_t)c * E + e;
      const int n = hist[i];
      hist[i] = run;
      run += n;
    }
  }
}

// ---- align, pass 3: stable scatter. Slot s goes to base[c][e] + (number of
// earlier slots of chunk c routed to e).
__global__ void __launch_bounds__(256)
    align_scatter_kernel(const int32_t* __restrict__ topk_ids, int S, int E, const int32_t* __restrict__ base,
                         int32_t* __restrict__ sorted_ids) {
  __shared__ int32_t ex[256];
  const int s = blockIdx.x * 256 + threadIdx.x;
  const int e = s < S ? topk_ids[s] : -1;
  ex[threadIdx.x] = e;
  __syncthreads();
  if (s >= S || e < 0 || e >= E) return;
  int rank = 0;
  for (int j = 0; j < (int)threadIdx.x; ++j) rank += (ex[j] == e);
  sorted_ids[base[(int64_t)blockIdx.x * E + e] + rank] = s;
}

// out[t, :] = sum_j y[t*k + j, :] (j ascending, fp32), optionally weighted.
template <bool F16>
__global__ void __launch_bounds__(256)
    moe_sum_kernel(const uint16_t* __restrict__ y, int64_t ldy, int T, int k, int H,
                   const float* __restrict__ w, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int hv = H / 8;
  const int64_t t = idx / hv;
  if (t >= T) return;
  const int h = (int)(idx % hv) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // Four rows' loads in flight before any is used; the sum stays in row order.
  for (int j0 = 0; j0 < k; j0 += 4) {
    u32x4 raw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (j0 + q < k) raw[q] = *reinterpret_cast<const u32x4*>(y + (t * k + j0 + q) * ldy + h);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (j0 + q >= k) break;
      const float wj = w ? w[t * k + j0 + q] : 1.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = act_to_f32<F16>(raw[q][i] & 0xffffu), hi = act_to_f32<F16>(raw[q][i] >> 16);
        if (w) {
          acc[2 * i] = fmaf(wj, lo, acc[2 * i]);
          acc[2 * i + 1] = fmaf(wj, hi, acc[2 * i + 1]);
        } else {
          acc[2 * i] += lo;
          acc[2 * i + 1] += hi;
        }
      }
    }
  }
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32_to_act_bits<F16>(acc[2 * i]) | (f32_to_act_bits<F16>(acc[2 * i + 1]) << 16);
  *reinterpret_cast<u32x4*>(out + t * ldo + h) = o;
}

// Logits per lane for E experts (the router's unroll), and the logits type.
template <class F>
void per_dispatch(int64_t E, bool bf16, F&& go) {
  auto with = [&](auto per_tag) {
    if (bf16) go(std::true_type{}, per_tag);
    else go(std::false_type{}, per_tag);
  };
  if (E <= 64) with(std::integral_constant<int, 1>{});
  else if (E <= 128) with(std::integral_constant<int, 2>{});
  else if (E <= 256) with(std::integral_constant<int, 4>{});
  else if (E <= 512) with(std::integral_constant<int, 8>{});
  else with(std::integral_constant<int, kMaxExpertsPerLane>{});
}

}  // namespace
}  // namespace strix

using namespace strix;

extern "C" {

int strix_moe_route_topk(const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E,
                         int64_t top_k, int renormalize, int32_t* topk_ids, float* topk_weights,
                         int64_t ldo, void* stream) {
  const char* op = "moe_route_topk";
  STRIX_REQUIRE(logits_dtype == STRIX_F32 || logits_dtype == STRIX_BF16, "%s: logits must be float32 or bfloat16", op);
  STRIX_REQUIRE(E >= 1 && E <= 64 * kMaxExpertsPerLane, "%s: 1 <= E <= %d, got E=%lld", op,
                64 * kMaxExpertsPerLane, (long long)E);
  STRIX_REQUIRE(top_k >= 1 && top_k <= 64 && top_k <= E, "%s: 1 <= top_k <= min(E, 64), got %lld", op,
                (long long)top_k);
  STRIX_REQUIRE(ldl >= E && ldo >= top_k && T >= 0, "%s: bad strides", op);
  if (T == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  const unsigned blocks = (unsigned)((T + 3) / 4);
  auto go = [&](auto bf16_tag, auto per_tag) {
    constexpr bool BF = decltype(bf16_tag)::value;
    constexpr int PER = decltype(per_tag)::value;
    hipLaunchKernelGGL((route_topk_kernel<BF, PER>), dim3(blocks), dim3(256), 0, as_stream(stream), logits, ldl,
                       (int)T, (int)E, (int)top_k, renormalize, topk_ids, topk_weights, ldo);
  };
  per_dispatch(E, logits_dtype == STRIX_BF16, go);
  return check_launch(op);
}

int64_t strix_moe_align_sorted_capacity(int64_t num_slots, int64_t E, int64_t block_m) {
  return num_slots + E * (block_m - 1);
}

int64_t strix_moe_align_workspace_bytes(int64_t num_slots, int64_t E) {
  const int64_t chunks = (num_slots + 255) / 256;
  return (chunks > 0 ? chunks : 1) * E * 4;
}

}  // extern "C"

namespace strix {
namespace {

int align_impl(const char* op, const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
               int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap, int32_t* num_post,
               void* workspace, int64_t workspace_bytes, const ActQuant& act, int64_t T, int x_dtype, void* stream) {
  STRIX_REQUIRE(E >= 1 && E <= 1024, "%s: 1 <= E <= 1024, got %lld", op, (long long)E);
  STRIX_REQUIRE(block_m >= 1 && block_m <= 1024, "%s: block_m must be in 1..1024", op);
  STRIX_REQUIRE(num_slots >= 0 && num_slots < INT32_MAX / 2, "%s: bad slot count", op);
  STRIX_REQUIRE(sorted_cap >= strix_moe_align_sorted_capacity(num_slots, E, block_m),
                "%s: sorted_ids needs %lld entries", op,
                (long long)strix_moe_align_sorted_capacity(num_slots, E, block_m));
  STRIX_REQUIRE(blocks_cap * block_m >= sorted_cap, "%s: expert_ids needs ceil(capacity / block_m) entries", op);
  STRIX_REQUIRE(workspace_bytes >= strix_moe_align_workspace_bytes(num_slots, E), "%s: workspace too small", op);
  STRIX_ARCH_GATE();
  hipStream_t st = as_stream(stream);
  const int S = (int)num_slots;
  // One block also quantizes up to 64 token rows (at most 8 passes of its
  // threads); more rows, or more slots, take the separate quantizer.
  const bool fuse = act.x != nullptr && T <= 64;
  if (S <= kAlignSmall) {
    const ActQuant none = {};
    hipLaunchKernelGGL(align_small_kernel, dim3(1), dim3(1024), 0, st, topk_ids, S, (int)E, (int)block_m, sorted_ids,
                       sorted_cap, expert_ids, blocks_cap, num_post, fuse ? act : none, (int)T);
    int rc = check_launch(op);
    if (rc || fuse || act.x == nullptr) return rc;
    return strix_fp8_quant_group128(act.x, x_dtype, act.ldx, act.q, act.ldq, act.s, act.lds, T, act.K, stream);
  }
  const int chunks = (S + 255) / 256;
  int32_t* hist = static_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(align_hist_kernel, dim3(chunks), dim3(256), (size_t)E * 4, st, topk_ids, S, (int)E, hist);
  int rc = check_launch(op);
  if (rc) return rc;
  const int parts = (int)std::max<int64_t>(1, 1024 / E);
  const size_t scan_lds = ((size_t)parts * E + 2 * E + 16) * 4;
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(1024), scan_lds, st, hist, chunks, S, (int)E,
                     (int)block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post);
  rc = check_launch(op);
  if (rc) return rc;
  hipLaunchKernelGGL(align_scatter_kernel, dim3(chunks), dim3(256), 0, st, topk_ids, S, (int)E, hist, sorted_ids);
  rc = check_launch(op);
  if (rc || act.x == nullptr) return rc;
  return strix_fp8_quant_group128(act.x, x_dtype, act.ldx, act.q, act.ldq, act.s, act.lds, T, act.K, stream);
}

// Checks the activation-quantizer arguments of the *_quant entry points and
// packs them.
int make_act_quant(const char* op, const void* x, int x_dtype, int64_t ldx, uint8_t* q, int64_t ldq, float* s,
                   int64_t lds, int64_t K, ActQuant& act) {
  STRIX_REQUIRE(x != nullptr && q != nullptr && s != nullptr, "%s: x, q and s are required", op);
  STRIX_REQUIRE(x_dtype == STRIX_BF16 || x_dtype == STRIX_F16, "%s: activation must be float16 or bfloat16", op);
  STRIX_REQUIRE(K > 0 && K % 128 == 0 && K <= INT32_MAX, "%s: K must be a positive multiple of 128, got K=%lld", op,
                (long long)K);
  STRIX_REQUIRE(ldx >= K && ldx % 8 == 0 && ldq >= K && ldq % 8 == 0 && lds >= K / 128,
                "%s: activation, output and scale row strides must cover K (multiples of 8)", op);
  STRIX_REQUIRE(aligned(x, 16) && aligned(q, 8), "%s: activation must be 16-byte aligned and output 8-byte aligned",
                op);
  act.x = static_cast<const uint16_t*>(x);
  act.ldx = ldx;
  act.q = q;
  act.ldq = ldq;
  act.s = s;
  act.lds = lds;
  act.K = (int)K;
  act.f16 = x_dtype == STRIX_F16;
  return STRIX_OK;
}

}  // namespace
}  // namespace strix

extern "C" {

int strix_moe_align(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                    int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                    int32_t* num_post, void* workspace, int64_t workspace_bytes, void* stream) {
  const ActQuant none = {};
  return align_impl("moe_align", topk_ids, num_slots, E, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap,
                    num_post, workspace, workspace_bytes, none, 0, STRIX_BF16, stream);
}

int strix_moe_align_quant(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                          int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                          int32_t* num_post, void* workspace, int64_t workspace_bytes, const void* x, int x_dtype,
                          int64_t ldx, uint8_t* q, int64_t ldq, float* s, int64_t lds, int64_t T, int64_t K,
                          void* stream) {
  const char* op = "moe_align_quant";
  ActQuant act;
  int rc = make_act_quant(op, x, x_dtype, ldx, q, ldq, s, lds, K, act);
  if (rc) return rc;
  STRIX_REQUIRE(T >= 0 && T <= num_slots, "%s: bad token count", op);
  return align_impl(op, topk_ids, num_slots, E, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post,
                    workspace, workspace_bytes, act, T, x_dtype, stream);
}

}  // extern "C"

// ------------------------------------------------------------ no-allocation align
// The align's histogram workspace as a device array of the library, for
// callers that cannot allocate (HIP graph capture, serving loops). Each GPU
// holds its own copy for the life of the process. Every call on a GPU shares
// it, so calls that overlap on one GPU (different streams, different host
// threads) race. Nothing in it must start at zero: pass 1 writes every
// (chunk, expert) count before pass 2 reads it.
namespace strix {
namespace {

constexpr int64_t kAlignScratchBytes = int64_t(1) << 20;  // 1 MiB: chunks(num_slots) * E <= 262144
__device__ __align__(256) int32_t scratch[kAlignScratchBytes / 4];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};  // device address of `scratch` per device, set on first use

// Device address of this device's `scratch` (looked up once per device, with
// that device current). In host code the array's name is only a stand-in, so
// kernels always receive this address.
int align_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(STRIX_ERR_DEVICE, "moe_align_noalloc: no usable current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(STRIX_ERR_DEVICE, "moe_align_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return STRIX_OK;
}

}  // namespace
}  // namespace strix

extern "C" {

int64_t strix_moe_align_noalloc_max_bytes(void) { return strix::kAlignScratchBytes; }

int strix_moe_align_noalloc(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                            int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                            int32_t* num_post, void* stream) {
  const char* op = "moe_align_noalloc";
  STRIX_REQUIRE(E >= 1 && E <= 1024, "%s: 1 <= E <= 1024, got %lld", op, (long long)E);
  STRIX_REQUIRE(num_slots >= 0 && num_slots < INT32_MAX / 2, "%s: bad slot count", op);
  const int64_t need = strix_moe_align_workspace_bytes(num_slots, E);
  STRIX_REQUIRE(need <= strix::kAlignScratchBytes,
                "%s: %lld slots x %lld experts need %lld bytes of histogram, over the %lld-byte static scratch; "
                "use strix_moe_align with a workspace",
                op, (long long)num_slots, (long long)E, (long long)need, (long long)strix::kAlignScratchBytes);
  STRIX_ARCH_GATE();
  void* ws = nullptr;
  int rc = strix::align_scratch(&ws);
  if (rc) return rc;
  const strix::ActQuant none = {};
  return strix::align_impl(op, topk_ids, num_slots, E, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap,
                           num_post, ws, strix::kAlignScratchBytes, none, 0, STRIX_BF16, stream);
}

}  // extern "C"

namespace strix {
namespace {

int route_align_impl(const char* op, const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E,
                     int64_t top_k, int renormalize, int32_t* topk_ids, float* topk_weights, int64_t block_m,
                     int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                     int32_t* num_post, void* workspace, int64_t workspace_bytes, const ActQuant& act,
                     int x_dtype, void* stream) {
  // One block routes at most one token per wave (16 tokens) before the
  // separate, grid-wide router is faster.
  if (T * top_k > kAlignSmall || T > 16 || T == 0) {
    int rc = strix_moe_route_topk(logits, logits_dtype, ldl, T, E, top_k, renormalize, topk_ids, topk_weights, top_k,
                                  stream);
    if (rc) return rc;
    rc = strix_moe_align(topk_ids, T * top_k, E, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post,
                         workspace, workspace_bytes, stream);
    if (rc || act.x == nullptr) return rc;
    return strix_fp8_quant_group128(act.x, x_dtype, act.ldx, act.q, act.ldq, act.s, act.lds, T, act.K, stream);
  }
  STRIX_REQUIRE(logits_dtype == STRIX_F32 || logits_dtype == STRIX_BF16, "%s: logits must be float32 or bfloat16", op);
  STRIX_REQUIRE(E >= 1 && E <= 64 * kMaxExpertsPerLane, "%s: 1 <= E <= %d, got E=%lld", op,
                64 * kMaxExpertsPerLane, (long long)E);
  STRIX_REQUIRE(top_k >= 1 && top_k <= 64 && top_k <= E, "%s: 1 <= top_k <= min(E, 64), got %lld", op,
                (long long)top_k);
  STRIX_REQUIRE(ldl >= E, "%s: bad logits stride", op);
  STRIX_REQUIRE(block_m >= 1 && block_m <= 1024, "%s: block_m must be in 1..1024", op);
  STRIX_REQUIRE(sorted_cap >= strix_moe_align_sorted_capacity(T * top_k, E, block_m), "%s: sorted_ids too small", op);
  STRIX_REQUIRE(blocks_cap * block_m >= sorted_cap, "%s: expert_ids needs ceil(capacity / block_m) entries", op);
  STRIX_ARCH_GATE();
  auto go = [&](auto bf16_tag, auto per_tag) {
    constexpr bool BF = decltype(bf16_tag)::value;
    constexpr int PER = decltype(per_tag)::value;
    hipLaunchKernelGGL((route_align_small_kernel<BF, PER>), dim3(1), dim3(1024), 0, as_stream(stream), logits, ldl,
                       (int)T, (int)E, (int)top_k, renormalize, topk_ids, topk_weights, (int)block_m, sorted_ids,
                       sorted_cap, expert_ids, blocks_cap, num_post, act);
  };
  per_dispatch(E, logits_dtype == STRIX_BF16, go);
  return check_launch(op);
}

}  // namespace
}  // namespace strix

extern "C" {

int strix_moe_route_align(const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E, int64_t top_k,
                          int renormalize, int32_t* topk_ids, float* topk_weights, int64_t block_m,
                          int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                          int32_t* num_post, void* workspace, int64_t workspace_bytes, void* stream) {
  const ActQuant none = {};
  return route_align_impl("moe_route_align", logits, logits_dtype, ldl, T, E, top_k, renormalize, topk_ids,
                          topk_weights, block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post, workspace,
                          workspace_bytes, none, STRIX_BF16, stream);
}

int strix_moe_route_align_quant(const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E,
                                int64_t top_k, int renormalize, int32_t* topk_ids, float* topk_weights,
                                int64_t block_m, int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids,
                                int64_t blocks_cap, int32_t* num_post, void* workspace, int64_t workspace_bytes,
                                const void* x, int x_dtype, int64_t ldx, uint8_t* q, int64_t ldq, float* s,
                                int64_t lds, int64_t K, void* stream) {
  const char* op = "moe_route_align_quant";
  ActQuant act;
  int rc = make_act_quant(op, x, x_dtype, ldx, q, ldq, s, lds, K, act);
  if (rc) return rc;
  return route_align_impl(op, logits, logits_dtype, ldl, T, E, top_k, renormalize, topk_ids, topk_weights, block_m,
                          sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post, workspace, workspace_bytes, act,
                          x_dtype, stream);
}

int strix_moe_sum(const void* y, int dtype, int64_t ldy, int64_t T, int64_t top_k, int64_t H,
                  const float* weights, void* out, int64_t ldo, void* stream) {
  const char* op = "moe_sum";
  STRIX_REQUIRE(dtype == STRIX_BF16 || dtype == STRIX_F16, "%s: input must be bfloat16 or float16", op);
  STRIX_REQUIRE(H % 8 == 0 && ldy % 8 == 0 && ldo % 8 == 0, "%s: hidden size and strides must be multiples of 8", op);
  STRIX_REQUIRE(aligned(y, 16) && aligned(out, 16), "%s: buffers must be 16-byte aligned", op);
  STRIX_REQUIRE(T >= 0 && top_k >= 1 && ldy >= H && ldo >= H, "%s: bad sizes", op);
  if (T == 0 || H == 0) return STRIX_OK;
  STRIX_ARCH_GATE();
  const int64_t n = T * (H / 8);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  const uint16_t* yp = static_cast<const uint16_t*>(y);
  uint16_t* op_ = static_cast<uint16_t*>(out);
  if (dtype == STRIX_F16)
    hipLaunchKernelGGL(moe_sum_kernel<true>, dim3(blocks), dim3(256), 0, as_stream(stream), yp, ldy, (int)T,
                       (int)top_k, (int)H, weights, op_, ldo);
  else
    hipLaunchKernelGGL(moe_sum_kernel<false>, dim3(blocks), dim3(256), 0, as_stream(stream), yp, ldy, (int)T,
                       (int)top_k, (int)H, weights, op_, ldo);
  return check_launch(op);
}

}  // extern "C"
