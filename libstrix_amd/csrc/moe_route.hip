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
#include "capi_internal.h"
#include "strix_common.h"

namespace strix {
namespace {

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024

// One wave per token.
template <bool BF16_LOGITS>
__global__ void __launch_bounds__(256)
    route_topk_kernel(const void* __restrict__ logits, int64_t ldl, int T, int E, int k, int renorm,
                      int32_t* __restrict__ ids, float* __restrict__ wts, int64_t ldo) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float v[kMaxExpertsPerLane];
  const int per = (E + 63) / 64;
#pragma unroll
  for (int j = 0; j < kMaxExpertsPerLane; ++j) {
    const int e = lane + 64 * j;
    float x = -INFINITY;
    if (j < per && e < E) {
      if constexpr (BF16_LOGITS)
        x = bf16_bits_to_f32(static_cast<const uint16_t*>(logits)[(int64_t)t * ldl + e]);
      else
        x = static_cast<const float*>(logits)[(int64_t)t * ldl + e];
    }
    v[j] = x;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxExpertsPerLane; ++j) mx = fmaxf(mx, v[j]);
  mx = wave_max(mx);
  float denom_all = 0.0f;
  if (!renorm) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxExpertsPerLane; ++j)
      if (j < per && lane + 64 * j < E) s += __expf(v[j] - mx);
    denom_all = wave_sum(s);
  }
  uint32_t taken = 0;  // bit j: element j of this lane already selected
  float sel_sum = 0.0f;
  float my_e = 0.0f;   // lane r keeps exp(sel_r - mx)
  int my_id = 0;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kMaxExpertsPerLane; ++j) {
      const int e = lane + 64 * j;
      if (j < per && e < E && !((taken >> j) & 1u)) {
        if (v[j] > bv || (v[j] == bv && e < bi)) { bv = v[j]; bi = e; }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    const float ev = __expf(bv - mx);
    sel_sum += ev;
    if (lane == r) { my_e = ev; my_id = bi; }
  }
  if (lane < k) {
    ids[(int64_t)t * ldo + lane] = my_id;
    wts[(int64_t)t * ldo + lane] = renorm ? my_e / sel_sum : my_e / denom_all;
  }
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
// over hist), expert_ids, num_post_padded and the padding fill.
__global__ void __launch_bounds__(1024)
    align_scan_kernel(int32_t* __restrict__ hist, int chunks, int S, int E, int block_m,
                      int32_t* __restrict__ sorted_ids, int64_t sorted_cap, int32_t* __restrict__ expert_ids,
                      int64_t blocks_cap, int32_t* __restrict__ num_post) {
  extern __shared__ int32_t sm[];  // [E] padded counts, then [E] offsets
  int32_t* padded = sm;
  int32_t* off = sm + E;
  for (int e = threadIdx.x; e < E; e += 1024) {
    int cnt = 0;
    for (int c = 0; c < chunks; ++c) cnt += hist[(int64_t)c * E + e];
    padded[e] = (cnt + block_m - 1) / block_m * block_m;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // E <= 1024: a serial scan is a few microseconds at most
    int run = 0;
    for (int e = 0; e < E; ++e) { off[e] = run; run += padded[e]; }
    num_post[0] = run;
  }
  __syncthreads();
  const int total = off[E - 1] + padded[E - 1];
  for (int64_t i = threadIdx.x; i < sorted_cap; i += 1024) sorted_ids[i] = S;
  for (int64_t b = threadIdx.x; b < blocks_cap; b += 1024) {
    int ex = -1;
    const int64_t pos = b * block_m;
    if (pos < total) {  // binary search: last expert whose offset <= pos
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= pos) lo = mid; else hi = mid - 1;
      }
      // Experts with zero slots share the offset of the next; skip to the one that owns pos.
      while (lo < E - 1 && padded[lo] == 0) ++lo;
      ex = lo;
    }
    expert_ids[b] = ex;
  }
  for (int e = threadIdx.x; e < E; e += 1024) {
    int run = off[e];
    for (int c = 0; c < chunks; ++c) {
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
  for (int j = 0; j < k; ++j) {
    const u32x4 raw = *reinterpret_cast<const u32x4*>(y + (t * k + j) * ldy + h);
    const float wj = w ? w[t * k + j] : 1.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = act_to_f32<F16>(raw[i] & 0xffffu), hi = act_to_f32<F16>(raw[i] >> 16);
      if (w) {
        acc[2 * i] = fmaf(wj, lo, acc[2 * i]);
        acc[2 * i + 1] = fmaf(wj, hi, acc[2 * i + 1]);
      } else {
        acc[2 * i] += lo;
        acc[2 * i + 1] += hi;
      }
    }
  }
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f32_to_act_bits<F16>(acc[2 * i]) | (f32_to_act_bits<F16>(acc[2 * i + 1]) << 16);
  *reinterpret_cast<u32x4*>(out + t * ldo + h) = o;
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
  if (logits_dtype == STRIX_BF16)
    hipLaunchKernelGGL(route_topk_kernel<true>, dim3(blocks), dim3(256), 0, as_stream(stream), logits, ldl,
                       (int)T, (int)E, (int)top_k, renormalize, topk_ids, topk_weights, ldo);
  else
    hipLaunchKernelGGL(route_topk_kernel<false>, dim3(blocks), dim3(256), 0, as_stream(stream), logits, ldl,
                       (int)T, (int)E, (int)top_k, renormalize, topk_ids, topk_weights, ldo);
  return check_launch(op);
}

int64_t strix_moe_align_sorted_capacity(int64_t num_slots, int64_t E, int64_t block_m) {
  return num_slots + E * (block_m - 1);
}

int64_t strix_moe_align_workspace_bytes(int64_t num_slots, int64_t E) {
  const int64_t chunks = (num_slots + 255) / 256;
  return (chunks > 0 ? chunks : 1) * E * 4;
}

int strix_moe_align(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                    int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                    int32_t* num_post, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* op = "moe_align";
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
  const int chunks = S > 0 ? (S + 255) / 256 : 1;
  int32_t* hist = static_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(align_hist_kernel, dim3(chunks), dim3(256), (size_t)E * 4, st, topk_ids, S, (int)E, hist);
  int rc = check_launch(op);
  if (rc) return rc;
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(1024), (size_t)E * 8, st, hist, chunks, S, (int)E,
                     (int)block_m, sorted_ids, sorted_cap, expert_ids, blocks_cap, num_post);
  rc = check_launch(op);
  if (rc) return rc;
  if (S == 0) return STRIX_OK;
  hipLaunchKernelGGL(align_scatter_kernel, dim3(chunks), dim3(256), 0, st, topk_ids, S, (int)E, hist, sorted_ids);
  return check_launch(op);
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
