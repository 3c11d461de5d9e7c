// SPDX-License-Identifier: MIT
// torch.ops.strix.* in C++ for the ops on the configurations' call chains: the
// W8A8 quantizers and GEMMs (configs 1, 2), the K-block-major re-layout, the
// MoE router / align / combine and the expert GEMMs of configs 3-5.
//
// The reference registers its ops the same way (csrc/torch_ops.cpp:179-344:
// TORCH_LIBRARY schemas, CUDA-key impls under a device guard on the current
// stream). Each impl here checks its arguments with the messages of the
// Python registration, allocates outputs with the caching allocator and calls
// the C ABI of libstrix_amd/_strix_amd.so (include/strix_amd.h), which it is
// linked against. Nothing syncs the host, so the ops stay graph-capturable.
// The schemas are the same strings the Python layer holds (a test compares
// them); fake (meta) kernels are registered from Python.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <optional>
#include <string>

#include "strix_amd.h"

namespace {

using at::Tensor;

void call(int rc, const char* op) {
  TORCH_CHECK(rc == STRIX_OK, strix_last_error()[0] ? strix_last_error() : op);
}

void* stream_of(const Tensor& t) {
  return reinterpret_cast<void*>(at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

int act_code(const Tensor& t) {
  if (t.scalar_type() == at::kBFloat16) return STRIX_BF16;
  if (t.scalar_type() == at::kHalf) return STRIX_F16;
  TORCH_CHECK(false, "Activation must be float16 or bfloat16, got ", t.scalar_type());
}

int out_code(at::ScalarType s) {
  if (s == at::kBFloat16) return STRIX_BF16;
  if (s == at::kHalf) return STRIX_F16;
  TORCH_CHECK(s == at::kInt, "unsupported output dtype ", s);
  return STRIX_I32;
}

int activation_code(const std::string& a) {
  TORCH_CHECK(a == "silu" || a == "gelu_tanh", "activation must be 'silu' or 'gelu_tanh', got '", a, "'");
  return a == "silu" ? 0 : 1;
}

bool unit_last(const Tensor& t) { return t.size(-1) == 1 || t.stride(-1) == 1; }

void rowmajor(const Tensor& t, const char* what) {
  TORCH_CHECK(t.dim() == 2 && t.stride(1) == 1, what, " must be 2-D and contiguous in dim 1");
}

std::pair<int64_t, int64_t> align_capacity(int64_t slots, int64_t experts, int64_t block_m) {
  const int64_t cap = slots + experts * (block_m - 1);
  return {cap, (cap + block_m - 1) / block_m};
}

// ---------------------------------------------------------------- quantizers
std::tuple<Tensor, Tensor> int8_quant_per_token(const Tensor& x) {
  rowmajor(x, "x");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  const int64_t m = x.size(0), k = x.size(1);
  Tensor q = at::empty({m, k}, x.options().dtype(at::kChar));
  Tensor s = at::empty({m}, x.options().dtype(at::kFloat));
  call(strix_int8_quant_per_token(x.data_ptr(), act_code(x), x.stride(0), static_cast<int8_t*>(q.data_ptr()), k,
                                  s.data_ptr<float>(), m,
                                  k, stream_of(x)),
       "int8_quant_per_token");
  return {q, s};
}

std::tuple<Tensor, Tensor> fp8_quant_group128(const Tensor& x) {
  rowmajor(x, "x");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  const int64_t m = x.size(0), k = x.size(1);
  Tensor q = at::empty({m, k}, x.options().dtype(at::kFloat8_e4m3fn));
  Tensor s = at::empty({m, k / 128}, x.options().dtype(at::kFloat));
  call(strix_fp8_quant_group128(x.data_ptr(), act_code(x), x.stride(0), static_cast<uint8_t*>(q.data_ptr()), k,
                                s.data_ptr<float>(), std::max<int64_t>(k / 128, 1), m, k, stream_of(x)),
       "fp8_quant_group128");
  return {q, s};
}

// ---------------------------------------------------------------- W8A8 GEMMs
Tensor i8_gemm(const Tensor& qa, const std::optional<Tensor>& sa, const Tensor& w, const std::optional<Tensor>& sw,
               at::ScalarType out_dtype, int64_t cfg) {
  rowmajor(qa, "qa");
  rowmajor(w, "w");
  TORCH_CHECK(qa.scalar_type() == at::kChar && w.scalar_type() == at::kChar, "qa and w must be int8");
  const int64_t m = qa.size(0), k = qa.size(1), n = w.size(0);
  TORCH_CHECK(w.size(1) == k, "Activation K (", k, ") must match weight K (", w.size(1), ")");
  std::optional<Tensor> sac, swc;
  if (sa.has_value()) {
    TORCH_CHECK(sa->scalar_type() == at::kFloat && sa->numel() == m, "sa must be float32 [M]");
    TORCH_CHECK(sw.has_value() && sw->scalar_type() == at::kFloat && sw->numel() == n, "sw must be float32 [N]");
    sac = sa->contiguous();
    swc = sw->contiguous();
  }
  const at::hip::HIPGuardMasqueradingAsCUDA guard(qa.device());
  Tensor out = at::empty({m, n}, qa.options().dtype(out_dtype));
  call(strix_w8a8_int8_gemm(static_cast<const int8_t*>(qa.data_ptr()), qa.stride(0),
                            sac.has_value() ? sac->data_ptr<float>() : nullptr, static_cast<const int8_t*>(w.data_ptr()),
                            w.stride(0), swc.has_value() ? swc->data_ptr<float>() : nullptr, out.data_ptr(), n,
                            out_code(out_dtype), m, n, k, (int)cfg, stream_of(qa)),
       "w8a8_scaled_mm");
  return out;
}

Tensor w8a8_scaled_mm(const Tensor& qa, const Tensor& sa, const Tensor& w, const Tensor& sw) {
  return i8_gemm(qa, sa, w, sw, at::kBFloat16, -1);
}

Tensor w8a8_scaled_mm_cfg(const Tensor& qa, const Tensor& sa, const Tensor& w, const Tensor& sw, int64_t cfg) {
  return i8_gemm(qa, sa, w, sw, at::kBFloat16, cfg);
}

void check_fp8_scales(const Tensor& sa, const Tensor& sw, int64_t m, int64_t n, int64_t k) {
  TORCH_CHECK(sa.scalar_type() == at::kFloat && sa.dim() == 2 && sa.size(0) == m && sa.size(1) == k / 128 &&
                  sa.stride(1) == 1,
              "sa must be float32 [M, K/128]");
  TORCH_CHECK(sw.scalar_type() == at::kFloat && sw.dim() == 2 && sw.size(0) == (n + 127) / 128 &&
                  sw.size(1) == k / 128 && sw.stride(1) == 1,
              "sw must be float32 [ceil(N/128), K/128]");
}

Tensor fp8_block(const Tensor& qa, const Tensor& sa, const Tensor& w, const Tensor& sw, int64_t cfg) {
  rowmajor(qa, "qa");
  rowmajor(w, "w");
  TORCH_CHECK(qa.scalar_type() == at::kFloat8_e4m3fn && w.scalar_type() == at::kFloat8_e4m3fn,
              "qa and w must be float8_e4m3fn");
  const int64_t m = qa.size(0), k = qa.size(1), n = w.size(0);
  TORCH_CHECK(w.size(1) == k, "Activation K (", k, ") must match weight K (", w.size(1), ")");
  TORCH_CHECK(k % 128 == 0, "K must be a multiple of 128, got K=", k);
  check_fp8_scales(sa, sw, m, n, k);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(qa.device());
  Tensor out = at::empty({m, n}, qa.options().dtype(at::kBFloat16));
  call(strix_fp8_w8a8_block_gemm(static_cast<const uint8_t*>(qa.data_ptr()), qa.stride(0), sa.data_ptr<float>(),
                                 sa.stride(0), static_cast<const uint8_t*>(w.data_ptr()), w.stride(0),
                                 sw.data_ptr<float>(), sw.stride(0), out.data_ptr(), n, STRIX_BF16, m, n, k, (int)cfg,
                                 stream_of(qa)),
       "fp8_w8a8_block_gemm");
  return out;
}

Tensor fp8_w8a8_block_gemm(const Tensor& qa, const Tensor& sa, const Tensor& w, const Tensor& sw) {
  return fp8_block(qa, sa, w, sw, -1);
}

Tensor fp8_w8a8_block_gemm_cfg(const Tensor& qa, const Tensor& sa, const Tensor& w, const Tensor& sw, int64_t cfg) {
  return fp8_block(qa, sa, w, sw, cfg);
}

Tensor weight8_kmajor(const Tensor& w) {
  const auto dt = w.scalar_type();
  TORCH_CHECK((dt == at::kFloat8_e4m3fn || dt == at::kChar || dt == at::kByte) && (w.dim() == 2 || w.dim() == 3) &&
                  w.stride(-1) == 1,
              "w must be 8-bit [N, K] or [E, N, K]");
  const int64_t k = w.size(-1);
  TORCH_CHECK(k % 128 == 0, "K must be a multiple of 128, got K=", k);
  const int64_t e = w.dim() == 2 ? 1 : w.size(0), n = w.dim() == 2 ? w.size(0) : w.size(1);
  TORCH_CHECK(w.dim() == 2 || w.stride(0) == n * w.stride(1), "expert slices must follow each other");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(w.device());
  Tensor out = w.dim() == 2 ? at::empty({k / 128, n, 128}, w.options()) : at::empty({e, k / 128, n, 128}, w.options());
  call(strix_weight8_kmajor(static_cast<const uint8_t*>(w.data_ptr()), w.stride(-2), e, n, k,
                            static_cast<uint8_t*>(out.data_ptr()), stream_of(w)),
       "weight8_kmajor");
  return out;
}

Tensor fp8_w8a8_block_gemm_kmajor(const Tensor& qa, const Tensor& sa, const Tensor& wk, const Tensor& sw,
                                  int64_t cfg) {
  rowmajor(qa, "qa");
  TORCH_CHECK(qa.scalar_type() == at::kFloat8_e4m3fn && wk.scalar_type() == at::kFloat8_e4m3fn,
              "qa and w must be float8_e4m3fn");
  TORCH_CHECK(wk.dim() == 3 && wk.size(2) == 128 && wk.is_contiguous(), "w_kmajor must be contiguous [K/128, N, 128]");
  const int64_t m = qa.size(0), k = qa.size(1), n = wk.size(1);
  TORCH_CHECK(wk.size(0) * 128 == k, "Activation K (", k, ") must match weight K (", wk.size(0) * 128, ")");
  check_fp8_scales(sa, sw, m, n, k);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(qa.device());
  Tensor out = at::empty({m, n}, qa.options().dtype(at::kBFloat16));
  call(strix_fp8_w8a8_block_gemm_kmajor(static_cast<const uint8_t*>(qa.data_ptr()), qa.stride(0), sa.data_ptr<float>(),
                                        sa.stride(0), static_cast<const uint8_t*>(wk.data_ptr()), sw.data_ptr<float>(),
                                        sw.stride(0), out.data_ptr(), n, STRIX_BF16, m, n, k, (int)cfg, stream_of(qa)),
       "fp8_w8a8_block_gemm_kmajor");
  return out;
}

// ---------------------------------------------------------------- MoE plumbing
std::tuple<Tensor, Tensor> moe_route_topk(const Tensor& logits, int64_t top_k, bool renormalize) {
  rowmajor(logits, "logits");
  TORCH_CHECK(logits.scalar_type() == at::kFloat || logits.scalar_type() == at::kBFloat16,
              "logits must be float32 or bfloat16");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(logits.device());
  const int64_t t = logits.size(0), e = logits.size(1);
  Tensor ids = at::empty({t, top_k}, logits.options().dtype(at::kInt));
  Tensor w = at::empty({t, top_k}, logits.options().dtype(at::kFloat));
  call(strix_moe_route_topk(logits.data_ptr(), logits.scalar_type() == at::kFloat ? STRIX_F32 : STRIX_BF16,
                            logits.stride(0), t, e, top_k, renormalize ? 1 : 0, ids.data_ptr<int32_t>(),
                            w.data_ptr<float>(), top_k, stream_of(logits)),
       "moe_route_topk");
  return {ids, w};
}

std::tuple<Tensor, Tensor, Tensor> moe_align(const Tensor& topk_ids, int64_t num_experts, int64_t block_m) {
  TORCH_CHECK(topk_ids.scalar_type() == at::kInt && topk_ids.is_contiguous(), "topk_ids must be contiguous int32");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(topk_ids.device());
  const int64_t s = topk_ids.numel();
  const auto [cap, nblk] = align_capacity(s, num_experts, block_m);
  const auto opt = topk_ids.options();
  Tensor sorted_ids = at::empty({cap}, opt), expert_ids = at::empty({nblk}, opt), num_post = at::empty({1}, opt);
  const int64_t wsb = strix_moe_align_workspace_bytes(s, num_experts);
  Tensor ws = at::empty({wsb}, opt.dtype(at::kByte));
  call(strix_moe_align(topk_ids.data_ptr<int32_t>(), s, num_experts, block_m, sorted_ids.data_ptr<int32_t>(), cap,
                       expert_ids.data_ptr<int32_t>(), nblk, num_post.data_ptr<int32_t>(), ws.data_ptr(), wsb,
                       stream_of(topk_ids)),
       "moe_align");
  return {sorted_ids, expert_ids, num_post};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> moe_align_quant(const Tensor& topk_ids, const Tensor& x,
                                                                   int64_t num_experts, int64_t block_m) {
  TORCH_CHECK(topk_ids.scalar_type() == at::kInt && topk_ids.is_contiguous(), "topk_ids must be contiguous int32");
  rowmajor(x, "x");
  const int64_t t = x.size(0), k = x.size(1);
  TORCH_CHECK(topk_ids.dim() == 2 && topk_ids.size(0) == t, "topk_ids must be [T, top_k] with one row per token of x");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(topk_ids.device());
  const int64_t n = topk_ids.numel();
  const auto [cap, nblk] = align_capacity(n, num_experts, block_m);
  const auto opt = topk_ids.options();
  Tensor sorted_ids = at::empty({cap}, opt), expert_ids = at::empty({nblk}, opt), num_post = at::empty({1}, opt);
  Tensor q = at::empty({t, k}, x.options().dtype(at::kFloat8_e4m3fn));
  Tensor s = at::empty({t, k / 128}, x.options().dtype(at::kFloat));
  const int64_t wsb = strix_moe_align_workspace_bytes(n, num_experts);
  Tensor ws = at::empty({wsb}, opt.dtype(at::kByte));
  call(strix_moe_align_quant(topk_ids.data_ptr<int32_t>(), n, num_experts, block_m, sorted_ids.data_ptr<int32_t>(),
                             cap, expert_ids.data_ptr<int32_t>(), nblk, num_post.data_ptr<int32_t>(), ws.data_ptr(),
                             wsb, x.data_ptr(), act_code(x), x.stride(0), static_cast<uint8_t*>(q.data_ptr()), k,
                             s.data_ptr<float>(), std::max<int64_t>(k / 128, 1), t, k, stream_of(topk_ids)),
       "moe_align_quant");
  return {sorted_ids, expert_ids, num_post, q, s};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> moe_route_align(const Tensor& logits, int64_t top_k,
                                                                   int64_t block_m, bool renormalize) {
  rowmajor(logits, "logits");
  TORCH_CHECK(logits.scalar_type() == at::kFloat || logits.scalar_type() == at::kBFloat16,
              "logits must be float32 or bfloat16");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(logits.device());
  const int64_t t = logits.size(0), e = logits.size(1);
  const auto i32 = logits.options().dtype(at::kInt);
  Tensor ids = at::empty({t, top_k}, i32), w = at::empty({t, top_k}, logits.options().dtype(at::kFloat));
  const auto [cap, nblk] = align_capacity(t * top_k, e, block_m);
  Tensor sorted_ids = at::empty({cap}, i32), expert_ids = at::empty({nblk}, i32), num_post = at::empty({1}, i32);
  const int64_t wsb = strix_moe_align_workspace_bytes(t * top_k, e);
  Tensor ws = at::empty({wsb}, logits.options().dtype(at::kByte));
  call(strix_moe_route_align(logits.data_ptr(), logits.scalar_type() == at::kFloat ? STRIX_F32 : STRIX_BF16,
                             logits.stride(0), t, e, top_k, renormalize ? 1 : 0, ids.data_ptr<int32_t>(),
                             w.data_ptr<float>(), block_m, sorted_ids.data_ptr<int32_t>(), cap,
                             expert_ids.data_ptr<int32_t>(), nblk, num_post.data_ptr<int32_t>(), ws.data_ptr(), wsb,
                             stream_of(logits)),
       "moe_route_align");
  return {ids, w, sorted_ids, expert_ids, num_post};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> moe_route_align_quant(
    const Tensor& logits, const Tensor& x, int64_t top_k, int64_t block_m, bool renormalize) {
  rowmajor(logits, "logits");
  rowmajor(x, "x");
  TORCH_CHECK(logits.scalar_type() == at::kFloat || logits.scalar_type() == at::kBFloat16,
              "logits must be float32 or bfloat16");
  const int64_t t = logits.size(0), e = logits.size(1), k = x.size(1);
  TORCH_CHECK(x.size(0) == t, "x must have one row per token");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(logits.device());
  const auto i32 = logits.options().dtype(at::kInt);
  Tensor ids = at::empty({t, top_k}, i32), w = at::empty({t, top_k}, logits.options().dtype(at::kFloat));
  const auto [cap, nblk] = align_capacity(t * top_k, e, block_m);
  Tensor sorted_ids = at::empty({cap}, i32), expert_ids = at::empty({nblk}, i32), num_post = at::empty({1}, i32);
  Tensor q = at::empty({t, k}, x.options().dtype(at::kFloat8_e4m3fn));
  Tensor s = at::empty({t, k / 128}, x.options().dtype(at::kFloat));
  const int64_t wsb = strix_moe_align_workspace_bytes(t * top_k, e);
  Tensor ws = at::empty({wsb}, logits.options().dtype(at::kByte));
  call(strix_moe_route_align_quant(logits.data_ptr(), logits.scalar_type() == at::kFloat ? STRIX_F32 : STRIX_BF16,
                                   logits.stride(0), t, e, top_k, renormalize ? 1 : 0, ids.data_ptr<int32_t>(),
                                   w.data_ptr<float>(), block_m, sorted_ids.data_ptr<int32_t>(), cap,
                                   expert_ids.data_ptr<int32_t>(), nblk, num_post.data_ptr<int32_t>(), ws.data_ptr(),
                                   wsb, x.data_ptr(), act_code(x), x.stride(0), static_cast<uint8_t*>(q.data_ptr()),
                                   k, s.data_ptr<float>(), std::max<int64_t>(k / 128, 1), k, stream_of(logits)),
       "moe_route_align_quant");
  return {ids, w, sorted_ids, expert_ids, num_post, q, s};
}

void sum_impl(const Tensor& inp, const std::optional<Tensor>& weights, const Tensor& output) {
  TORCH_CHECK(inp.dim() == 3 && inp.is_contiguous(), "input must be contiguous [T, top_k, H]");
  const int64_t t = inp.size(0), k = inp.size(1), h = inp.size(2);
  TORCH_CHECK(output.dim() == 2 && output.size(0) == t && output.size(1) == h && output.stride(1) == 1 &&
                  output.scalar_type() == inp.scalar_type(),
              "output must be [T, H] with the input dtype");
  std::optional<Tensor> wc;
  if (weights.has_value()) {
    TORCH_CHECK(weights->scalar_type() == at::kFloat && weights->numel() == t * k, "weights must be float32 [T, top_k]");
    wc = weights->contiguous();
  }
  const at::hip::HIPGuardMasqueradingAsCUDA guard(inp.device());
  call(strix_moe_sum(inp.data_ptr(), act_code(inp), h, t, k, h,
                     wc.has_value() ? wc->data_ptr<float>() : nullptr, output.data_ptr(), output.stride(0),
                     stream_of(inp)),
       "moe_sum");
}

void moe_sum(const Tensor& inp, const Tensor& output) { sum_impl(inp, std::nullopt, output); }

void moe_weighted_sum(const Tensor& inp, const Tensor& weights, const Tensor& output) {
  sum_impl(inp, weights, output);
}

// ---------------------------------------------------------------- expert GEMMs
void moe_common(const Tensor& c, const Tensor& sorted_ids, const Tensor& expert_ids, const Tensor& num_post,
                const std::optional<Tensor>& topk_weights, int64_t block_m) {
  TORCH_CHECK(sorted_ids.scalar_type() == at::kInt && expert_ids.scalar_type() == at::kInt &&
                  num_post.scalar_type() == at::kInt,
              "sorted_ids, expert_ids and num_post_padded must be int32");
  TORCH_CHECK(sorted_ids.is_contiguous() && expert_ids.is_contiguous(), "routing tensors must be contiguous");
  TORCH_CHECK(expert_ids.numel() * block_m >= sorted_ids.numel(),
              "expert_ids.numel() * block_m must cover sorted_ids");
  if (topk_weights.has_value())
    TORCH_CHECK(topk_weights->scalar_type() == at::kFloat && topk_weights->is_contiguous() &&
                    topk_weights->numel() == c.size(0),
                "topk_weights must be float32 with one weight per slot");
}

void moe_gemm_fp8_w8a8(const Tensor& c, const Tensor& qa, const Tensor& sa, const Tensor& b, const Tensor& scales,
                       const Tensor& sorted_ids, const Tensor& expert_ids, const Tensor& num_post,
                       const std::optional<Tensor>& topk_weights, int64_t top_k, int64_t block_m, int64_t block_n,
                       bool silu_mul, const std::string& activation) {
  const bool kmajor = b.dim() == 4;
  int64_t e, n, k;
  if (kmajor) {
    TORCH_CHECK(b.scalar_type() == at::kFloat8_e4m3fn && b.size(3) == 128 && b.is_contiguous(),
                "K-block-major b must be contiguous float8_e4m3fn [E, K/128, N, 128]");
    e = b.size(0), n = b.size(2), k = b.size(1) * 128;
  } else {
    TORCH_CHECK(b.dim() == 3 && b.scalar_type() == at::kFloat8_e4m3fn && b.stride(2) == 1,
                "b must be float8_e4m3fn [E, N, K] or [E, K/128, N, 128]");
    e = b.size(0), n = b.size(1), k = b.size(2);
  }
  rowmajor(qa, "qa");
  TORCH_CHECK(qa.scalar_type() == at::kFloat8_e4m3fn && qa.size(1) == k, "qa must be float8_e4m3fn [rows, K]");
  TORCH_CHECK(sa.scalar_type() == at::kFloat && sa.dim() == 2 && sa.size(1) == k / 128 && sa.stride(1) == 1,
              "sa must be float32 [rows, K/128]");
  TORCH_CHECK(scales.scalar_type() == at::kFloat && scales.dim() == 3 && scales.size(0) == e &&
                  scales.size(1) == (n + 127) / 128 && scales.size(2) == k / 128 && unit_last(scales),
              "scales must be float32 [E, N/128, K/128]");
  TORCH_CHECK(c.dim() == 2 && c.stride(1) == 1 && (c.scalar_type() == at::kBFloat16 || c.scalar_type() == at::kHalf),
              "c must be bf16/fp16 2-D");
  TORCH_CHECK(n % block_n == 0, "N=", n, " is not a multiple of block_n=", block_n);
  moe_common(c, sorted_ids, expert_ids, num_post, topk_weights, block_m);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(c.device());
  const float* tw = topk_weights.has_value() ? topk_weights->data_ptr<float>() : nullptr;
  const int act = activation_code(activation);
  if (kmajor) {
    call(strix_moe_gemm_fp8_w8a8_kmajor(
             c.data_ptr(), c.stride(0), out_code(c.scalar_type()), static_cast<const uint8_t*>(qa.data_ptr()),
             qa.stride(0), sa.data_ptr<float>(), sa.stride(0), static_cast<const uint8_t*>(b.data_ptr()),
             scales.data_ptr<float>(), scales.stride(0), scales.stride(1), sorted_ids.data_ptr<int32_t>(),
             sorted_ids.numel(), expert_ids.data_ptr<int32_t>(), expert_ids.numel(), num_post.data_ptr<int32_t>(), tw,
             c.size(0), top_k, block_m, silu_mul ? 1 : 0, act, n, k, stream_of(c)),
         "moe_gemm_fp8_w8a8");
    return;
  }
  call(strix_moe_gemm_fp8_w8a8(c.data_ptr(), c.stride(0), out_code(c.scalar_type()),
                               static_cast<const uint8_t*>(qa.data_ptr()), qa.stride(0), sa.data_ptr<float>(),
                               sa.stride(0), static_cast<const uint8_t*>(b.data_ptr()), b.stride(0), b.stride(1),
                               scales.data_ptr<float>(), scales.stride(0), scales.stride(1),
                               sorted_ids.data_ptr<int32_t>(), sorted_ids.numel(), expert_ids.data_ptr<int32_t>(),
                               expert_ids.numel(), num_post.data_ptr<int32_t>(), tw, c.size(0), top_k, block_m,
                               silu_mul ? 1 : 0, act, n, k, stream_of(c)),
       "moe_gemm_fp8_w8a8");
}

// Shared tail of the 16-bit expert GEMMs (STRIX_MOE16_PARAMS).
struct Moe16 {
  void* c; int64_t ldc; int c_dtype; const void* a; int64_t lda; int a_dtype;
  const int32_t* sorted_ids; int64_t sorted_len; const int32_t* expert_ids; int64_t num_blocks;
  const int32_t* num_post; const float* topk_w; int64_t num_slots; int64_t top_k; int64_t block_m;
  int silu_mul; int activation; int64_t N; int64_t K; void* stream;
};

Moe16 moe16_tail(const Tensor& c, const Tensor& a, const Tensor& sorted_ids, const Tensor& expert_ids,
                 const Tensor& num_post, const std::optional<Tensor>& topk_weights, int64_t top_k, int64_t block_m,
                 bool silu_mul, const std::string& activation, int64_t n, int64_t k) {
  TORCH_CHECK(c.dim() == 2 && c.stride(1) == 1 && (c.scalar_type() == at::kBFloat16 || c.scalar_type() == at::kHalf),
              "c must be bf16/fp16 2-D");
  TORCH_CHECK(a.dim() == 2 && a.stride(1) == 1 && a.size(1) == k, "a must be [rows, K=", k,
              "] and contiguous in dim 1");
  moe_common(c, sorted_ids, expert_ids, num_post, topk_weights, block_m);
  return Moe16{c.data_ptr(), c.stride(0), out_code(c.scalar_type()), a.data_ptr(), a.stride(0), act_code(a),
               sorted_ids.data_ptr<int32_t>(), sorted_ids.numel(), expert_ids.data_ptr<int32_t>(),
               expert_ids.numel(), num_post.data_ptr<int32_t>(),
               topk_weights.has_value() ? topk_weights->data_ptr<float>() : nullptr, c.size(0), top_k, block_m,
               silu_mul ? 1 : 0, activation_code(activation), n, k, stream_of(c)};
}

#define MOE16_ARGS(t)                                                                                               \
  t.c, t.ldc, t.c_dtype, t.a, t.lda, t.a_dtype, t.sorted_ids, t.sorted_len, t.expert_ids, t.num_blocks,          \
      t.num_post, t.topk_w, t.num_slots, t.top_k, t.block_m, t.silu_mul, t.activation, t.N, t.K, t.stream

void expert_stack(const Tensor& b, const char* what) {
  TORCH_CHECK(b.dim() == 3 && b.stride(2) == 1, what, " must be [E, N, K'] and contiguous in the last dim");
}

void moe_gemm_mxfp4(const Tensor& c, const Tensor& a, const Tensor& b, const Tensor& scales, const Tensor& sorted_ids,
                    const Tensor& expert_ids, const Tensor& num_post, const std::optional<Tensor>& topk_weights,
                    int64_t top_k, int64_t block_m, int64_t block_n, bool silu_mul, const std::string& activation) {
  expert_stack(b, "b");
  TORCH_CHECK(b.scalar_type() == at::kByte, "b must be uint8 packed e2m1 [E, N, K/2]");
  TORCH_CHECK(scales.scalar_type() == at::kByte, "scale must be uint8 (e8m0)");
  const int64_t e = b.size(0), n = b.size(1), k = 2 * b.size(2);
  TORCH_CHECK(scales.dim() == 3 && scales.size(0) == e && scales.size(1) == n && scales.size(2) == k / 32 &&
                  unit_last(scales),
              "scales must be e8m0 [E, N, K/32]");
  const Moe16 t = moe16_tail(c, a, sorted_ids, expert_ids, num_post, topk_weights, top_k, block_m, silu_mul,
                             activation, n, k);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(c.device());
  call(strix_moe_gemm_mxfp4(static_cast<const uint8_t*>(b.data_ptr()), b.stride(0), b.stride(1),
                            static_cast<const uint8_t*>(scales.data_ptr()), scales.stride(0), scales.stride(1),
                            MOE16_ARGS(t)),
       "moe_gemm_mxfp4");
}

void moe_gemm_w4a16_zp(const Tensor& c, const Tensor& a, const Tensor& b, const Tensor& scales, const Tensor& zeros,
                       const Tensor& sorted_ids, const Tensor& expert_ids, const Tensor& num_post,
                       const std::optional<Tensor>& topk_weights, int64_t top_k, int64_t block_m, int64_t block_n,
                       bool silu_mul, const std::string& activation, int64_t group_size) {
  expert_stack(b, "b");
  TORCH_CHECK(b.scalar_type() == at::kInt || b.scalar_type() == at::kByte,
              "b must be int32 [E, N, K/8] or uint8 [E, N, K/2] packed int4");
  const Tensor bu = b.scalar_type() == at::kInt ? b.view(at::kByte) : b;
  const int64_t e = bu.size(0), n = bu.size(1), k = 2 * bu.size(2);
  TORCH_CHECK(group_size > 0, "group_size must be positive");
  TORCH_CHECK((scales.scalar_type() == at::kBFloat16 || scales.scalar_type() == at::kHalf) && scales.dim() == 3 &&
                  scales.size(0) == e && scales.size(1) == n && scales.size(2) == k / group_size && unit_last(scales),
              "scales must be bf16/fp16 [E, N, K/group_size]");
  TORCH_CHECK(zeros.scalar_type() == at::kByte && zeros.dim() == 3 && zeros.size(0) == e && zeros.size(1) == n / 2 &&
                  zeros.size(2) == k / group_size && unit_last(zeros),
              "zeros must be uint8 [E, N/2, K/group_size] (two uint4 zero points per byte along N)");
  const Moe16 t = moe16_tail(c, a, sorted_ids, expert_ids, num_post, topk_weights, top_k, block_m, silu_mul,
                             activation, n, k);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(c.device());
  call(strix_moe_gemm_w4a16_zp(static_cast<const uint8_t*>(bu.data_ptr()), bu.stride(0), bu.stride(1),
                               scales.data_ptr(), scales.scalar_type() == at::kBFloat16 ? 1 : 2, scales.stride(0),
                               scales.stride(1), static_cast<const uint8_t*>(zeros.data_ptr()), zeros.stride(0),
                               zeros.stride(1), group_size, MOE16_ARGS(t)),
       "moe_gemm_w4a16_zp");
}

}  // namespace

// Schemas: the strings of libstrix_amd/torch_ops.py (the Python layer defines
// every op this library does not).
TORCH_LIBRARY_FRAGMENT(strix, m) {
  m.def("int8_quant_per_token(Tensor x) -> (Tensor, Tensor)");
  m.def("fp8_quant_group128(Tensor x) -> (Tensor, Tensor)");
  m.def("w8a8_scaled_mm(Tensor qa, Tensor sa, Tensor w, Tensor sw) -> Tensor");
  m.def("w8a8_scaled_mm_cfg(Tensor qa, Tensor sa, Tensor w, Tensor sw, int cfg) -> Tensor");
  m.def("fp8_w8a8_block_gemm(Tensor qa, Tensor sa, Tensor w, Tensor sw) -> Tensor");
  m.def("fp8_w8a8_block_gemm_cfg(Tensor qa, Tensor sa, Tensor w, Tensor sw, int cfg) -> Tensor");
  m.def("weight8_kmajor(Tensor w) -> Tensor");
  m.def("fp8_w8a8_block_gemm_kmajor(Tensor qa, Tensor sa, Tensor w_kmajor, Tensor sw, int cfg=-1) -> Tensor");
  m.def("moe_route_topk(Tensor logits, int top_k, bool renormalize=True) -> (Tensor, Tensor)");
  m.def("moe_align(Tensor topk_ids, int num_experts, int block_m) -> (Tensor, Tensor, Tensor)");
  m.def("moe_align_quant(Tensor topk_ids, Tensor x, int num_experts, int block_m) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("moe_route_align(Tensor logits, int top_k, int block_m, bool renormalize=True) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("moe_route_align_quant(Tensor logits, Tensor x, int top_k, int block_m, bool renormalize=True) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("moe_sum(Tensor input, Tensor(a!) output) -> ()");
  m.def("moe_weighted_sum(Tensor input, Tensor weights, Tensor(a!) output) -> ()");
  m.def("moe_gemm_fp8_w8a8(Tensor(a!) c, Tensor qa, Tensor sa, Tensor b, Tensor scales, "
        "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, Tensor? topk_weights, "
        "int top_k, int block_m, int block_n, bool silu_mul=False, str activation='silu') -> ()");
  m.def("moe_gemm_mxfp4(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, Tensor sorted_ids, Tensor expert_ids, "
        "Tensor num_post_padded, Tensor? topk_weights, int top_k, int block_m, int block_n, bool silu_mul=False, "
        "str activation='silu') -> ()");
  m.def("moe_gemm_w4a16_zp(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, Tensor zeros, Tensor sorted_ids, "
        "Tensor expert_ids, Tensor num_post_padded, Tensor? topk_weights, int top_k, int block_m, int block_n, "
        "bool silu_mul=False, str activation='silu', int group_size=128) -> ()");
}

TORCH_LIBRARY_IMPL(strix, CUDA, m) {
  m.impl("int8_quant_per_token", &int8_quant_per_token);
  m.impl("fp8_quant_group128", &fp8_quant_group128);
  m.impl("w8a8_scaled_mm", &w8a8_scaled_mm);
  m.impl("w8a8_scaled_mm_cfg", &w8a8_scaled_mm_cfg);
  m.impl("fp8_w8a8_block_gemm", &fp8_w8a8_block_gemm);
  m.impl("fp8_w8a8_block_gemm_cfg", &fp8_w8a8_block_gemm_cfg);
  m.impl("weight8_kmajor", &weight8_kmajor);
  m.impl("fp8_w8a8_block_gemm_kmajor", &fp8_w8a8_block_gemm_kmajor);
  m.impl("moe_route_topk", &moe_route_topk);
  m.impl("moe_align", &moe_align);
  m.impl("moe_align_quant", &moe_align_quant);
  m.impl("moe_route_align", &moe_route_align);
  m.impl("moe_route_align_quant", &moe_route_align_quant);
  m.impl("moe_sum", &moe_sum);
  m.impl("moe_weighted_sum", &moe_weighted_sum);
  m.impl("moe_gemm_fp8_w8a8", &moe_gemm_fp8_w8a8);
  m.impl("moe_gemm_mxfp4", &moe_gemm_mxfp4);
  m.impl("moe_gemm_w4a16_zp", &moe_gemm_w4a16_zp);
}
