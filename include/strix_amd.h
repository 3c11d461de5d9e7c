/* SPDX-License-Identifier: MIT
 *
 * libstrix_amd: C ABI of the MI355X (gfx950) quantized-GEMM hot path.
 *
 * The reference exposes this path only as torch ops registered in
 * csrc/torch_ops.cpp (TORCH_LIBRARY(strix, m), lines 179-304). Each entry
 * point below is the torch-free launch layer under one of those ops: plain
 * device pointers, element strides, sizes and a hipStream_t passed as void*.
 * The Python package libstrix_amd binds them with ctypes and registers the
 * same torch.ops.strix.* schemas on top.
 *
 * Conventions
 *   - Every function returns STRIX_OK (0) or an error code; the message of the
 *     last error on the calling thread is strix_last_error(). Argument checks
 *     run before any HIP call, so they work on a machine without a GPU.
 *   - Launches are asynchronous on `stream`; nothing synchronizes the host.
 *   - Strides ("ld*") are in elements of the pointed-to type; byte tensors
 *     (int8 / e4m3 / packed int4) count bytes.
 *   - Activation dtype codes: STRIX_BF16, STRIX_F16 (16-bit storage).
 *   - Weights are never copied or converted per call.
 */
#ifndef STRIX_AMD_H
#define STRIX_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STRIX_ABI_VERSION 1

enum {
  STRIX_OK = 0,
  STRIX_ERR_INVALID = 1, /* bad argument: shape, dtype, stride, alignment */
  STRIX_ERR_DEVICE = 2,  /* no device / not gfx950 */
  STRIX_ERR_LAUNCH = 3   /* the HIP launch itself failed */
};

enum {
  STRIX_BF16 = 0,
  STRIX_F16 = 1,
  STRIX_F32 = 2,
  STRIX_I32 = 3
};

enum { STRIX_ACT_SILU = 0, STRIX_ACT_GELU_TANH = 1 };

const char* strix_last_error(void);
int strix_abi_version(void);

/* ------------------------------------------------------------------ quant
 * int8 per-token: s[m] = max|x[m,:]|/127 (1 if 0), q = clamp(rint(x/s),-127,127).
 * New for BASELINE config 1 (the reference quantizes per 128-group inside
 * w8a8_wmma_gemm, csrc/gemm/w8a8_wmma_gemm.hip:456-548). */
int strix_int8_quant_per_token(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                               float* s, int64_t M, int64_t K, void* stream);
/* int8 per (row, 128-group), s [M, lds]: moe_act_quant_i8
 * (csrc/torch_ops.cpp:217, csrc/moe/moe_gemm_w4a8.hip:282-316). */
int strix_int8_quant_group128(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                              float* s, int64_t lds, int64_t M, int64_t K, void* stream);
/* out[m,k] = q[m,k] * s[m, k/128] in bf16/fp16 (STRIX_BF16/F16): the int8
 * activations of moe_gemm_w4a8 and w4a8_wmma_gemm (csrc/torch_ops.cpp:214-217, 283),
 * handed to the 16-bit MFMA GEMMs over the int4 weights. */
int strix_int8_dequant_group128(const int8_t* q, int64_t ldq, const float* s, int64_t lds, void* out,
                                int out_dtype, int64_t ldo, int64_t M, int64_t K, void* stream);
/* e4m3fn per (row, 128-group): s = max|x|/448 (1 if 0), q = e4m3_rne(x/s).
 * Absent in the reference (its FP8 path is W8A16, python/strix_vllm/fp8.py:122-124);
 * the input quant step of vLLM's Fp8BlockScaledMMLinearKernel that strix disables. */
int strix_fp8_quant_group128(const void* x, int x_dtype, int64_t ldx, uint8_t* q, int64_t ldq,
                             float* s, int64_t lds, int64_t M, int64_t K, void* stream);

/* ------------------------------------------------------------------ 8-bit GEMMs
 * FP8-block W8A8: out[M,N] = sum_kb sa[m,kb] sw[n/128,kb] (qa[m,kb] . qw[n,kb]).
 * qa e4m3 [M, lda], sa fp32 [M, sa_ld], w e4m3 [N, ldw], sw fp32 [ceil(N/128), sw_ld].
 * cfg -1 picks the tile by shape; 0..12 pins one (tile sweeps, cf. fp8_wmma_gemm_cfg,
 * csrc/torch_ops.cpp:253). Replaces fp8_wmma_gemm's dense FP8 role
 * (csrc/gemm/fp8_wmma_gemm.hip:253-322) with native e4m3 MFMA. */
int strix_fp8_w8a8_block_gemm(const uint8_t* qa, int64_t lda, const float* sa, int64_t sa_ld,
                              const uint8_t* w, int64_t ldw, const float* sw, int64_t sw_ld,
                              void* out, int64_t ldo, int out_dtype, int64_t M, int64_t N,
                              int64_t K, int cfg, void* stream);
/* 8-bit weights [E][N][ldw] -> K-block-major [E][K/128][N][128] (one
 * contiguous run per 128-K block of all rows). No counterpart in the
 * reference, whose kernels read row-major weights: a one-time weight
 * preparation in the place of the plugin's weight processing, which
 * re-strides FP8 weights for the memory system's sake
 * (python/strix_vllm/fp8.py:147-160), for the *_kmajor GEMM below. */
int strix_weight8_kmajor(const uint8_t* w, int64_t ldw, int64_t E, int64_t N, int64_t K, uint8_t* out,
                         void* stream);
/* strix_fp8_w8a8_block_gemm on K-block-major weights (w_kmajor[kb][n][128]),
 * bit-identical output. The concurrently streamed weight blocks sit together
 * in memory, which DRAM serves faster at decode. */
int strix_fp8_w8a8_block_gemm_kmajor(const uint8_t* qa, int64_t lda, const float* sa, int64_t sa_ld,
                                     const uint8_t* w_kmajor, const float* sw, int64_t sw_ld, void* out,
                                     int64_t ldo, int out_dtype, int64_t M, int64_t N, int64_t K, int cfg,
                                     void* stream);
/* INT8 per-token W8A8: out = bf16((float(qa.qw) * sa[m]) * sw[n]); out_dtype
 * STRIX_I32 writes the raw int32 accumulator (the bit-exactness probe). The
 * per-token sibling of w8a8_wmma_gemm (csrc/gemm/w8a8_wmma_gemm.hip:799-918). */
int strix_w8a8_int8_gemm(const int8_t* qa, int64_t lda, const float* sa, const int8_t* w, int64_t ldw,
                         const float* sw, void* out, int64_t ldo, int out_dtype, int64_t M, int64_t N,
                         int64_t K, int cfg, void* stream);
/* INT8 per-128-group activations x int8 weights (signed, or uint8b128 when
 * w_excess128), group or per-channel weight scales sw[n*sw_ns + g*sw_gs]:
 * the GEMM of w8a8_wmma_gemm (csrc/torch_ops.cpp:277, csrc/gemm/w8a8_wmma_gemm.hip:151-443). */
int strix_w8a8_int8_group_gemm(const int8_t* qa, int64_t lda, const float* sa, int64_t sa_ld,
                               const uint8_t* w, int64_t ldw, int w_excess128, const float* sw,
                               int64_t sw_ns, int64_t sw_gs, void* out, int64_t ldo, int out_dtype,
                               int64_t M, int64_t N, int64_t K, int cfg, void* stream);
/* FP8-block W8A8 grouped expert GEMM over aligned sorted ids (the W8A8
 * sibling of moe_gemm_fp8, csrc/torch_ops.cpp:225-228,
 * csrc/moe/moe_gemm_w8a16.hip:444-579). Rows of qa are tokens (slot / top_k);
 * silu_mul fuses act(gate)*up ([gate; up] weight rows, c gets N/2 columns);
 * topk_weights (may be NULL) scales each output row. With sorted_len,
 * num_blocks or num_slots 0 the call returns STRIX_OK without launching
 * (nothing is routed, c is left as it is); the same holds for every MoE GEMM
 * below. */
int strix_moe_gemm_fp8_w8a8(void* c, int64_t ldc, int c_dtype, const uint8_t* qa, int64_t lda,
                            const float* sa, int64_t sa_ld, const uint8_t* w, int64_t w_es, int64_t ldw,
                            const float* sw, int64_t sw_es, int64_t sw_ns, const int32_t* sorted_ids,
                            int64_t sorted_len, const int32_t* expert_ids, int64_t num_blocks,
                            const int32_t* num_post, const float* topk_weights, int64_t num_slots,
                            int64_t top_k, int64_t block_m, int silu_mul, int activation, int64_t N,
                            int64_t K, void* stream);
/* strix_moe_gemm_fp8_w8a8 on K-block-major expert weights
 * w_kmajor[E][K/128][N][128] (strix_weight8_kmajor with E experts),
 * bit-identical output. */
int strix_moe_gemm_fp8_w8a8_kmajor(void* c, int64_t ldc, int c_dtype, const uint8_t* qa, int64_t lda,
                                   const float* sa, int64_t sa_ld, const uint8_t* w_kmajor, const float* sw,
                                   int64_t sw_es, int64_t sw_ns, const int32_t* sorted_ids, int64_t sorted_len,
                                   const int32_t* expert_ids, int64_t num_blocks, const int32_t* num_post,
                                   const float* topk_weights, int64_t num_slots, int64_t top_k, int64_t block_m,
                                   int silu_mul, int activation, int64_t N, int64_t K, void* stream);

/* ------------------------------------------------------------------ 16-bit MFMA GEMMs over dequantized weights
 * Common MoE arguments (STRIX_MOE16_ARGS in gemm16.hip): c [num_slots, ldc]
 * (N/2 columns when silu_mul), activations a [rows, lda] (bf16 or fp16; a
 * row is slot / top_k), routing tensors as for strix_moe_gemm_fp8_w8a8,
 * N = weight rows per expert, K. Scale dtype codes: 0 f32, 1 bf16, 2 f16, 3 e8m0.
 * Weight strides (w_es, ldw) are in bytes. */
#define STRIX_MOE16_PARAMS                                                                                         \
  void *c, int64_t ldc, int c_dtype, const void *a, int64_t lda, int a_dtype, const int32_t *sorted_ids,          \
      int64_t sorted_len, const int32_t *expert_ids, int64_t num_blocks, const int32_t *num_post,                 \
      const float *topk_weights, int64_t num_slots, int64_t top_k, int64_t block_m, int silu_mul, int activation, \
      int64_t N, int64_t K, void *stream
/* MXFP4 experts: e2m1 [E, N, K/2] + e8m0 [E, N, K/32]; decoded to bf16 in LDS,
 * bf16 MFMA. Absent in the reference (its MXFP4 path is dense only,
 * csrc/gemm/mxfp4_wmma_gemm.hip:45-390); config 4. */
int strix_moe_gemm_mxfp4(const uint8_t* w, int64_t w_es, int64_t ldw, const uint8_t* scales, int64_t s_es,
                         int64_t s_ns, STRIX_MOE16_PARAMS);
/* WNA16 int4 experts with zero points: uint4 [E, N, K/2] (= int32 [E, N, K/8]),
 * scales [E, N, K/G], zeros uint8 [E, N/2, K/G]; value (q - z) s. The reference
 * rejects zero points (python/strix_vllm/moe.py:376); config 5. */
int strix_moe_gemm_w4a16_zp(const uint8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind,
                            int64_t s_es, int64_t s_ns, const uint8_t* zeros, int64_t z_es, int64_t z_ns,
                            int64_t group, STRIX_MOE16_PARAMS);
/* moe_gemm_w4a16 (csrc/torch_ops.cpp:191-195): symmetric (q - 8) s. */
int strix_moe_gemm_w4a16(const uint8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind, int64_t s_es,
                         int64_t s_ns, int64_t group, STRIX_MOE16_PARAMS);
/* moe_gemm_bf16 (csrc/torch_ops.cpp:185-189): bf16 experts; w_es and ldw in elements here. */
int strix_moe_gemm_bf16(const uint16_t* w, int64_t w_es, int64_t ldw, STRIX_MOE16_PARAMS);
/* moe_gemm_fp8 / moe_gemm_fp8_raw (csrc/torch_ops.cpp:225-232): e4m3 experts,
 * W8A16 (bf16 or fp16 activations), block [E, N/128, K/128] or channel [E, N] scales. */
int strix_moe_gemm_fp8_w8a16(const uint8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind,
                             int64_t s_es, int64_t s_ns, int64_t s_ks, int block_scales, STRIX_MOE16_PARAMS);
/* moe_gemm_w8a16 (csrc/torch_ops.cpp:221-224): int8 experts, per-channel scales. */
int strix_moe_gemm_w8a16(const int8_t* w, int64_t w_es, int64_t ldw, const void* scales, int s_kind, int64_t s_es,
                         int64_t s_ns, STRIX_MOE16_PARAMS);
/* mxfp4_wmma_gemm (csrc/torch_ops.cpp:283-286): dense MXFP4 W4A16 (+ bias, bias_rs 0 = [N]). */
int strix_mxfp4_gemm(const uint8_t* w, int64_t ldw, const uint8_t* scales, int64_t s_ld, const void* x, int x_dtype,
                     int64_t ldx, const void* bias, int64_t bias_rs, void* out, int64_t ldo, int out_dtype, int64_t M,
                     int64_t N, int64_t K, int cfg, void* stream);
/* fp8_wmma_gemm(_raw) (csrc/torch_ops.cpp:253-256): dense FP8 W8A16. */
int strix_fp8_w8a16_gemm(const uint8_t* w, int64_t ldw, const float* scales, int64_t s_ld, int block_scales,
                         const void* x, int x_dtype, int64_t ldx, void* out, int64_t ldo, int out_dtype, int64_t M,
                         int64_t N, int64_t K, int cfg, void* stream);
/* Dense weight-only GEMM over a packed weight format: out[m,n] = sum_k x[m,k]
 * decode(w[n,k]) (+ bias, bias_rs 0 = [N]). Scale of (n,k) at
 * scales[(n/nblock)*s_ns + (k/kgroup)*s_ks] (kgroup 0: one per row), s_kind
 * 0 f32, 1 bf16, 2 f16, 3 e8m0. fmt: 1 MXFP4, 3 INT4 (q-8) plain nibbles,
 * 4 e4m3, 5 int8, 6 uint4b8 in the RDNAHybridW4A16 word order (k 0 2 4 6 1 3
 * 5 7 per nibble), 7 uint8b128. Replaces the weight-only ops
 * fp8_skinny_gemm, w8a16_skinny_gemm (csrc/torch_ops.cpp:250-255;
 * csrc/gemm/w8a16_skinny_gemm.hip:525-775), w4a16_wmma_gemm
 * (csrc/torch_ops.cpp:266-268; csrc/gemm/w4a16_wmma_gemm.hip:1-245) and
 * mxfp4_gemv (csrc/torch_ops.cpp:293; csrc/gemm/mxfp4_gemv.hip:37-147). */
int strix_w16_gemm(int fmt, const uint8_t* w, int64_t ldw, const void* scales, int s_kind, int64_t s_ns,
                   int64_t s_ks, int64_t kgroup, int64_t nblock, const void* x, int x_dtype, int64_t ldx,
                   const void* bias, int64_t bias_rs, void* out, int64_t ldo, int out_dtype, int64_t M, int64_t N,
                   int64_t K, int cfg, void* stream);
/* Whole-matrix dequant to bf16 (mxfp4_dequant, fp8_dequant, w4a16_dequant,
 * csrc/torch_ops.cpp:252, 294-295): fmt as strix_w16_gemm (1, 3, 4, 5, 6, 7);
 * FP8 block scales use kgroup 128 + nblock 128, channel scales kgroup 0. */
int strix_dequant_bf16(int fmt, const uint8_t* w, int64_t ldw, const void* scales, int s_kind, int64_t s_ld,
                       int64_t kgroup, int64_t nblock, uint16_t* out, int64_t ldo, int64_t N, int64_t K, void* stream);

/* W4A8 on the int8 MFMA: int8 activations per (row, 128-group) x 4-bit weights
 * (value q - 8) widened to int8 in the tile, an exact int32 sum per 128-group
 * folded in fp32 with the activation and weight scales. w4a8_wmma_gemm
 * (csrc/torch_ops.cpp:283; csrc/gemm/w8a8_wmma_gemm.hip:128-135 is the
 * reference's W4 variant): weights [N, K/2] bytes, order 1 = nibble j of each
 * word is k j, 2 = RDNAHybridW4A16 words (k 0 2 4 6 1 3 5 7); fp32 weight
 * scales sw[n * sw_ns + g * sw_gs] per 128-group g (sw_gs 0: one per row). */
int strix_w4a8_gemm(const int8_t* qa, int64_t lda, const float* sa, int64_t sa_ld, const uint8_t* w4, int64_t ldw,
                    int order, const float* sw, int64_t sw_ns, int64_t sw_gs, void* out, int64_t ldo, int out_dtype,
                    int64_t M, int64_t N, int64_t K, void* stream);
/* moe_gemm_w4a8 (csrc/torch_ops.cpp:213-217; csrc/moe/moe_gemm_w4a8.hip:57-277):
 * int4 experts [E, N, K/2] (low nibble = even k) with fp32 scales [E, N, K/128],
 * int8 activations with fp32 scales [rows, K/128]; block_m 64, 128 or 256. */
int strix_moe_gemm_w4a8(void* c, int64_t ldc, int c_dtype, const int8_t* qa, int64_t lda, const float* sa,
                        int64_t sa_ld, const uint8_t* w4, int64_t w_es, int64_t ldw, const float* sw, int64_t sw_es,
                        int64_t sw_ns, const int32_t* sorted_ids, int64_t sorted_len, const int32_t* expert_ids,
                        int64_t num_blocks, const int32_t* num_post, const float* topk_weights, int64_t num_slots,
                        int64_t top_k, int64_t block_m, int silu_mul, int activation, int64_t N, int64_t K,
                        void* stream);

/* ------------------------------------------------------------------ MoE plumbing
 * Router: softmax -> top-k -> optional renormalize (vLLM fused_topk, called at
 * python/strix_vllm/moe.py:181-184). ids by logit value, ties to the lower id. */
int strix_moe_route_topk(const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E,
                         int64_t top_k, int renormalize, int32_t* topk_ids, float* topk_weights,
                         int64_t ldo, void* stream);
/* moe_align_block_size contract (tests/test_moe_gemm.py:9-31): slot ids
 * grouped by expert (ascending, stable), each run padded to block_m with id
 * num_slots; expert_ids per block (-1 past the end); num_post = padded total. */
int64_t strix_moe_align_sorted_capacity(int64_t num_slots, int64_t E, int64_t block_m);
int64_t strix_moe_align_workspace_bytes(int64_t num_slots, int64_t E);
int strix_moe_align(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                    int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                    int32_t* num_post, void* workspace, int64_t workspace_bytes, void* stream);
/* strix_moe_align plus the tokens' e4m3 1x128 quantization
 * (strix_fp8_quant_group128 of x [T, K] into q, s): the align and the
 * activation quant the reference's FP8 expert forward runs after vLLM's
 * router (python/strix_vllm/moe.py:286-288, 905-1014). Up to 1024 slots and
 * 64 tokens both run in the single-block align launch; otherwise in turn.
 * Same outputs, bit for bit. */
int strix_moe_align_quant(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                          int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                          int32_t* num_post, void* workspace, int64_t workspace_bytes, const void* x, int x_dtype,
                          int64_t ldx, uint8_t* q, int64_t ldq, float* s, int64_t lds, int64_t T, int64_t K,
                          void* stream);
/* strix_moe_align without a workspace argument and without any allocation:
 * no counterpart in the reference. For callers that cannot allocate (code
 * under HIP graph capture, serving loops that forbid hipMalloc). The
 * histogram lives in a 1 MiB device array of the library (one per GPU, held
 * until the process ends), so chunks * E <= 262144 with chunks =
 * ceil(num_slots / 256) (e.g. 524288 slots at E = 128); larger inputs are
 * rejected with an error. Calls that overlap on one GPU share the array and
 * race. Same outputs as strix_moe_align, bit for bit.
 * strix_moe_align_noalloc_max_bytes() returns the array's size. */
int64_t strix_moe_align_noalloc_max_bytes(void);
int strix_moe_align_noalloc(const int32_t* topk_ids, int64_t num_slots, int64_t E, int64_t block_m,
                            int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                            int32_t* num_post, void* stream);
/* Router and align in one call: the reference runs vLLM's fused_topk then
 * moe_align_block_size (python/strix_vllm/moe.py:181-184, 286-288). Same
 * outputs as strix_moe_route_topk (ldo = top_k) followed by strix_moe_align;
 * up to 16 tokens and 1024 slots (T * top_k) both run in one single-block
 * kernel launch.
 * Workspace: strix_moe_align_workspace_bytes(T * top_k, E). */
int strix_moe_route_align(const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E, int64_t top_k,
                          int renormalize, int32_t* topk_ids, float* topk_weights, int64_t block_m,
                          int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids, int64_t blocks_cap,
                          int32_t* num_post, void* workspace, int64_t workspace_bytes, void* stream);
/* strix_moe_route_align plus the tokens' e4m3 1x128 quantization
 * (strix_fp8_quant_group128 of x [T, K] into q, s), the steps the reference's
 * FP8 MoE forward runs first (python/strix_vllm/moe.py:181-184, 905-1014).
 * Up to 16 tokens the single-block kernel quantizes the rows with the waves
 * the router leaves idle, so the three steps are one launch; above, the
 * separate kernels run in turn. Same outputs, bit for bit. */
int strix_moe_route_align_quant(const void* logits, int logits_dtype, int64_t ldl, int64_t T, int64_t E,
                                int64_t top_k, int renormalize, int32_t* topk_ids, float* topk_weights,
                                int64_t block_m, int32_t* sorted_ids, int64_t sorted_cap, int32_t* expert_ids,
                                int64_t blocks_cap, int32_t* num_post, void* workspace, int64_t workspace_bytes,
                                const void* x, int x_dtype, int64_t ldx, uint8_t* q, int64_t ldq, float* s,
                                int64_t lds, int64_t K, void* stream);
/* moe_sum (python/strix_vllm/moe.py:328-330): out[t] = sum_j w[t,j] * y[t*k+j]
 * (w NULL = unweighted), fp32 in slot order. */
int strix_moe_sum(const void* y, int dtype, int64_t ldy, int64_t T, int64_t top_k, int64_t H,
                  const float* weights, void* out, int64_t ldo, void* stream);

/* ------------------------------------------------------------------ probes
 * Fragment-layout probes (the reference's _wmma_bf16_tile,
 * csrc/torch_ops.cpp:183, csrc/testing/wmma_layout_test.hip:12-36).
 * kind 0: bf16 a,b [16,K] -> fp32 d [16,16]; 1: e4m3 -> fp32; 2: int8 -> int32.
 * d = a . b^T through one wave's MFMA chain. */
int strix_probe_mfma(int kind, const void* a, const void* b, void* d, int64_t K, void* stream);
/* global_load_lds_dwordx4 placement: dst = src with its 64 16-byte chunks reversed. */
int strix_probe_g2l(const uint8_t* src, uint8_t* dst, void* stream);
/* Hardware converters: fp4_out [nscales][4 byte lanes][256 bytes][2] bf16 bits of
 * v_cvt_scalef32_pk_bf16_fp4; fp8_out [256] of v_cvt_pk_f32_fp8; bf16_out[i] =
 * v_cvt_pk_bf16_f32(bf16_in[i]). */
int strix_probe_cvt(const float* scales, int64_t nscales, uint16_t* fp4_out, float* fp8_out, uint16_t* bf16_out,
                    const float* bf16_in, int64_t nbf16, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRIX_AMD_H */
