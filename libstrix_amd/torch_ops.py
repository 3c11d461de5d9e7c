# SPDX-License-Identifier: MIT
"""torch.ops.strix.* on top of the C ABI.

The reference registers its ops from C++ (csrc/torch_ops.cpp:179-344). Here
the ops on the configurations' call chains (quantizers, W8A8 GEMMs, MoE
router / align / combine / expert GEMMs) are registered from C++ as well:
libstrix_amd/_strix_torch.so (torch_ext/strix_ops.cpp), loaded first, defines
their schemas and CUDA-key impls under a device guard, so a call does not go
through Python. The remaining ops (the reference's API-parity surface) are
defined here with torch.library, each CUDA-key implementation a thin call
into libstrix_amd/_strix_amd.so through ctypes. Every schema string is
recorded in SCHEMAS (the C++ ones too; a test compares them with the
registered schemas). Launches go on the current stream with no host
synchronization, so the ops are HIP-graph capturable. Reference schemas are
kept byte-identical; the ops this build adds are additive.

Every op raises RuntimeError on a bad argument (message from the library) and
when the library is not built; there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

from pathlib import Path

import torch

from libstrix_amd import _lib

TORCH_EXT = Path(__file__).with_name("_strix_torch.so")
# The C++ registration, when built: it must load (a broken build raises).
if TORCH_EXT.exists():
    _lib.load()  # the kernels library the extension links against, by the same path
    torch.ops.load_library(str(TORCH_EXT))

_LIB = torch.library.Library("strix", "FRAGMENT")
SCHEMAS: dict[str, str] = {}
NATIVE_OPS: set[str] = set()   # ops whose schema and impl come from the C++ registration
_ACT = {"silu": _lib.ACT_SILU, "gelu_tanh": _lib.ACT_GELU_TANH}


def _registered(name: str) -> bool:
    """Whether the C++ registration defines `name` with a CUDA-key impl."""
    try:
        return torch._C._dispatch_has_kernel_for_dispatch_key(f"strix::{name}", "CUDA")
    except RuntimeError:   # no such operator yet
        return False


def _define(schema: str):
    """Defines `schema` and registers the decorated function as its CUDA impl,
    unless the C++ registration already provides the op (then the Python
    function stays as the ctypes rendering of the same call, unused)."""
    name = schema.split("(", 1)[0]
    SCHEMAS[name] = schema
    native = _registered(name)
    if native:
        NATIVE_OPS.add(name)
    else:
        _LIB.define(schema)

    def deco(fn):
        if not native:
            _LIB.impl(name, fn, "CUDA")
        return fn

    return deco


def _fake(name: str):
    return torch.library.register_fake(f"strix::{name}")


# ----------------------------------------------------------------- helpers
def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _act_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype == torch.float16:
        return _lib.F16
    raise RuntimeError(f"Activation must be float16 or bfloat16, got {t.dtype}")


def _out_code(dtype: torch.dtype) -> int:
    return {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.int32: _lib.I32}[dtype]


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _unit_last(t: torch.Tensor) -> bool:
    """The last dim is unit-stride, or has one element (then its stride is never used)."""
    return t.size(-1) == 1 or t.stride(-1) == 1


def _rowmajor(t: torch.Tensor, what: str) -> None:
    _check(t.dim() == 2 and t.stride(1) == 1, f"{what} must be 2-D and contiguous in dim 1")


def _activation(name: str) -> int:
    _check(name in _ACT, f"activation must be 'silu' or 'gelu_tanh', got {name!r}")
    return _ACT[name]


# ----------------------------------------------------------------- quant
@_define("int8_quant_per_token(Tensor x) -> (Tensor, Tensor)")
def int8_quant_per_token(x):
    _rowmajor(x, "x")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    _lib.call("strix_int8_quant_per_token", _ptr(x), _act_code(x), x.stride(0), _ptr(q), k, _ptr(s), m, k,
              _stream(x))
    return q, s


@_fake("int8_quant_per_token")
def _(x):
    return x.new_empty(x.shape, dtype=torch.int8), x.new_empty((x.size(0),), dtype=torch.float32)


@_define("fp8_quant_group128(Tensor x) -> (Tensor, Tensor)")
def fp8_quant_group128(x):
    _rowmajor(x, "x")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((m, k // 128), dtype=torch.float32, device=x.device)
    _lib.call("strix_fp8_quant_group128", _ptr(x), _act_code(x), x.stride(0), _ptr(q), k, _ptr(s), max(k // 128, 1),
              m, k, _stream(x))
    return q, s


@_fake("fp8_quant_group128")
def _(x):
    return (x.new_empty(x.shape, dtype=torch.float8_e4m3fn),
            x.new_empty((x.size(0), x.size(1) // 128), dtype=torch.float32))


# Reference schema: csrc/torch_ops.cpp:217 (int8 per (row, 128-group)).
@_define("moe_act_quant_i8(Tensor x, Tensor(a!) q, Tensor(b!) sa) -> ()")
def moe_act_quant_i8(x, q, sa):
    _rowmajor(x, "x")
    m, k = x.shape
    _check(q.dtype == torch.int8 and tuple(q.shape) == (m, k) and q.stride(1) == 1, "q must be int8 [M, K]")
    _check(sa.dtype == torch.float32 and tuple(sa.shape) == (m, k // 128) and sa.stride(1) == 1,
           "sa must be float32 [M, K/128]")
    _lib.call("strix_int8_quant_group128", _ptr(x), _act_code(x), x.stride(0), _ptr(q), q.stride(0), _ptr(sa),
              sa.stride(0), m, k, _stream(x))


@_fake("moe_act_quant_i8")
def _(x, q, sa):
    return None


# ----------------------------------------------------------------- int8 W8A8
def _i8_gemm(qa, sa, w, sw, out_dtype, cfg):
    _rowmajor(qa, "qa")
    _rowmajor(w, "w")
    _check(qa.dtype == torch.int8 and w.dtype == torch.int8, "qa and w must be int8")
    m, k = qa.shape
    n = w.size(0)
    _check(w.size(1) == k, f"Activation K ({k}) must match weight K ({w.size(1)})")
    if out_dtype != torch.int32:
        _check(sa.dtype == torch.float32 and sa.numel() == m, "sa must be float32 [M]")
        _check(sw.dtype == torch.float32 and sw.numel() == n, "sw must be float32 [N]")
        sa, sw = sa.contiguous(), sw.contiguous()
    out = torch.empty((m, n), dtype=out_dtype, device=qa.device)
    _lib.call("strix_w8a8_int8_gemm", _ptr(qa), qa.stride(0), _ptr(sa), _ptr(w), w.stride(0), _ptr(sw), _ptr(out),
              n, _out_code(out_dtype), m, n, k, cfg, _stream(qa))
    return out


@_define("w8a8_scaled_mm(Tensor qa, Tensor sa, Tensor w, Tensor sw) -> Tensor")
def w8a8_scaled_mm(qa, sa, w, sw):
    return _i8_gemm(qa, sa, w, sw, torch.bfloat16, -1)


@_fake("w8a8_scaled_mm")
def _(qa, sa, w, sw):
    return qa.new_empty((qa.size(0), w.size(0)), dtype=torch.bfloat16)


@_define("w8a8_scaled_mm_cfg(Tensor qa, Tensor sa, Tensor w, Tensor sw, int cfg) -> Tensor")
def w8a8_scaled_mm_cfg(qa, sa, w, sw, cfg):
    return _i8_gemm(qa, sa, w, sw, torch.bfloat16, int(cfg))


@_fake("w8a8_scaled_mm_cfg")
def _(qa, sa, w, sw, cfg):
    return qa.new_empty((qa.size(0), w.size(0)), dtype=torch.bfloat16)


@_define("_w8a8_i32_acc(Tensor qa, Tensor w) -> Tensor")
def _w8a8_i32_acc(qa, w):
    return _i8_gemm(qa, None, w, None, torch.int32, -1)


@_fake("_w8a8_i32_acc")
def _(qa, w):
    return qa.new_empty((qa.size(0), w.size(0)), dtype=torch.int32)


# Reference schemas: csrc/torch_ops.cpp:277-282. uint8b128 weights [N, K]
# (rows may be padded), activations quantized per (row, 128-group) in the op,
# fp32 scales [G, N], [N, G] or [N].
def _w8a8_wmma(in_w8, in_act, in_scale, cfg):
    _check(in_w8.dim() == 2, f"Weights must be [N, K], got {in_w8.dim()} dims")
    _check(in_act.dim() == 2, f"Activation must be [M, K], got {in_act.dim()} dims")
    n, k = in_w8.shape
    m = in_act.size(0)
    _check(in_act.size(1) == k, f"Activation K ({in_act.size(1)}) must match weight K ({k})")
    _check(in_w8.dtype == torch.uint8, f"Weights must be uint8 (uint8b128 layout, one byte per element), got {in_w8.dtype}")
    _check(in_scale.dtype == torch.float32, f"Scale must be float32, got {in_scale.dtype}")
    _check(k % 128 == 0, f"K must be divisible by the weight group 128, got K={k}")
    _check(in_w8.stride(1) == 1, "Weights must be contiguous in dim 1")
    g = k // 128
    if in_scale.dim() == 1:
        _check(in_scale.numel() == n and in_scale.stride(0) == 1, f"Per-channel scale must be [N={n}] contiguous")
        ns, gs = 1, 0
    else:
        _check(in_scale.dim() == 2 and in_scale.stride(1) == 1, "Scale must be [G, N], [N, G] or [N]")
        if tuple(in_scale.shape) == (g, n):
            ns, gs = 1, in_scale.stride(0)
        else:
            _check(tuple(in_scale.shape) == (n, g),
                   f"Scale must be [G, N] = [{g}, {n}], [N, G] or [N={n}] but got {list(in_scale.shape)}")
            ns, gs = in_scale.stride(0), 1
    x = in_act.contiguous()
    out = torch.empty((m, n), dtype=in_act.dtype, device=in_act.device)
    if m == 0 or n == 0:
        return out
    q = torch.empty((m, k), dtype=torch.int8, device=in_act.device)
    sa = torch.empty((m, g), dtype=torch.float32, device=in_act.device)
    st = _stream(in_act)
    _lib.call("strix_int8_quant_group128", _ptr(x), _act_code(x), k, _ptr(q), k, _ptr(sa), g, m, k, st)
    _lib.call("strix_w8a8_int8_group_gemm", _ptr(q), k, _ptr(sa), g, _ptr(in_w8), in_w8.stride(0), 1, _ptr(in_scale),
              ns, gs, _ptr(out), n, _act_code(out), m, n, k, cfg, st)
    return out


@_define("w8a8_wmma_gemm(Tensor in_w8, Tensor in_act, Tensor in_scale) -> Tensor")
def w8a8_wmma_gemm(in_w8, in_act, in_scale):
    return _w8a8_wmma(in_w8, in_act, in_scale, -1)


@_fake("w8a8_wmma_gemm")
def _(in_w8, in_act, in_scale):
    return in_act.new_empty((in_act.size(0), in_w8.size(0)))


@_define("w8a8_wmma_gemm_cfg(Tensor in_w8, Tensor in_act, Tensor in_scale, int cfg) -> Tensor")
def w8a8_wmma_gemm_cfg(in_w8, in_act, in_scale, cfg):
    return _w8a8_wmma(in_w8, in_act, in_scale, int(cfg))


@_fake("w8a8_wmma_gemm_cfg")
def _(in_w8, in_act, in_scale, cfg):
    return in_act.new_empty((in_act.size(0), in_w8.size(0)))


# ----------------------------------------------------------------- FP8-block W8A8
def _fp8_block(qa, sa, w, sw, cfg):
    _rowmajor(qa, "qa")
    _rowmajor(w, "w")
    _check(qa.dtype == torch.float8_e4m3fn and w.dtype == torch.float8_e4m3fn, "qa and w must be float8_e4m3fn")
    m, k = qa.shape
    n = w.size(0)
    _check(w.size(1) == k, f"Activation K ({k}) must match weight K ({w.size(1)})")
    _check(k % 128 == 0, f"K must be a multiple of 128, got K={k}")
    _check(sa.dtype == torch.float32 and tuple(sa.shape) == (m, k // 128) and sa.stride(1) == 1,
           "sa must be float32 [M, K/128]")
    _check(sw.dtype == torch.float32 and tuple(sw.shape) == ((n + 127) // 128, k // 128) and sw.stride(1) == 1,
           "sw must be float32 [ceil(N/128), K/128]")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=qa.device)
    _lib.call("strix_fp8_w8a8_block_gemm", _ptr(qa), qa.stride(0), _ptr(sa), sa.stride(0), _ptr(w), w.stride(0),
              _ptr(sw), sw.stride(0), _ptr(out), n, _lib.BF16, m, n, k, cfg, _stream(qa))
    return out


@_define("fp8_w8a8_block_gemm(Tensor qa, Tensor sa, Tensor w, Tensor sw) -> Tensor")
def fp8_w8a8_block_gemm(qa, sa, w, sw):
    return _fp8_block(qa, sa, w, sw, -1)


@_fake("fp8_w8a8_block_gemm")
def _(qa, sa, w, sw):
    return qa.new_empty((qa.size(0), w.size(0)), dtype=torch.bfloat16)


@_define("fp8_w8a8_block_gemm_cfg(Tensor qa, Tensor sa, Tensor w, Tensor sw, int cfg) -> Tensor")
def fp8_w8a8_block_gemm_cfg(qa, sa, w, sw, cfg):
    return _fp8_block(qa, sa, w, sw, int(cfg))


@_fake("fp8_w8a8_block_gemm_cfg")
def _(qa, sa, w, sw, cfg):
    return qa.new_empty((qa.size(0), w.size(0)), dtype=torch.bfloat16)


_W8_DTYPES = (torch.float8_e4m3fn, torch.int8, torch.uint8)


@_define("weight8_kmajor(Tensor w) -> Tensor")
def weight8_kmajor(w):
    """8-bit weights [N, K] or [E, N, K] (rows contiguous) -> K-block-major
    [K/128, N, 128] or [E, K/128, N, 128], the layout the *_kmajor GEMMs read."""
    _check(w.dtype in _W8_DTYPES and w.dim() in (2, 3) and w.stride(-1) == 1, "w must be 8-bit [N, K] or [E, N, K]")
    k = w.size(-1)
    _check(k % 128 == 0, f"K must be a multiple of 128, got K={k}")
    e, n = (1, w.size(0)) if w.dim() == 2 else (w.size(0), w.size(1))
    _check(w.dim() == 2 or w.stride(0) == n * w.stride(1), "expert slices must follow each other")
    shape = (k // 128, n, 128) if w.dim() == 2 else (e, k // 128, n, 128)
    out = torch.empty(shape, dtype=w.dtype, device=w.device)
    _lib.call("strix_weight8_kmajor", _ptr(w), w.stride(-2), e, n, k, _ptr(out), _stream(w))
    return out


@_fake("weight8_kmajor")
def _(w):
    k = w.size(-1)
    shape = (k // 128, w.size(0), 128) if w.dim() == 2 else (w.size(0), k // 128, w.size(1), 128)
    return w.new_empty(shape)


@_define("fp8_w8a8_block_gemm_kmajor(Tensor qa, Tensor sa, Tensor w_kmajor, Tensor sw, int cfg=-1) -> Tensor")
def fp8_w8a8_block_gemm_kmajor(qa, sa, w_kmajor, sw, cfg=-1):
    """fp8_w8a8_block_gemm on weights already in K-block-major order
    (weight8_kmajor): the same result, bit for bit."""
    _rowmajor(qa, "qa")
    _check(qa.dtype == torch.float8_e4m3fn and w_kmajor.dtype == torch.float8_e4m3fn, "qa and w must be float8_e4m3fn")
    _check(w_kmajor.dim() == 3 and w_kmajor.size(2) == 128 and w_kmajor.is_contiguous(),
           "w_kmajor must be contiguous [K/128, N, 128]")
    m, k = qa.shape
    n = w_kmajor.size(1)
    _check(w_kmajor.size(0) * 128 == k, f"Activation K ({k}) must match weight K ({w_kmajor.size(0) * 128})")
    _check(sa.dtype == torch.float32 and tuple(sa.shape) == (m, k // 128) and sa.stride(1) == 1,
           "sa must be float32 [M, K/128]")
    _check(sw.dtype == torch.float32 and tuple(sw.shape) == ((n + 127) // 128, k // 128) and sw.stride(1) == 1,
           "sw must be float32 [ceil(N/128), K/128]")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=qa.device)
    _lib.call("strix_fp8_w8a8_block_gemm_kmajor", _ptr(qa), qa.stride(0), _ptr(sa), sa.stride(0), _ptr(w_kmajor),
              _ptr(sw), sw.stride(0), _ptr(out), n, _lib.BF16, m, n, k, int(cfg), _stream(qa))
    return out


@_fake("fp8_w8a8_block_gemm_kmajor")
def _(qa, sa, w_kmajor, sw, cfg=-1):
    return qa.new_empty((qa.size(0), w_kmajor.size(1)), dtype=torch.bfloat16)


# ----------------------------------------------------------------- MoE
def _moe_common(c, sorted_ids, expert_ids, num_post_padded, topk_weights, block_m):
    _check(sorted_ids.dtype == torch.int32 and expert_ids.dtype == torch.int32 and num_post_padded.dtype == torch.int32,
           "sorted_ids, expert_ids and num_post_padded must be int32")
    _check(sorted_ids.is_contiguous() and expert_ids.is_contiguous(), "routing tensors must be contiguous")
    _check(expert_ids.numel() * block_m >= sorted_ids.numel(),
           "expert_ids.numel() * block_m must cover sorted_ids")
    if topk_weights is not None:
        _check(topk_weights.dtype == torch.float32 and topk_weights.is_contiguous()
               and topk_weights.numel() == c.size(0), "topk_weights must be float32 with one weight per slot")


@_define(
    "moe_gemm_fp8_w8a8(Tensor(a!) c, Tensor qa, Tensor sa, Tensor b, Tensor scales, "
    "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, Tensor? topk_weights, "
    "int top_k, int block_m, int block_n, bool silu_mul=False, str activation='silu') -> ()"
)
def moe_gemm_fp8_w8a8(c, qa, sa, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m,
                      block_n, silu_mul=False, activation="silu"):
    # b: row-major [E, N, K], or K-block-major [E, K/128, N, 128] (weight8_kmajor).
    kmajor = b.dim() == 4
    if kmajor:
        _check(b.dtype == torch.float8_e4m3fn and b.size(3) == 128 and b.is_contiguous(),
               "K-block-major b must be contiguous float8_e4m3fn [E, K/128, N, 128]")
        e, n, k = b.size(0), b.size(2), b.size(1) * 128
    else:
        _check(b.dim() == 3 and b.dtype == torch.float8_e4m3fn and b.stride(2) == 1,
               "b must be float8_e4m3fn [E, N, K] or [E, K/128, N, 128]")
        e, n, k = b.shape
    _rowmajor(qa, "qa")
    _check(qa.dtype == torch.float8_e4m3fn and qa.size(1) == k, "qa must be float8_e4m3fn [rows, K]")
    _check(sa.dtype == torch.float32 and sa.dim() == 2 and sa.size(1) == k // 128 and sa.stride(1) == 1,
           "sa must be float32 [rows, K/128]")
    _check(scales.dtype == torch.float32 and tuple(scales.shape) == (e, (n + 127) // 128, k // 128)
           and _unit_last(scales), "scales must be float32 [E, N/128, K/128]")
    _check(c.dim() == 2 and c.stride(1) == 1 and c.dtype in (torch.bfloat16, torch.float16), "c must be bf16/fp16 2-D")
    _check(n % block_n == 0, f"N={n} is not a multiple of block_n={block_n}")
    _moe_common(c, sorted_ids, expert_ids, num_post_padded, topk_weights, block_m)
    if kmajor:
        _lib.call("strix_moe_gemm_fp8_w8a8_kmajor", _ptr(c), c.stride(0), _out_code(c.dtype), _ptr(qa), qa.stride(0),
                  _ptr(sa), sa.stride(0), _ptr(b), _ptr(scales), scales.stride(0), scales.stride(1),
                  _ptr(sorted_ids), sorted_ids.numel(), _ptr(expert_ids), expert_ids.numel(), _ptr(num_post_padded),
                  _ptr(topk_weights), c.size(0), top_k, block_m, int(bool(silu_mul)), _activation(activation), n, k,
                  _stream(c))
        return
    _lib.call("strix_moe_gemm_fp8_w8a8", _ptr(c), c.stride(0), _out_code(c.dtype), _ptr(qa), qa.stride(0), _ptr(sa),
              sa.stride(0), _ptr(b), b.stride(0), b.stride(1), _ptr(scales), scales.stride(0), scales.stride(1),
              _ptr(sorted_ids), sorted_ids.numel(), _ptr(expert_ids), expert_ids.numel(), _ptr(num_post_padded),
              _ptr(topk_weights), c.size(0), top_k, block_m, int(bool(silu_mul)), _activation(activation), n, k,
              _stream(c))


@_fake("moe_gemm_fp8_w8a8")
def _(c, qa, sa, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu"):
    return None


@_define("moe_route_topk(Tensor logits, int top_k, bool renormalize=True) -> (Tensor, Tensor)")
def moe_route_topk(logits, top_k, renormalize=True):
    _rowmajor(logits, "logits")
    _check(logits.dtype in (torch.float32, torch.bfloat16), "logits must be float32 or bfloat16")
    t, e = logits.shape
    ids = torch.empty((t, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((t, top_k), dtype=torch.float32, device=logits.device)
    code = _lib.F32 if logits.dtype == torch.float32 else _lib.BF16
    _lib.call("strix_moe_route_topk", _ptr(logits), code, logits.stride(0), t, e, top_k, int(bool(renormalize)),
              _ptr(ids), _ptr(w), top_k, _stream(logits))
    return ids, w


@_fake("moe_route_topk")
def _(logits, top_k, renormalize=True):
    t = logits.size(0)
    return (logits.new_empty((t, top_k), dtype=torch.int32), logits.new_empty((t, top_k), dtype=torch.float32))


def align_capacity(num_slots: int, num_experts: int, block_m: int) -> tuple[int, int]:
    cap = num_slots + num_experts * (block_m - 1)
    return cap, (cap + block_m - 1) // block_m


@_define("moe_align(Tensor topk_ids, int num_experts, int block_m) -> (Tensor, Tensor, Tensor)")
def moe_align(topk_ids, num_experts, block_m):
    _check(topk_ids.dtype == torch.int32 and topk_ids.is_contiguous(), "topk_ids must be contiguous int32")
    s = topk_ids.numel()
    cap, nblk = align_capacity(s, num_experts, block_m)
    dev = topk_ids.device
    sorted_ids = torch.empty((cap,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((nblk,), dtype=torch.int32, device=dev)
    num_post = torch.empty((1,), dtype=torch.int32, device=dev)
    ws_bytes = _lib.query("strix_moe_align_workspace_bytes", s, num_experts)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    _lib.call("strix_moe_align", _ptr(topk_ids), s, num_experts, block_m, _ptr(sorted_ids), cap, _ptr(expert_ids),
              nblk, _ptr(num_post), _ptr(ws), ws_bytes, _stream(topk_ids))
    return sorted_ids, expert_ids, num_post


@_fake("moe_align")
def _(topk_ids, num_experts, block_m):
    cap, nblk = align_capacity(topk_ids.numel(), num_experts, block_m)
    return (topk_ids.new_empty((cap,)), topk_ids.new_empty((nblk,)), topk_ids.new_empty((1,)))


@_define("moe_align_quant(Tensor topk_ids, Tensor x, int num_experts, int block_m) "
         "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
def moe_align_quant(topk_ids, x, num_experts, block_m):
    """moe_align(topk_ids) and fp8_quant_group128(x) in one call: (sorted_ids,
    expert_ids, num_post_padded, qx, sx), the same bits as the two ops; up to
    1024 slots and 64 tokens it is one kernel launch."""
    _check(topk_ids.dtype == torch.int32 and topk_ids.is_contiguous(), "topk_ids must be contiguous int32")
    _rowmajor(x, "x")
    t, k = x.shape
    _check(topk_ids.dim() == 2 and topk_ids.size(0) == t, "topk_ids must be [T, top_k] with one row per token of x")
    n = topk_ids.numel()
    cap, nblk = align_capacity(n, num_experts, block_m)
    dev = topk_ids.device
    sorted_ids = torch.empty((cap,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((nblk,), dtype=torch.int32, device=dev)
    num_post = torch.empty((1,), dtype=torch.int32, device=dev)
    q = torch.empty((t, k), dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty((t, k // 128), dtype=torch.float32, device=dev)
    ws_bytes = _lib.query("strix_moe_align_workspace_bytes", n, num_experts)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    _lib.call("strix_moe_align_quant", _ptr(topk_ids), n, num_experts, block_m, _ptr(sorted_ids), cap,
              _ptr(expert_ids), nblk, _ptr(num_post), _ptr(ws), ws_bytes, _ptr(x), _act_code(x), x.stride(0), _ptr(q),
              k, _ptr(s), max(k // 128, 1), t, k, _stream(topk_ids))
    return sorted_ids, expert_ids, num_post, q, s


@_fake("moe_align_quant")
def _(topk_ids, x, num_experts, block_m):
    cap, nblk = align_capacity(topk_ids.numel(), num_experts, block_m)
    return (topk_ids.new_empty((cap,)), topk_ids.new_empty((nblk,)), topk_ids.new_empty((1,)),
            x.new_empty(x.shape, dtype=torch.float8_e4m3fn), x.new_empty((x.size(0), x.size(1) // 128),
                                                                         dtype=torch.float32))


# Extension: the router and the align as one op (up to 16 tokens and 1024
# slots it runs as one single-block kernel); same outputs as moe_route_topk
# then moe_align.
@_define("moe_route_align(Tensor logits, int top_k, int block_m, bool renormalize=True) "
         "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
def moe_route_align(logits, top_k, block_m, renormalize=True):
    _rowmajor(logits, "logits")
    _check(logits.dtype in (torch.float32, torch.bfloat16), "logits must be float32 or bfloat16")
    t, e = logits.shape
    dev = logits.device
    ids = torch.empty((t, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((t, top_k), dtype=torch.float32, device=dev)
    cap, nblk = align_capacity(t * top_k, e, block_m)
    sorted_ids = torch.empty((cap,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((nblk,), dtype=torch.int32, device=dev)
    num_post = torch.empty((1,), dtype=torch.int32, device=dev)
    ws_bytes = _lib.query("strix_moe_align_workspace_bytes", t * top_k, e)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    code = _lib.F32 if logits.dtype == torch.float32 else _lib.BF16
    _lib.call("strix_moe_route_align", _ptr(logits), code, logits.stride(0), t, e, top_k, int(bool(renormalize)),
              _ptr(ids), _ptr(w), block_m, _ptr(sorted_ids), cap, _ptr(expert_ids), nblk, _ptr(num_post), _ptr(ws),
              ws_bytes, _stream(logits))
    return ids, w, sorted_ids, expert_ids, num_post


@_fake("moe_route_align")
def _(logits, top_k, block_m, renormalize=True):
    t, e = logits.shape
    cap, nblk = align_capacity(t * top_k, e, block_m)
    i32 = torch.int32
    return (logits.new_empty((t, top_k), dtype=i32), logits.new_empty((t, top_k), dtype=torch.float32),
            logits.new_empty((cap,), dtype=i32), logits.new_empty((nblk,), dtype=i32), logits.new_empty((1,), dtype=i32))


@_define(
    "moe_route_align_quant(Tensor logits, Tensor x, int top_k, int block_m, bool renormalize=True) -> "
    "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)"
)
def moe_route_align_quant(logits, x, top_k, block_m, renormalize=True):
    """moe_route_align and fp8_quant_group128(x) in one call: (topk_ids,
    topk_weights, sorted_ids, expert_ids, num_post_padded, qx, sx), the same
    bits as the two ops; up to 16 tokens it is one kernel launch."""
    _rowmajor(logits, "logits")
    _rowmajor(x, "x")
    _check(logits.dtype in (torch.float32, torch.bfloat16), "logits must be float32 or bfloat16")
    t, e = logits.shape
    _check(x.size(0) == t, "x must have one row per token")
    k = x.size(1)
    dev = logits.device
    ids = torch.empty((t, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((t, top_k), dtype=torch.float32, device=dev)
    cap, nblk = align_capacity(t * top_k, e, block_m)
    sorted_ids = torch.empty((cap,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((nblk,), dtype=torch.int32, device=dev)
    num_post = torch.empty((1,), dtype=torch.int32, device=dev)
    q = torch.empty((t, k), dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty((t, k // 128), dtype=torch.float32, device=dev)
    ws_bytes = _lib.query("strix_moe_align_workspace_bytes", t * top_k, e)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    code = _lib.F32 if logits.dtype == torch.float32 else _lib.BF16
    _lib.call("strix_moe_route_align_quant", _ptr(logits), code, logits.stride(0), t, e, top_k,
              int(bool(renormalize)), _ptr(ids), _ptr(w), block_m, _ptr(sorted_ids), cap, _ptr(expert_ids), nblk,
              _ptr(num_post), _ptr(ws), ws_bytes, _ptr(x), _act_code(x), x.stride(0), _ptr(q), k, _ptr(s),
              max(k // 128, 1), k, _stream(logits))
    return ids, w, sorted_ids, expert_ids, num_post, q, s


@_fake("moe_route_align_quant")
def _(logits, x, top_k, block_m, renormalize=True):
    t, e = logits.shape
    cap, nblk = align_capacity(t * top_k, e, block_m)
    i32 = torch.int32
    return (logits.new_empty((t, top_k), dtype=i32), logits.new_empty((t, top_k), dtype=torch.float32),
            logits.new_empty((cap,), dtype=i32), logits.new_empty((nblk,), dtype=i32), logits.new_empty((1,), dtype=i32),
            x.new_empty(x.shape, dtype=torch.float8_e4m3fn), x.new_empty((t, x.size(1) // 128), dtype=torch.float32))


def _sum_impl(inp, weights, output):
    _check(inp.dim() == 3 and inp.is_contiguous(), "input must be contiguous [T, top_k, H]")
    t, k, h = inp.shape
    _check(output.dim() == 2 and tuple(output.shape) == (t, h) and output.stride(1) == 1
           and output.dtype == inp.dtype, "output must be [T, H] with the input dtype")
    if weights is not None:
        _check(weights.dtype == torch.float32 and weights.numel() == t * k, "weights must be float32 [T, top_k]")
        weights = weights.contiguous()
    _lib.call("strix_moe_sum", _ptr(inp), _act_code(inp), h, t, k, h, _ptr(weights), _ptr(output), output.stride(0),
              _stream(inp))


# Same schema as vLLM's _moe_C::moe_sum (called at python/strix_vllm/moe.py:328-330).
@_define("moe_sum(Tensor input, Tensor(a!) output) -> ()")
def moe_sum(inp, output):
    _sum_impl(inp, None, output)


@_fake("moe_sum")
def _(inp, output):
    return None


@_define("moe_weighted_sum(Tensor input, Tensor weights, Tensor(a!) output) -> ()")
def moe_weighted_sum(inp, weights, output):
    _sum_impl(inp, weights, output)


@_fake("moe_weighted_sum")
def _(inp, weights, output):
    return None


# ----------------------------------------------------------------- probes
@_define("_mfma_tile(Tensor a, Tensor b) -> Tensor")
def _mfma_tile(a, b):
    _check(a.dim() == 2 and a.shape == b.shape and a.size(0) == 16 and a.dtype == b.dtype, "a, b must be [16, K]")
    a, b = a.contiguous(), b.contiguous()
    kind = {torch.bfloat16: 0, torch.float8_e4m3fn: 1, torch.int8: 2}.get(a.dtype)
    _check(kind is not None, "probe dtypes: bfloat16, float8_e4m3fn or int8")
    d = torch.empty((16, 16), dtype=torch.int32 if kind == 2 else torch.float32, device=a.device)
    _lib.call("strix_probe_mfma", kind, _ptr(a), _ptr(b), _ptr(d), a.size(1), _stream(a))
    return d


@_fake("_mfma_tile")
def _(a, b):
    return a.new_empty((16, 16), dtype=torch.int32 if a.dtype == torch.int8 else torch.float32)


@_define("_g2l_probe(Tensor src) -> Tensor")
def _g2l_probe(src):
    _check(src.dtype == torch.uint8 and src.numel() == 1024 and src.is_contiguous(), "src must be 1024 uint8")
    dst = torch.empty_like(src)
    _lib.call("strix_probe_g2l", _ptr(src), _ptr(dst), _stream(src))
    return dst


@_fake("_g2l_probe")
def _(src):
    return torch.empty_like(src)


# ----------------------------------------------------------------- 16-bit MFMA over dequantized weights
_SCALE_KIND = {torch.float32: _lib.S_F32, torch.bfloat16: _lib.S_BF16, torch.float16: _lib.S_F16}


def _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul, activation,
                n, k):
    _check(c.dim() == 2 and c.stride(1) == 1 and c.dtype in (torch.bfloat16, torch.float16), "c must be bf16/fp16 2-D")
    _check(a.dim() == 2 and a.stride(1) == 1 and a.size(1) == k, f"a must be [rows, K={k}] and contiguous in dim 1")
    _moe_common(c, sorted_ids, expert_ids, num_post_padded, topk_weights, block_m)
    return [_ptr(c), c.stride(0), _out_code(c.dtype), _ptr(a), a.stride(0), _act_code(a), _ptr(sorted_ids),
            sorted_ids.numel(), _ptr(expert_ids), expert_ids.numel(), _ptr(num_post_padded), _ptr(topk_weights),
            c.size(0), top_k, block_m, int(bool(silu_mul)), _activation(activation), n, k, _stream(c)]


def _expert_stack(b, what):
    _check(b.dim() == 3 and b.stride(2) == 1, f"{what} must be [E, N, K'] and contiguous in the last dim")


@_define(
    "moe_gemm_mxfp4(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, Tensor sorted_ids, Tensor expert_ids, "
    "Tensor num_post_padded, Tensor? topk_weights, int top_k, int block_m, int block_n, bool silu_mul=False, "
    "str activation='silu') -> ()"
)
def moe_gemm_mxfp4(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                   silu_mul=False, activation="silu"):
    _expert_stack(b, "b")
    _check(b.dtype == torch.uint8, "b must be uint8 packed e2m1 [E, N, K/2]")
    _check(scales.dtype == torch.uint8, "scale must be uint8 (e8m0)")
    e, n, k2 = b.shape
    k = 2 * k2
    _check(tuple(scales.shape) == (e, n, k // 32) and _unit_last(scales), "scales must be e8m0 [E, N, K/32]")
    tail = _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul,
                       activation, n, k)
    _lib.call("strix_moe_gemm_mxfp4", _ptr(b), b.stride(0), b.stride(1), _ptr(scales), scales.stride(0),
              scales.stride(1), *tail)


@_fake("moe_gemm_mxfp4")
def _(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu"):
    return None


def _int4_bytes(b):
    """int32 [E, N, K/8] or uint8 [E, N, K/2] packed int4 -> the uint8 view."""
    if b.dtype == torch.int32:
        return b.view(torch.uint8)
    _check(b.dtype == torch.uint8, "b must be int32 [E, N, K/8] or uint8 [E, N, K/2] packed int4")
    return b


@_define(
    "moe_gemm_w4a16_zp(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, Tensor zeros, Tensor sorted_ids, "
    "Tensor expert_ids, Tensor num_post_padded, Tensor? topk_weights, int top_k, int block_m, int block_n, "
    "bool silu_mul=False, str activation='silu', int group_size=128) -> ()"
)
def moe_gemm_w4a16_zp(c, a, b, scales, zeros, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m,
                      block_n, silu_mul=False, activation="silu", group_size=128):
    _expert_stack(b, "b")
    bu = _int4_bytes(b)
    e, n, k2 = bu.shape
    k = 2 * k2
    _check(scales.dtype in (torch.bfloat16, torch.float16) and tuple(scales.shape) == (e, n, k // group_size)
           and _unit_last(scales), "scales must be bf16/fp16 [E, N, K/group_size]")
    _check(zeros.dtype == torch.uint8 and tuple(zeros.shape) == (e, n // 2, k // group_size) and _unit_last(zeros),
           "zeros must be uint8 [E, N/2, K/group_size] (two uint4 zero points per byte along N)")
    tail = _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul,
                       activation, n, k)
    _lib.call("strix_moe_gemm_w4a16_zp", _ptr(bu), bu.stride(0), bu.stride(1), _ptr(scales), _SCALE_KIND[scales.dtype],
              scales.stride(0), scales.stride(1), _ptr(zeros), zeros.stride(0), zeros.stride(1), group_size, *tail)


@_fake("moe_gemm_w4a16_zp")
def _(c, a, b, scales, zeros, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu", group_size=128):
    return None


# Reference schema: csrc/torch_ops.cpp:191-195.
@_define(
    "moe_gemm_w4a16(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, "
    "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, "
    "Tensor? topk_weights, int top_k, int block_m, int block_n, "
    "bool silu_mul=False, str activation='silu', int group_size=32) -> ()"
)
def moe_gemm_w4a16(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                   silu_mul=False, activation="silu", group_size=32):
    _expert_stack(b, "b")
    bu = _int4_bytes(b)
    e, n, k2 = bu.shape
    k = 2 * k2
    _check(scales.dtype in (torch.bfloat16, torch.float16, torch.float32)
           and tuple(scales.shape) == (e, n, k // group_size) and _unit_last(scales),
           "scales must be [E, N, K/group_size]")
    _check(n % block_n == 0, f"N={n} is not a multiple of block_n={block_n}")
    tail = _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul,
                       activation, n, k)
    _lib.call("strix_moe_gemm_w4a16", _ptr(bu), bu.stride(0), bu.stride(1), _ptr(scales), _SCALE_KIND[scales.dtype],
              scales.stride(0), scales.stride(1), group_size, *tail)


@_fake("moe_gemm_w4a16")
def _(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu", group_size=32):
    return None


# Reference schema: csrc/torch_ops.cpp:185-189.
@_define(
    "moe_gemm_bf16(Tensor(a!) c, Tensor a, Tensor b, Tensor sorted_ids, "
    "Tensor expert_ids, Tensor num_post_padded, Tensor? topk_weights, "
    "int top_k, int block_m, int block_n, bool silu_mul=False, "
    "str activation='silu') -> ()"
)
def moe_gemm_bf16(c, a, b, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                  silu_mul=False, activation="silu"):
    _expert_stack(b, "b")
    _check(b.dtype == a.dtype == torch.bfloat16, "a and b must be bfloat16")
    e, n, k = b.shape
    _check(n % block_n == 0, f"N={n} is not a multiple of block_n={block_n}")
    tail = _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul,
                       activation, n, k)
    _lib.call("strix_moe_gemm_bf16", _ptr(b), b.stride(0), b.stride(1), *tail)


@_fake("moe_gemm_bf16")
def _(c, a, b, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n, silu_mul=False,
      activation="silu"):
    return None


def _channel_scales(scales, e, n):
    """[E, N] or [E, N, 1] per-channel scales -> (tensor, expert stride, row stride)."""
    _check(scales.dim() in (2, 3) and scales.size(0) == e and scales.size(1) == n
           and (scales.dim() == 2 or scales.size(2) == 1), f"scales must be [E, N] or [E, N, 1], E={e}, N={n}")
    _check(scales.dtype in _SCALE_KIND, "scales must be float32, bfloat16 or float16")
    return scales, scales.stride(0), scales.stride(1)


def _moe_fp8_w8a16(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                   silu_mul, activation):
    _expert_stack(b, "b")
    _check(b.dtype == torch.float8_e4m3fn, "b must be float8_e4m3fn [E, N, K]")
    e, n, k = b.shape
    _check(n % block_n == 0, f"N={n} is not a multiple of block_n={block_n}")
    block = scales.dim() == 3 and tuple(scales.shape) == (e, (n + 127) // 128, k // 128) and scales.size(2) != 1
    if block:
        _check(scales.dtype == torch.float32 and _unit_last(scales), "block scales must be float32 [E, N/128, K/128]")
        s_es, s_ns, s_ks = scales.stride(0), scales.stride(1), scales.stride(2)
    else:
        scales, s_es, s_ns = _channel_scales(scales, e, n)
        s_ks = 0
    tail = _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul,
                       activation, n, k)
    _lib.call("strix_moe_gemm_fp8_w8a16", _ptr(b), b.stride(0), b.stride(1), _ptr(scales), _SCALE_KIND[scales.dtype],
              s_es, s_ns, s_ks, int(block), *tail)


# Reference schemas: csrc/torch_ops.cpp:225-232 (W8A16: bf16 or fp16 "raw" activations).
@_define(
    "moe_gemm_fp8(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, "
    "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, "
    "Tensor? topk_weights, int top_k, int block_m, int block_n, "
    "bool silu_mul=False, str activation='silu') -> ()"
)
def moe_gemm_fp8(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                 silu_mul=False, activation="silu"):
    _check(a.dtype == torch.bfloat16, "a must be bfloat16 (moe_gemm_fp8_raw takes float16)")
    _moe_fp8_w8a16(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                   silu_mul, activation)


@_fake("moe_gemm_fp8")
def _(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu"):
    return None


@_define(
    "moe_gemm_fp8_raw(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, "
    "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, "
    "Tensor? topk_weights, int top_k, int block_m, int block_n, "
    "bool silu_mul=False, str activation='silu') -> ()"
)
def moe_gemm_fp8_raw(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                     silu_mul=False, activation="silu"):
    _check(a.dtype == torch.float16, "a must be float16")
    _moe_fp8_w8a16(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                   silu_mul, activation)


@_fake("moe_gemm_fp8_raw")
def _(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu"):
    return None


# Reference schema: csrc/torch_ops.cpp:221-224 (int8 experts, per-channel scales).
@_define(
    "moe_gemm_w8a16(Tensor(a!) c, Tensor a, Tensor b, Tensor scales, "
    "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, "
    "Tensor? topk_weights, int top_k, int block_m, int block_n, "
    "bool silu_mul=False, str activation='silu') -> ()"
)
def moe_gemm_w8a16(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
                   silu_mul=False, activation="silu"):
    _expert_stack(b, "b")
    _check(b.dtype == torch.int8, "b must be int8 [E, N, K]")
    e, n, k = b.shape
    _check(n % block_n == 0, f"N={n} is not a multiple of block_n={block_n}")
    scales, s_es, s_ns = _channel_scales(scales, e, n)
    tail = _moe16_tail(c, a, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, silu_mul,
                       activation, n, k)
    _lib.call("strix_moe_gemm_w8a16", _ptr(b), b.stride(0), b.stride(1), _ptr(scales), _SCALE_KIND[scales.dtype], s_es,
              s_ns, *tail)


@_fake("moe_gemm_w8a16")
def _(c, a, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu"):
    return None


# ----------------------------------------------------------------- dense MXFP4 / FP8 W8A16
def _mxfp4_dense(w, x, scales, bias, cfg):
    _check(w.dim() == 2 and x.dim() == 2, "w must be [N, K/2] and x [M, K]")
    n, k = w.size(0), x.size(1)
    _check(w.dtype == torch.uint8 and w.stride(1) == 1 and 2 * w.size(1) == k, "w must be uint8 [N, K/2]")
    _check(scales.dtype == torch.uint8, "scale must be uint8 (e8m0)")
    _check(k % 64 == 0, f"K must be a multiple of 64, got K={k}")
    _check(tuple(scales.shape) == (n, k // 32) and _unit_last(scales), "scales must be [N, K/32]")
    _check(x.dtype in (torch.bfloat16, torch.float16) and x.stride(1) == 1, "x must be bf16/fp16, contiguous in dim 1")
    m = x.size(0)
    out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    bias_rs = 0
    if bias is not None:
        _check(bias.dtype == x.dtype, "bias must have the activation dtype")
        if bias.dim() == 2:
            _check(tuple(bias.shape) == (m, n) and bias.stride(1) == 1, "bias must be [N] or [M, N]")
            bias_rs = bias.stride(0)
        else:
            _check(bias.numel() == n, "bias must be [N] or [M, N]")
            bias = bias.contiguous()
    _lib.call("strix_mxfp4_gemm", _ptr(w), w.stride(0), _ptr(scales), scales.stride(0), _ptr(x), _act_code(x),
              x.stride(0), _ptr(bias), bias_rs, _ptr(out), n, _act_code(out), m, n, k, cfg, _stream(x))
    return out


# Reference schemas: csrc/torch_ops.cpp:283-292.
@_define("mxfp4_wmma_gemm(Tensor w, Tensor x, Tensor scales, Tensor? bias) -> Tensor")
def mxfp4_wmma_gemm(w, x, scales, bias):
    return _mxfp4_dense(w, x, scales, bias, -1)


@_fake("mxfp4_wmma_gemm")
def _(w, x, scales, bias):
    return x.new_empty((x.size(0), w.size(0)))


@_define("mxfp4_wmma_gemm_cfg(Tensor w, Tensor x, Tensor scales, Tensor? bias, int cfg) -> Tensor")
def mxfp4_wmma_gemm_cfg(w, x, scales, bias, cfg):
    return _mxfp4_dense(w, x, scales, bias, int(cfg))


@_fake("mxfp4_wmma_gemm_cfg")
def _(w, x, scales, bias, cfg):
    return x.new_empty((x.size(0), w.size(0)))


@_define("mxfp4_dequant(Tensor w, Tensor scales) -> Tensor")
def mxfp4_dequant(w, scales):
    _check(w.dim() == 2 and w.dtype == torch.uint8 and w.stride(1) == 1, "w must be uint8 [N, K/2]")
    _check(scales.dtype == torch.uint8, "scale must be uint8 (e8m0)")
    n, k = w.size(0), 2 * w.size(1)
    _check(tuple(scales.shape) == (n, k // 32) and _unit_last(scales), "scales must be [N, K/32]")
    out = torch.empty((n, k), dtype=torch.bfloat16, device=w.device)
    _lib.call("strix_dequant_bf16", _lib.FMT_MXFP4, _ptr(w), w.stride(0), _ptr(scales), _lib.S_E8M0, scales.stride(0),
              32, 1, _ptr(out), k, n, k, _stream(w))
    return out


@_fake("mxfp4_dequant")
def _(w, scales):
    return w.new_empty((w.size(0), w.size(1) * 2), dtype=torch.bfloat16)


def _fp8_scales_dense(scales, n, k):
    """128x128 block scales [ceil(N/128), K/128] or per-channel [N] (fp32)."""
    _check(scales.dtype == torch.float32, f"scales must be float32, got {scales.dtype}")
    if scales.dim() == 2 and tuple(scales.shape) == ((n + 127) // 128, k // 128) and scales.stride(1) == 1:
        _check(k % 128 == 0, f"K must be a multiple of 128 with block scales, got K={k}")
        return True, scales.stride(0)
    _check(scales.numel() == n, f"scales must be [ceil(N/128), K/128] block or [N] channel scales, got "
           f"{list(scales.shape)}")
    return False, 1


def _fp8_w8a16(w, x, scales, raw, cfg):
    _check(w.dim() == 2 and x.dim() == 2, "w must be [N, K] and x [M, K]")
    _check(w.dtype == torch.float8_e4m3fn and w.stride(1) == 1, "w must be float8_e4m3fn [N, K], contiguous in dim 1")
    n, k = w.shape
    _check(x.size(1) == k, f"x K ({x.size(1)}) must match w K ({k})")
    _check(x.dtype == (torch.float16 if raw else torch.bfloat16), f"x must be {'float16' if raw else 'bfloat16'}")
    _check(x.stride(1) == 1, "x must be contiguous in dim 1")
    block, s_ld = _fp8_scales_dense(scales, n, k)
    if not block:
        scales = scales.contiguous()
    m = x.size(0)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _lib.call("strix_fp8_w8a16_gemm", _ptr(w), w.stride(0), _ptr(scales), s_ld, int(block), _ptr(x), _act_code(x),
              x.stride(0), _ptr(out), n, _lib.BF16, m, n, k, cfg, _stream(x))
    return out


# Reference schemas: csrc/torch_ops.cpp:253-256.
@_define("fp8_wmma_gemm(Tensor w, Tensor x, Tensor scales) -> Tensor")
def fp8_wmma_gemm(w, x, scales):
    return _fp8_w8a16(w, x, scales, False, -1)


@_fake("fp8_wmma_gemm")
def _(w, x, scales):
    return x.new_empty((x.size(0), w.size(0)))


@_define("fp8_wmma_gemm_cfg(Tensor w, Tensor x, Tensor scales, int cfg) -> Tensor")
def fp8_wmma_gemm_cfg(w, x, scales, cfg):
    return _fp8_w8a16(w, x, scales, False, int(cfg))


@_fake("fp8_wmma_gemm_cfg")
def _(w, x, scales, cfg):
    return x.new_empty((x.size(0), w.size(0)))


@_define("fp8_wmma_gemm_raw(Tensor w, Tensor x, Tensor scales) -> Tensor")
def fp8_wmma_gemm_raw(w, x, scales):
    return _fp8_w8a16(w, x, scales, True, -1)


@_fake("fp8_wmma_gemm_raw")
def _(w, x, scales):
    return x.new_empty((x.size(0), w.size(0)), dtype=torch.bfloat16)


@_define("fp8_wmma_gemm_raw_cfg(Tensor w, Tensor x, Tensor scales, int cfg) -> Tensor")
def fp8_wmma_gemm_raw_cfg(w, x, scales, cfg):
    return _fp8_w8a16(w, x, scales, True, int(cfg))


@_fake("fp8_wmma_gemm_raw_cfg")
def _(w, x, scales, cfg):
    return x.new_empty((x.size(0), w.size(0)), dtype=torch.bfloat16)


@_define("fp8_dequant(Tensor w, Tensor scales) -> Tensor")
def fp8_dequant(w, scales):
    _check(w.dim() == 2 and w.dtype == torch.float8_e4m3fn and w.stride(1) == 1, "w must be float8_e4m3fn [N, K]")
    n, k = w.shape
    block, s_ld = _fp8_scales_dense(scales, n, k)
    if not block:
        scales = scales.contiguous()
    out = torch.empty((n, k), dtype=torch.bfloat16, device=w.device)
    _lib.call("strix_dequant_bf16", _lib.FMT_FP8, _ptr(w), w.stride(0), _ptr(scales), _lib.S_F32, s_ld,
              128 if block else 0, 128 if block else 1, _ptr(out), k, n, k, _stream(w))
    return out


@_fake("fp8_dequant")
def _(w, scales):
    return w.new_empty((w.size(0), w.size(1)), dtype=torch.bfloat16)


@_define("_cvt_probe(Tensor scales, Tensor bf16_in) -> (Tensor, Tensor, Tensor)")
def _cvt_probe(scales, bf16_in):
    _check(scales.dtype == torch.float32 and bf16_in.dtype == torch.float32, "float32 inputs")
    s = scales.contiguous()
    x = bf16_in.contiguous()
    fp4 = torch.empty((s.numel(), 4, 256, 2), dtype=torch.int16, device=s.device)
    fp8 = torch.empty((256,), dtype=torch.float32, device=s.device)
    b16 = torch.empty((x.numel(),), dtype=torch.int16, device=s.device)
    _lib.call("strix_probe_cvt", _ptr(s), s.numel(), _ptr(fp4), _ptr(fp8), _ptr(b16), _ptr(x), x.numel(), _stream(s))
    return fp4, fp8, b16


@_fake("_cvt_probe")
def _(scales, bf16_in):
    return (scales.new_empty((scales.numel(), 4, 256, 2), dtype=torch.int16), scales.new_empty((256,)),
            bf16_in.new_empty((bf16_in.numel(),), dtype=torch.int16))


# ----------------------------------------------------------------- weight-only decode / ExLlama int4 / W4A8
# All of these run on strix_w16_gemm: the packed weights are decoded to
# bf16/fp16 in registers (decode M) or LDS (prefill M) and contracted with
# 16-bit MFMA. CuCount arguments are accepted for schema compatibility; the
# gfx950 kernels size their grids themselves.
def _w16(fmt, w, x, scales, s_kind, s_ns, s_ks, kgroup, nblock, bias, cfg=-1):
    n, m, k = w.size(0), x.size(0), x.size(1)
    out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    bias_rs = 0
    if bias is not None:
        _check(bias.dtype == x.dtype, "bias must have the activation dtype")
        if bias.dim() == 2:
            _check(tuple(bias.shape) == (m, n) and bias.stride(1) == 1, "bias must be [N] or [M, N]")
            bias_rs = bias.stride(0)
        else:
            _check(bias.numel() == n, "bias must be [N] or [M, N]")
            bias = bias.contiguous()
    _lib.call("strix_w16_gemm", fmt, _ptr(w), w.stride(0), _ptr(scales), s_kind, s_ns, s_ks, kgroup, nblock, _ptr(x),
              _act_code(x), x.stride(0), _ptr(bias), bias_rs, _ptr(out), n, _act_code(out), m, n, k, cfg, _stream(x))
    return out


def _skinny_rows(x, name="w8a16_skinny_gemm"):
    _check(1 <= x.size(0) <= 8, f"{name} takes 1-8 rows, got {x.size(0)}")


# Reference schema: csrc/torch_ops.cpp:250-252 (csrc/gemm/w8a16_skinny_gemm.hip:525-766).
@_define(
    "w8a16_skinny_gemm(Tensor in_a, Tensor in_b, Tensor in_scale, "
    "Tensor? in_bias, int CuCount, int group_size) -> Tensor"
)
def w8a16_skinny_gemm(in_a, in_b, in_scale, in_bias, CuCount, group_size):
    _check(in_a.dim() == 2 and in_b.dim() == 2, "Weights must be [N, K] and activations [M, K]")
    _check(in_a.dtype == torch.uint8, f"Weights must be uint8 (uint8b128), got {in_a.dtype}")
    _check(in_b.dtype in (torch.float16, torch.bfloat16), "Activation must be float16 or bfloat16")
    _check(in_scale.dtype == in_b.dtype, "Scale dtype must match activation dtype")
    _check(group_size in (0, 32, 64, 128), f"group_size must be 0 (per-channel), 32, 64, or 128, got {group_size}")
    n, k = in_a.shape
    _check(in_b.size(1) == k and in_b.stride(1) == 1 and in_a.stride(1) == 1, "K mismatch or non-contiguous rows")
    _skinny_rows(in_b)
    if group_size:
        _check(k % group_size == 0, f"K must be divisible by group_size={group_size}")
        _check(in_scale.dim() == 2 and tuple(in_scale.shape) == (n, k // group_size) and _unit_last(in_scale),
               f"Scale must be [{n}, {k // group_size}] but got {list(in_scale.shape)}")
        s_ns, s_ks = in_scale.stride(0), 1
    else:
        _check(in_scale.dim() == 1 and in_scale.numel() == n, f"Per-channel scale must be [{n}]")
        in_scale = in_scale.contiguous()
        s_ns, s_ks = 1, 0
    return _w16(_lib.FMT_U8B128, in_a, in_b, in_scale, _SCALE_KIND[in_scale.dtype], s_ns, s_ks, group_size, 1,
                in_bias)


@_fake("w8a16_skinny_gemm")
def _(in_a, in_b, in_scale, in_bias, CuCount, group_size):
    return in_b.new_empty((in_b.size(0), in_a.size(0)))


# New op (no reference schema): the same uint8b128 W8A16 contraction at any
# M, for the group sizes the W8A8 op does not take (32, 64). Bf16/fp16
# activations are used as given; weights are decoded exactly in registers
# (M <= 64) or LDS (larger M) and contracted with 16-bit MFMA.
@_define("w8a16_gemm(Tensor in_a, Tensor in_b, Tensor in_scale, Tensor? in_bias, int group_size) -> Tensor")
def w8a16_gemm(in_a, in_b, in_scale, in_bias, group_size):
    _check(in_a.dim() == 2 and in_b.dim() == 2, "Weights must be [N, K] and activations [M, K]")
    _check(in_a.dtype == torch.uint8, f"Weights must be uint8 (uint8b128), got {in_a.dtype}")
    _check(in_b.dtype in (torch.float16, torch.bfloat16), "Activation must be float16 or bfloat16")
    _check(in_scale.dtype == in_b.dtype, "Scale dtype must match activation dtype")
    _check(group_size in (0, 32, 64, 128), f"group_size must be 0 (per-channel), 32, 64, or 128, got {group_size}")
    n, k = in_a.shape
    _check(in_b.size(1) == k and in_b.stride(1) == 1 and in_a.stride(1) == 1, "K mismatch or non-contiguous rows")
    _check(k % 64 == 0, f"K must be a multiple of 64, got K={k}")
    if group_size:
        _check(k % group_size == 0, f"K must be divisible by group_size={group_size}")
        _check(in_scale.dim() == 2 and tuple(in_scale.shape) == (n, k // group_size) and _unit_last(in_scale),
               f"Scale must be [{n}, {k // group_size}] but got {list(in_scale.shape)}")
        s_ns, s_ks = in_scale.stride(0), 1
    else:
        _check(in_scale.numel() == n, f"Per-channel scale must be [{n}]")
        in_scale = in_scale.reshape(-1).contiguous()
        s_ns, s_ks = 1, 0
    return _w16(_lib.FMT_U8B128, in_a, in_b, in_scale, _SCALE_KIND[in_scale.dtype], s_ns, s_ks, group_size, 1,
                in_bias)


@_fake("w8a16_gemm")
def _(in_a, in_b, in_scale, in_bias, group_size):
    return in_b.new_empty((in_b.size(0), in_a.size(0)))


# Reference schema: csrc/torch_ops.cpp:253-255: e4m3 weights, fp32 scales per
# row [N] or per (row, 128-K block) [N, K/128].
@_define(
    "fp8_skinny_gemm(Tensor in_a, Tensor in_b, Tensor in_scale, "
    "Tensor? in_bias, int CuCount) -> Tensor"
)
def fp8_skinny_gemm(in_a, in_b, in_scale, in_bias, CuCount):
    _check(in_a.dim() == 2 and in_b.dim() == 2, "Weights must be [N, K] and activations [M, K]")
    _check(in_a.dtype == torch.float8_e4m3fn, f"Weights must be float8_e4m3fn, got {in_a.dtype}")
    _check(in_b.dtype in (torch.float16, torch.bfloat16), "Activation must be float16 or bfloat16")
    _check(in_scale.dtype == torch.float32, "fp8 scales must be float32")
    n, k = in_a.shape
    _check(in_b.size(1) == k and in_b.stride(1) == 1 and in_a.stride(1) == 1, "K mismatch or non-contiguous rows")
    _skinny_rows(in_b)
    if in_scale.dim() == 2:
        _check(tuple(in_scale.shape) == (n, k // 128) and _unit_last(in_scale) and k % 128 == 0,
               f"Scale must be [{n}, {k // 128}] but got {list(in_scale.shape)}")
        s_ns, s_ks, kgroup = in_scale.stride(0), 1, 128
    else:
        _check(in_scale.numel() == n, f"Per-channel scale must be [{n}]")
        in_scale = in_scale.contiguous()
        s_ns, s_ks, kgroup = 1, 0, 0
    return _w16(_lib.FMT_FP8, in_a.view(torch.uint8), in_b, in_scale, _lib.S_F32, s_ns, s_ks, kgroup, 1, in_bias)


@_fake("fp8_skinny_gemm")
def _(in_a, in_b, in_scale, in_bias, CuCount):
    return in_b.new_empty((in_b.size(0), in_a.size(0)))


# Reference schema: csrc/torch_ops.cpp:293 (csrc/gemm/mxfp4_gemv.hip:110-147).
@_define("mxfp4_gemv(Tensor x, Tensor w, Tensor scales) -> Tensor")
def mxfp4_gemv(x, w, scales):
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1 and x.stride(0) % 8 == 0,
           "x must be bf16 [M, K] with 16-byte aligned rows")
    _check(w.dtype == torch.uint8 and w.dim() == 2 and w.stride(1) == 1 and w.stride(0) % 16 == 0,
           "w must be uint8 [N, K/2] with 16-byte aligned rows")
    m, k = x.shape
    n = w.size(0)
    _check(1 <= m <= 8, "mxfp4_gemv is for M <= 8")
    _check(w.size(1) * 2 == k and k % 32 == 0, "K mismatch or K % 32")
    _check(scales.dtype == torch.uint8 and tuple(scales.shape) == (n, k // 32) and _unit_last(scales),
           "scales must be uint8 [N, K/32]")
    return _w16(_lib.FMT_MXFP4, w, x, scales, _lib.S_E8M0, scales.stride(0), 1, 32, 1, None)


@_fake("mxfp4_gemv")
def _(x, w, scales):
    return x.new_empty((x.size(0), w.size(0)))


def _int4_ex_checks(w, n_scales, k, group_size, scales):
    _check(w.dtype in (torch.int8, torch.uint8) and w.dim() == 2 and w.stride(1) == 1 and w.stride(0) % 8 == 0,
           "w must be int8 [N, K/2] (RDNAHybridW4A16 words) with 8-byte aligned rows")
    _check(w.size(1) * 2 == k and k % 64 == 0, "K mismatch or K % 64")
    _check(group_size % 32 == 0 and k % group_size == 0, "group_size % 32 and K % group")
    _check(scales.dtype == torch.bfloat16 and scales.dim() == 2 and tuple(scales.shape) == (n_scales, k // group_size)
           and _unit_last(scales), "scales must be bf16 [N, K / group_size]")


# Reference schema: csrc/torch_ops.cpp:266-268: uint4b8 weights in the
# RDNAHybridW4A16 word order, bf16 group scales, optional bf16 bias.
@_define("w4a16_wmma_gemm(Tensor x, Tensor w, Tensor scales, Tensor? bias, int group_size) -> Tensor")
def w4a16_wmma_gemm(x, w, scales, bias, group_size):
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1 and x.stride(0) % 8 == 0,
           "x must be bf16 [M, K] with 16-byte aligned rows")
    m, k = x.shape
    n = w.size(0)
    _int4_ex_checks(w, n, k, group_size, scales)
    if bias is not None:
        _check(bias.dtype == torch.bfloat16 and bias.numel() == n, "bias")
    return _w16(_lib.FMT_INT4_EX, w.view(torch.uint8), x, scales, _lib.S_BF16, scales.stride(0), 1, group_size, 1,
                bias)


@_fake("w4a16_wmma_gemm")
def _(x, w, scales, bias, group_size):
    return x.new_empty((x.size(0), w.size(0)))


# Reference schema: csrc/torch_ops.cpp:295: bf16 of (u4 - 8) * scale, exact.
@_define("w4a16_dequant(Tensor w, Tensor scales, int group_size) -> Tensor")
def w4a16_dequant(w, scales, group_size):
    n, k = w.size(0), 2 * w.size(1)
    _int4_ex_checks(w, n, k, group_size, scales)
    out = torch.empty((n, k), dtype=torch.bfloat16, device=w.device)
    _lib.call("strix_dequant_bf16", _lib.FMT_INT4_EX, _ptr(w), w.stride(0), _ptr(scales), _lib.S_BF16,
              scales.stride(0), group_size, 1, _ptr(out), k, n, k, _stream(w))
    return out


@_fake("w4a16_dequant")
def _(w, scales, group_size):
    return w.new_empty((w.size(0), 2 * w.size(1)), dtype=torch.bfloat16)


# Reference schema: csrc/torch_ops.cpp:283: uint4b8 RDNAHybridW4A16 weights,
# activations quantized to int8 per (row, 128-group) inside the op, fp32
# weight scales [N] (one group) or [G, N] / [N, G]
# (csrc/gemm/w8a8_wmma_gemm.hip:940-1000). Per-channel and 128-K weight
# groups run on the int8 MFMA (strix_w4a8_gemm: int32 sums per 128-group,
# folded in fp32 with both scales, as the reference's fold does); 32-K groups
# (which change the weight scale inside an MFMA's 64-K step) dequantize the
# int8 activations and run the int4 bf16-MFMA GEMM.
@_define("w4a8_wmma_gemm(Tensor in_w4, Tensor in_act, Tensor in_scale) -> Tensor")
def w4a8_wmma_gemm(in_w4, in_act, in_scale):
    _check(in_act.dim() == 2 and in_act.dtype == torch.bfloat16, "Activation must be bf16 [M, K]")
    m, k = in_act.shape
    n = in_w4.size(0)
    _check(in_w4.dim() == 2 and in_w4.dtype in (torch.int8, torch.uint8) and in_w4.stride(1) == 1
           and 2 * in_w4.size(1) == k, "Weights must be int8 [N, K/2]")
    _check(k % 128 == 0, f"K must be divisible by 128, got K={k}")
    _check(in_scale.dtype == torch.float32, f"Scale must be float32, got {in_scale.dtype}")
    if in_scale.dim() == 1:
        _check(in_scale.numel() == n, f"Per-channel scale must be [N={n}]")
        scale, s_ns, s_ks, group = in_scale.contiguous(), 1, 0, 0
    else:
        g = in_scale.size(0) if in_scale.size(1) == n else in_scale.size(1)
        _check(g >= 1 and k % g == 0, "Scale must be [G, N], [N, G] or [N]")
        group = k // g
        if tuple(in_scale.shape) == (g, n) and in_scale.stride(1) == 1:
            scale, s_ns, s_ks = in_scale, 1, in_scale.stride(0)
        else:
            _check(tuple(in_scale.shape) == (n, g) and in_scale.stride(1) == 1,
                   f"Scale must be [G, N], [N, G] or [N={n}] but got {list(in_scale.shape)}")
            scale, s_ns, s_ks = in_scale, in_scale.stride(0), 1
        _check(group % 32 == 0, f"weight group ({group}) must be a multiple of 32")
        if g == 1:
            s_ks, group = 0, 0          # one group over K: per-channel
    x = in_act.contiguous()
    st = _stream(x)
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    sa = torch.empty((m, k // 128), dtype=torch.float32, device=x.device)
    if m:
        _lib.call("strix_int8_quant_group128", _ptr(x), _act_code(x), k, _ptr(q), k, _ptr(sa), k // 128, m, k, st)
    w = in_w4.view(torch.uint8)
    if group in (0, 128) and w.stride(0) % 16 == 0 and w.data_ptr() % 16 == 0:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
        _lib.call("strix_w4a8_gemm", _ptr(q), k, _ptr(sa), k // 128, _ptr(w), w.stride(0), 2, _ptr(scale), s_ns,
                  s_ks, _ptr(out), n, _lib.BF16, m, n, k, st)
        return out
    xd = torch.empty((m, k), dtype=torch.bfloat16, device=x.device)
    if m:
        _lib.call("strix_int8_dequant_group128", _ptr(q), k, _ptr(sa), k // 128, _ptr(xd), _lib.BF16, k, m, k, st)
    return _w16(_lib.FMT_INT4_EX, w, xd, scale, _lib.S_F32, s_ns, s_ks, group, 1, None)


@_fake("w4a8_wmma_gemm")
def _(in_w4, in_act, in_scale):
    return in_act.new_empty((in_act.size(0), in_w4.size(0)))


# Reference schema: csrc/torch_ops.cpp:213-217: int8 activations per (row,
# 128-group) (moe_act_quant_i8) x int4 experts in the WNA16 layout (uint8
# [E, N, K/2], low nibble = even k, value q - 8) with bf16/fp16 scales per
# 128-K group (csrc/moe/moe_gemm_w4a8.hip:371-463, the same checks). The
# experts run on the int8 MFMA: nibbles widened to int8 in the tile, an exact
# int32 sum per 128-group, folded in fp32 with sa and the (exactly widened)
# weight scale. Tiles: the reference's three (block_m, block_n) pairs, and
# 256 x 256.
_W4A8_TILES = ((64, 256), (128, 128), (64, 128), (256, 256))


@_define(
    "moe_gemm_w4a8(Tensor(a!) c, Tensor qa, Tensor sa, Tensor b, Tensor scales, "
    "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_padded, "
    "Tensor? topk_weights, int top_k, int block_m, int block_n, "
    "bool silu_mul=False, str activation='silu') -> ()"
)
def moe_gemm_w4a8(c, qa, sa, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m,
                  block_n, silu_mul=False, activation="silu"):
    _check(qa.dtype == torch.int8 and sa.dtype == torch.float32 and b.dtype == torch.uint8
           and scales.dtype in (torch.bfloat16, torch.float16) and c.dtype == torch.bfloat16,
           "moe_gemm_w4a8: qa int8, sa fp32, w uint8, scales bf16/fp16, c bf16")
    _check(qa.dim() == 2 and b.dim() == 3 and scales.dim() == 3 and c.dim() == 2, "moe_gemm_w4a8: ranks")
    _check(qa.is_contiguous() and sa.is_contiguous() and b.stride(2) == 1 and _unit_last(scales)
           and c.stride(1) == 1, "moe_gemm_w4a8: layouts")
    rows, k = qa.shape
    e, n = b.size(0), b.size(1)
    _check(b.size(2) * 2 == k and qa.size(1) == k and sa.numel() == rows * (k // 128),
           "qa [rows, K], sa [rows, K/128], w [E, N, K/2]")
    _check(c.size(1) == (n // 2 if silu_mul else n), "c shape mismatch")
    _check(not silu_mul or (n % 2 == 0 and topk_weights is None), "silu_mul needs even N and no topk_weights")
    _check(k % 128 == 0 and n % block_n == 0, "K % 128 and N % block_n")
    _check(tuple(scales.shape) == (e, n, k // 128), "scales must be [E, N, K / 128]")
    _check(b.stride(1) % 8 == 0 and b.stride(0) % 8 == 0, "w strides must be multiples of 8")
    _check((block_m, block_n) in _W4A8_TILES, f"moe_gemm_w4a8: unsupported block_m/block_n {block_m}/{block_n}")
    _moe_common(c, sorted_ids, expert_ids, num_post_padded, topk_weights, block_m)
    code = _activation(activation)
    sw = scales.float()            # bf16 / fp16 -> fp32 is exact
    _lib.call("strix_moe_gemm_w4a8", _ptr(c), c.stride(0), _lib.BF16, _ptr(qa), k, _ptr(sa), k // 128, _ptr(b),
              b.stride(0), b.stride(1), _ptr(sw), sw.stride(0), sw.stride(1), _ptr(sorted_ids), sorted_ids.numel(),
              _ptr(expert_ids), expert_ids.numel(), _ptr(num_post_padded), _ptr(topk_weights), c.size(0), top_k,
              block_m, int(silu_mul), code, n, k, _stream(qa))


@_fake("moe_gemm_w4a8")
def _(c, qa, sa, b, scales, sorted_ids, expert_ids, num_post_padded, topk_weights, top_k, block_m, block_n,
      silu_mul=False, activation="silu"):
    return None


# Reference schema: csrc/torch_ops.cpp:183 (the fragment-layout probe of
# tests/test_wmma_layout.py): D[16,16] = A[16,K] . B[16,K]^T in fp32 through
# the bf16 MFMA. K is zero-padded to the MFMA's 32.
@_define("_wmma_bf16_tile(Tensor a, Tensor b) -> Tensor")
def _wmma_bf16_tile(a, b):
    _check(a.dim() == 2 and a.shape == b.shape and a.size(0) == 16 and a.dtype == b.dtype == torch.bfloat16,
           "a, b must be bf16 [16, K]")
    k = a.size(1)
    kp = -(-k // 32) * 32
    if kp != k:
        a = torch.nn.functional.pad(a, (0, kp - k))
        b = torch.nn.functional.pad(b, (0, kp - k))
    return _mfma_tile(a, b)


@_fake("_wmma_bf16_tile")
def _(a, b):
    return a.new_empty((16, 16), dtype=torch.float32)
