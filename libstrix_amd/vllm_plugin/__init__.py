# SPDX-License-Identifier: MIT
"""vLLM general plugin: swaps the quantized linears and fused-MoE experts of a
vLLM process onto libstrix_amd's gfx950 kernels.

The MI355X counterpart of the reference's `strix_vllm` package
(python/strix_vllm/__init__.py:1-199). vLLM loads it through the
`vllm.general_plugins` entry point (`strix = libstrix_amd.vllm_plugin:register`)
in every process, possibly more than once; `register()` is idempotent.

Environment, as in the reference (python/strix_vllm/__init__.py:18-24):
  STRIX_DISABLE=all, or a comma list of swap names, keeps vLLM's own kernels
  for those swaps. Names: w8a8, fp8, fp8_channel, fp8_w8a8, mxfp4, w8a16,
  w4a16, moe_gemm, moe_pad, moe_w4a16, moe_fp8, moe_fp8_w8a8, moe_w8a16,
  moe_w4a8, moe_mxfp4.
  STRIX_ENABLE=<names> turns on the opt-in swaps (ARCH_GATED) for any model.

The modules split as in the reference: `int8` (W8A8 int8 linears), `fp8`
(FP8 block and per-channel linears), `mxfp4` (MXFP4 W4A16 linears), `linear`
(W8A16 uint8b128 and W4A16 uint4b8 linears) and `moe` (fused-MoE experts).
Each keeps its tile tables, gates and per-forward dispatch (`_apply_impl`)
free of vLLM imports, so they run and are tested without vLLM; only the
`register()` functions and the kernel-class factories import vLLM.
"""

from __future__ import annotations

import hashlib
import os
from pathlib import Path

_registered = False
# vLLM env factor that ties compile caches to the plugin (see _cache_factor).
CACHE_FACTOR = "STRIX_VLLM_CACHE_KEY"
ARCH = "gfx950"

# Swaps that change numerics against the layer's own quantization scheme and
# so stay off unless STRIX_ENABLE names them or the model is listed here.
# moe_w4a8: int8 activations (per row and 128-element group) into the int4
# expert GEMMs. On gfx950 the bf16-activation int4 path is already
# MFMA-bound at bf16 rates, so no architecture turns it on by default.
ARCH_GATED: dict[str, tuple[str, ...]] = {
    "moe_w4a8": (),
}


def _env_names(var: str) -> set[str]:
    return {s.strip() for s in os.environ.get(var, "").split(",") if s.strip()}


def disabled(op: str) -> bool:
    """STRIX_DISABLE=all or a list naming `op` (python/strix_vllm/__init__.py:22-24)."""
    names = _env_names("STRIX_DISABLE")
    return "all" in names or op in names


def enabled(op: str) -> bool:
    """STRIX_ENABLE names `op` and STRIX_DISABLE does not."""
    return op in _env_names("STRIX_ENABLE") and not disabled(op)


def _model_architectures() -> list[str]:
    """Names the model being loaded goes by: its HF `architectures` list and
    vLLM's resolved architecture, without repeats. Empty without vLLM or
    outside a model load (the role of python/strix_vllm/__init__.py:62-75)."""
    try:
        from vllm.config import get_current_vllm_config_or_none
    except ImportError:
        return []
    mc = getattr(get_current_vllm_config_or_none(), "model_config", None)
    if mc is None:
        return []
    names = [*(getattr(getattr(mc, "hf_config", None), "architectures", None) or [])]
    resolved = getattr(type(mc), "architecture", None)
    if resolved is not None:
        try:
            names.append(mc.architecture)
        except (AttributeError, ValueError, RuntimeError):
            pass   # vLLM could not resolve one; the HF names stand
    return list(dict.fromkeys(n for n in names if isinstance(n, str)))


def model_gate(op: str, archs: list[str] | None = None) -> bool:
    """Whether an ARCH_GATED swap applies to the model being loaded
    (python/strix_vllm/__init__.py:78-95)."""
    if disabled(op):
        return False
    if op in _env_names("STRIX_ENABLE"):
        return True
    archs = _model_architectures() if archs is None else archs
    return any(a in ARCH_GATED.get(op, ()) for a in archs)


def on_gfx950() -> bool:
    """Whether device 0 is an MI355X-class gfx950 under ROCm torch."""
    import torch

    if torch.version.hip is None or not torch.cuda.is_available():
        return False
    return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0] == ARCH


def _cache_factor(active: bool) -> str:
    """A short key for vLLM's compile caches. The dispatchers run inside code
    torch.compile traces, and vLLM keys its caches on its own configuration
    only, so a graph traced with the plugin off, under other STRIX_* settings,
    or with other op wrappers must not be replayed. The key covers exactly
    those inputs: the activity flag, the two environment lists (as sorted
    sets, so order and spacing do not matter) and the source text of the
    plugin modules and of the torch op layer they call (the role of
    python/strix_vllm/__init__.py:119-134)."""
    import json

    pkg = Path(__file__).resolve().parent
    sources = sorted(pkg.glob("*.py")) + [pkg.parent / "torch_ops.py"]
    state = {
        "active": bool(active),
        "disable": sorted(_env_names("STRIX_DISABLE")),
        "enable": sorted(_env_names("STRIX_ENABLE")),
        "sources": {f.name: hashlib.blake2b(f.read_bytes(), digest_size=16).hexdigest()
                    for f in sources if f.exists()},
    }
    return hashlib.blake2b(json.dumps(state, sort_keys=True).encode(), digest_size=8).hexdigest()


def register() -> None:
    """vLLM entry point (python/strix_vllm/__init__.py:137-199): active on ROCm
    with a gfx950 device 0 and STRIX_DISABLE not `all`."""
    global _registered
    if _registered:
        return
    _registered = True

    from vllm import envs
    from vllm.logger import init_logger
    from vllm.platforms import current_platform

    active = current_platform.is_rocm() and on_gfx950()
    key = _cache_factor(active)
    envs.environment_variables.setdefault(CACHE_FACTOR, lambda: key)
    logger = init_logger(f"vllm.{__name__}")
    if not current_platform.is_rocm():
        return
    if not active:
        logger.info("libstrix_amd: device 0 is not %s, plugin inactive", ARCH)
        return
    if disabled("all"):
        logger.info("libstrix_amd: disabled by STRIX_DISABLE=all")
        return

    import libstrix_amd

    if not libstrix_amd.library_available():
        raise RuntimeError("libstrix_amd/_strix_amd.so is not built (python libstrix_amd/build.py)")

    from libstrix_amd.vllm_plugin import fp8, int8, linear, moe, mxfp4

    int8.register()
    linear.register()
    mxfp4.register()
    fp8.register()
    moe.register()
    logger.info("libstrix_amd: plugin registered")
