# SPDX-License-Identifier: MIT
"""strix_moe_align_noalloc: the align with its histogram in the library's
static device array, called through the C ABI. Its outputs must equal
strix_moe_align's (caller workspace) bit for bit, on consecutive calls that
reuse the array (the second call smaller than the first, so stale counts from
the first would show), and it must reject inputs whose histogram exceeds the
array before touching the GPU."""

import pytest
import torch

from libstrix_amd import _lib


def _align_args(ids: torch.Tensor, e: int, bm: int, fill: int):
    s = ids.numel()
    cap = _lib.query("strix_moe_align_sorted_capacity", s, e, bm)
    blocks = -(-cap // bm)
    dev = ids.device
    sorted_ids = torch.full((cap,), fill, dtype=torch.int32, device=dev)
    expert_ids = torch.full((blocks,), fill, dtype=torch.int32, device=dev)
    num_post = torch.full((1,), fill, dtype=torch.int32, device=dev)
    return s, cap, blocks, sorted_ids, expert_ids, num_post


def _with_workspace(ids, e, bm):
    s, cap, blocks, so, ex, npp = _align_args(ids, e, bm, -5)
    ws = torch.empty(_lib.query("strix_moe_align_workspace_bytes", s, e), dtype=torch.uint8, device=ids.device)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("strix_moe_align", ids.data_ptr(), s, e, bm, so.data_ptr(), cap, ex.data_ptr(), blocks,
              npp.data_ptr(), ws.data_ptr(), ws.numel(), st)
    return so, ex, npp


def _no_alloc(ids, e, bm):
    s, cap, blocks, so, ex, npp = _align_args(ids, e, bm, -9)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("strix_moe_align_noalloc", ids.data_ptr(), s, e, bm, so.data_ptr(), cap, ex.data_ptr(), blocks,
              npp.data_ptr(), st)
    return so, ex, npp


def _routing(t, k, e, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)


def test_no_alloc_rejects_oversized_histogram_on_host():
    assert _lib.query("strix_moe_align_noalloc_max_bytes") == 1 << 20
    # 262145 slots need 1025 chunks of 256; at E = 256 that is 1025 * 256 * 4 bytes > 1 MiB.
    with pytest.raises(RuntimeError, match="static scratch"):
        _lib.call("strix_moe_align_noalloc", 0, 262145, 256, 64, 0, 1 << 20, 0, 1 << 20, 0, 0)


@pytest.mark.gpu
def test_no_alloc_matches_workspace_align_on_consecutive_calls():
    dev = "cuda"
    # Large (three-pass align over 128 chunks), then smaller with fewer
    # experts (the array keeps the first call's counts), then the single-block
    # path, then the largest input the array takes.
    cases = [(4096, 8, 128, 64, 1), (600, 4, 32, 16, 2), (100, 8, 64, 32, 3), (65536, 8, 128, 256, 4)]
    for t, k, e, bm, seed in cases:
        print(f"no_alloc align: T={t} top_k={k} E={e} block_m={bm}", flush=True)
        ids = _routing(t, k, e, seed).to(dev)
        want = _with_workspace(ids, e, bm)
        got = _no_alloc(ids, e, bm)
        torch.cuda.synchronize()
        for w, g_ in zip(want, got):
            assert torch.equal(w.cpu(), g_.cpu())
        total = int(got[2].item())
        assert total >= t * k and (got[0].cpu()[total:] == t * k).all()
