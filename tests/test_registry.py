# SPDX-License-Identifier: MIT
"""The kernel table (CPU only): coverage of the registered ops and the query
semantics of the reference's tests/test_registry.py."""

import torch

import libstrix_amd
from libstrix_amd import torch_ops


def test_every_registered_op_is_in_the_table():
    registered = set(torch_ops.SCHEMAS)
    described = {k["name"] for k in libstrix_amd.kernels()}
    probes = {n for n in registered if n.startswith("_")}
    assert registered - described == probes, f"registered but not in the table: {registered - described - probes}"
    assert not (described - registered), f"in the table but not registered: {described - registered}"


def test_table_has_no_duplicate_rows():
    seen = set()
    for k in libstrix_amd.kernels():
        key = (k["name"], k["op"], tuple(sorted((a, str(b)) for a, b in k["constraints"].items())))
        assert key not in seen, k["name"]
        seen.add(key)


def test_select_first_match_and_reasons():
    geo = {"weight_dtype": "fp8_e4m3", "activation_dtype": torch.float8_e4m3fn, "group_size": 128}
    assert libstrix_amd.select("fp8_w8a8", **geo) == "fp8_w8a8_block_gemm"
    assert libstrix_amd.select("fp8_w8a8", **{**geo, "group_size": 64}) is None
    rows = libstrix_amd.explain("fp8_w8a8", **{**geo, "group_size": 64})
    assert rows[0]["reason"] == "group_size=64, needs == 128"
    assert libstrix_amd.select("w8a16", weight_bits=8, group_size=128, rows=512, dtype=torch.bfloat16) == "w8a8_wmma_gemm"
    reasons = [r["reason"] for r in libstrix_amd.explain("w8a16", weight_bits=8, group_size=128, rows=3,
                                                          dtype=torch.bfloat16)]
    assert "rows=3, needs >= 6" in reasons[0]


def test_range_semantics():
    r = libstrix_amd.Range(lo=6)
    assert r.covers(6) and not r.covers(5) and not r.covers(True) and str(r) == ">= 6"
    assert str(libstrix_amd.Range(hi=5)) == "<= 5" and str(libstrix_amd.Range(1, 4)) == "in 1..4"


def test_selections_record_queries():
    before = {(s["op"], tuple(sorted(s["query"].items()))): s["count"] for s in libstrix_amd.selections()}
    libstrix_amd.select("moe_align", num_experts=128)
    libstrix_amd.select("moe_align", num_experts=128)
    after = {(s["op"], tuple(sorted(s["query"].items()))): s for s in libstrix_amd.selections()}
    rec = after[("moe_align", (("num_experts", 128),))]
    assert rec["kernel"] == "moe_align"
    assert rec["count"] == before.get(("moe_align", (("num_experts", 128),)), 0) + 2


def test_unknown_op_explains_nothing():
    assert libstrix_amd.explain("no_such_op", head_dim=256) == []
    assert libstrix_amd.select("no_such_op") is None
