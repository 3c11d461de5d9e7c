# SPDX-License-Identifier: MIT
"""Measurement helpers behind the `roofline` fields of bench.py's JSON line
and the summaries under profiles/.

    python -m libstrix_amd.profiling probe [WORKLOAD]
        Launches, on the current stream, a plain copy kernel of known size
        (torch's bitwise_not over 1 GiB of int32: 1 GiB read, 1 GiB written,
        four times the 256 MB Infinity Cache) and then WORKLOAD three times
        (default `headline`, the config-2 FP8-block GEMM at M=4096 N=17408
        K=5120; the others are listed in WORKLOADS). Meant to run under
        `rocprofv3 --pmc FETCH_SIZE`, again under `--pmc WRITE_SIZE`, or
        under one pass of SQ counters: one counter pass per run.

    python -m libstrix_amd.profiling traffic FETCH_DB WRITE_DB OUT_PREFIX [WORKLOAD]
        Reads the two rocprofv3 databases, scales each kernel's FETCH_SIZE /
        WRITE_SIZE (KiB per dispatch) by what the same counter reads for the
        copy kernel of known size, and writes OUT_PREFIX.json (for the
        headline, read by bench.py: `bytes_per_launch` becomes
        roofline.traffic) and OUT_PREFIX.md (the figures and the commands).

    python -m libstrix_amd.profiling sq OUT_MD TITLE WORKLOAD DB [DB ...]
        Per-kernel SQ counters (one rocprofv3 --pmc pass per DB) of a probe
        run, as averages per dispatch and the derived MFMA-busy fraction,
        VALU and LDS instructions per MFMA and wait shares.

    python -m libstrix_amd.profiling stats DB OUT_MD TITLE COMMAND
        Per-kernel calls / average / minimum / share of a
        `rocprofv3 --kernel-trace --stats` database as a markdown table.

The memory counters count L2 (TCC) traffic to the memory fabric, so bytes
served by the Infinity Cache count as traffic too: the figure is what the
kernel asks of the fabric beyond L2, the quantity that re-reads inflate.
"""

from __future__ import annotations

import json
import re
import sqlite3
import sys

COPY_ELEMS = 1 << 28            # int32 elements: 1 GiB
COPY_BYTES = COPY_ELEMS * 4
HEADLINE = dict(m=4096, n=17408, k=5120)
COPY_TAG = "bitwise_not"
GEMM_TAG = "tiled8"


def headline_algorithmic_bytes(m: int, n: int, k: int) -> int:
    """Bytes the headline GEMM launch must move at least once: e4m3 weights,
    128x128 fp32 weight scales, e4m3 activations, 1x128 fp32 activation
    scales and the bf16 output."""
    return n * k + ((n + 127) // 128) * (k // 128) * 4 + m * k + m * (k // 128) * 4 + m * n * 2


def _fp8_decode(m: int, kmajor: bool):
    import torch

    from libstrix_amd import workloads

    S = torch.ops.strix
    d = workloads.c2_fp8(seed=2, device="cuda", m=m, n=HEADLINE["n"], k=HEADLINE["k"])
    w = S.weight8_kmajor(d["w"]) if kmajor else d["w"]
    q, s = S.fp8_quant_group128(d["x"])
    if kmajor:
        return lambda: S.fp8_w8a8_block_gemm_kmajor(q, s, w, d["sw"])
    return lambda: S.fp8_w8a8_block_gemm(q, s, w, d["sw"])


def _int8_decode():
    import torch

    from libstrix_amd import workloads

    S = torch.ops.strix
    d = workloads.c1_int8(seed=1, device="cuda")
    q, s = S.int8_quant_per_token(d["x"])
    return lambda: S.w8a8_scaled_mm(q, s, d["w"], d["sw"])


def _moe(cfg: str, t: int):
    import torch

    from libstrix_amd import functional, workloads

    if cfg == "c3":
        d = workloads.c3_fp8_moe(seed=3, t=t, device="cuda")
        return lambda: functional.fused_moe_fp8_w8a8(d["x"], d["logits"], d["w13"], d["w13_s"], d["w2"], d["w2_s"],
                                                     d["top_k"])
    if cfg == "c4":
        d = workloads.c4_mxfp4_moe(seed=4, t=t, device="cuda")
        return lambda: functional.fused_moe_mxfp4(d["x"], d["logits"], d["w13"], d["w13_s"], d["w2"], d["w2_s"],
                                                  d["top_k"])
    d = workloads.c5_wna16_moe(seed=5, t=t, device="cuda")
    return lambda: functional.fused_moe_wna16(d["x"], d["logits"], d["w13"], d["w13_s"], d["w13_z"], d["w2"],
                                              d["w2_s"], d["w2_z"], d["top_k"], d["group"])


# name -> (description, builder of a zero-argument call, algorithmic bytes of one call or None)
def _dense_bytes(m: int) -> int:
    return headline_algorithmic_bytes(m, HEADLINE["n"], HEADLINE["k"])


WORKLOADS = {
    "headline": ("config-2 FP8-block GEMM, M=4096 N=17408 K=5120", lambda: _fp8_decode(4096, False),
                 _dense_bytes(4096)),
    "c2_m1": ("config-2 FP8-block GEMM, M=1 (row-major weights)", lambda: _fp8_decode(1, False), _dense_bytes(1)),
    "c2_m1_kmajor": ("config-2 FP8-block GEMM, M=1 (K-block-major weights, the plugin's layout)",
                     lambda: _fp8_decode(1, True), _dense_bytes(1)),
    "c2_m16_kmajor": ("config-2 FP8-block GEMM, M=16 (K-block-major weights)", lambda: _fp8_decode(16, True),
                      _dense_bytes(16)),
    "c2_m256_kmajor": ("config-2 FP8-block GEMM, M=256 (K-block-major weights)", lambda: _fp8_decode(256, True),
                       _dense_bytes(256)),
    "c1_m32": ("config-1 int8 W8A8 GEMM, M=32 N=K=5120", _int8_decode,
               5120 * 5120 + 5120 * 4 + 32 * 5120 + 32 * 4 + 32 * 5120 * 2),
    "c3_t1": ("config-3 FP8-block MoE, T=1", lambda: _moe("c3", 1), None),
    "c4_t1": ("config-4 MXFP4 MoE, T=1", lambda: _moe("c4", 1), None),
    "c5_t1": ("config-5 WNA16 MoE, T=1", lambda: _moe("c5", 1), None),
    "c3_t4096": ("config-3 FP8-block MoE, T=4096 (route, align, quant, w13, quant, w2, sum)",
                 lambda: _moe("c3", 4096), None),
    "c4_t2048": ("config-4 MXFP4 MoE, T=2048", lambda: _moe("c4", 2048), None),
    "c5_t8192": ("config-5 WNA16 MoE, T=8192", lambda: _moe("c5", 8192), None),
}


def probe(workload: str = "headline") -> None:
    import torch

    import libstrix_amd

    if not libstrix_amd.library_available():
        raise SystemExit("libstrix_amd/_strix_amd.so is not built")
    if workload not in WORKLOADS:
        raise SystemExit(f"unknown workload {workload!r}: one of {sorted(WORKLOADS)}")
    src = torch.randint(-2**31, 2**31 - 1, (COPY_ELEMS,), dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    call = WORKLOADS[workload][1]()
    torch.cuda.synchronize()
    for i in range(3):
        torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        print(f"probe: copy {i} done", flush=True)
    del src, dst
    for i in range(3):
        call()
        torch.cuda.synchronize()
        print(f"probe: {workload} {i} done", flush=True)


def _counter_rows(db_path: str, counter: str) -> list[tuple[int, str, float]]:
    db = sqlite3.connect(db_path)
    rows = db.execute("select dispatch_id, kernel_name, value from counters_collection where counter_name = ?",
                      (counter,)).fetchall()
    per: dict[int, list] = {}
    for disp, name, val in rows:
        e = per.setdefault(disp, [name, 0.0])
        e[1] += float(val)       # one row per XCD / instance on some versions: sum them
    return [(d, n, v) for d, (n, v) in sorted(per.items())]


def _pick(rows, tag: str) -> dict[str, list[float]]:
    """Counter values of the dispatches whose kernel name holds `tag`, by kernel."""
    out: dict[str, list[float]] = {}
    for _, n, v in rows:
        if tag in n:
            out.setdefault(_short(n), []).append(v)
    return out


def _med(v: list[float]) -> float:
    return sorted(v)[len(v) // 2]


def traffic(fetch_db: str, write_db: str, out_prefix: str, workload: str = "headline") -> dict:
    """Per kernel the median over dispatches; for the headline one op call
    may launch more than one kernel (the 256x256 rounds and a 128x128 strip
    for the leftover columns), and a launch's traffic is their sum. For the
    other workloads every kernel of the call is listed with its own figures."""
    desc, _, alg = WORKLOADS[workload]
    fr = _counter_rows(fetch_db, "FETCH_SIZE")
    wr = _counter_rows(write_db, "WRITE_SIZE")
    cf = [v for vs in _pick(fr, COPY_TAG).values() for v in vs]
    cw = [v for vs in _pick(wr, COPY_TAG).values() for v in vs]
    tag = GEMM_TAG if workload == "headline" else ""
    # Kernels of the timed call run three times; set-up kernels (weight
    # re-layout, input quantization) once.
    gf = {n: v for n, v in _pick(fr, tag).items() if COPY_TAG not in n and len(v) >= 3}
    gw = {n: v for n, v in _pick(wr, tag).items() if n in gf}
    if not (cf and cw and gf) or set(gf) != set(gw):
        raise SystemExit(f"missing dispatches: copy {len(cf)}/{len(cw)}, kernels {sorted(gf)} / {sorted(gw)}")
    copy_kib = COPY_BYTES / 1024.0
    f_factor = copy_kib / _med(cf)
    w_factor = copy_kib / _med(cw)
    per_kernel = {name: {"fetch_kib": round(_med(gf[name]), 1), "write_kib": round(_med(gw[name]), 1),
                         "fetch_bytes": int(round(_med(gf[name]) * 1024.0 * f_factor)),
                         "write_bytes": int(round(_med(gw[name]) * 1024.0 * w_factor)),
                         "dispatches": len(gf[name])}
                  for name in sorted(gf)}
    fetch_b = sum(k["fetch_bytes"] for k in per_kernel.values())
    write_b = sum(k["write_bytes"] for k in per_kernel.values())
    res = {
        "workload": workload,
        "kernel": ("tiled8_kernel<fp8 block> launches of one config-2 GEMM call (M=4096 N=17408 K=5120)"
                   if workload == "headline" else desc),
        "bytes_per_launch": fetch_b + write_b,
        "fetch_bytes_per_launch": fetch_b,
        "write_bytes_per_launch": write_b,
        "algorithmic_bytes_per_launch": alg,
        "traffic_over_algorithmic": round((fetch_b + write_b) / alg, 3) if alg else None,
        "per_kernel": per_kernel,
        "copy_known_bytes": COPY_BYTES,
        "copy_fetch_kib_raw": [round(v, 1) for v in cf],
        "copy_write_kib_raw": [round(v, 1) for v in cw],
        "fetch_scale": round(f_factor, 4),
        "write_scale": round(w_factor, 4),
    }
    with open(out_prefix + ".json", "w") as f:
        json.dump(res, f, indent=1)
    arg = "" if workload == "headline" else f" {workload}"
    cmd_f = ("timeout -s KILL 150 rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_fetch -o p -- "
             f"python3 -m libstrix_amd.profiling probe{arg}")
    cmd_w = cmd_f.replace("FETCH_SIZE", "WRITE_SIZE").replace("pmc_fetch", "pmc_write")
    md = [
        f"# HBM-side traffic: {desc}",
        "",
        "Commands (repo root on the MI355X box, `TMPDIR=/tmp`):",
        "",
        f"    {cmd_f}",
        f"    {cmd_w}",
        "    python3 -m libstrix_amd.profiling traffic gpurun_out/pmc_fetch/p_results.db "
        f"gpurun_out/pmc_write/p_results.db {out_prefix}{arg}",
        "",
        "Calibration: torch `bitwise_not` over 1 GiB of int32 (1 GiB read + 1 GiB written).",
        "",
        "| quantity | value |",
        "|---|---|",
        f"| copy FETCH_SIZE (KiB, median of {len(cf)}) | {_med(cf):.0f} (known {copy_kib:.0f}) -> scale {f_factor:.4f} |",
        f"| copy WRITE_SIZE (KiB, median of {len(cw)}) | {_med(cw):.0f} (known {copy_kib:.0f}) -> scale {w_factor:.4f} |",
    ]
    for name, k in per_kernel.items():
        md.append(f"| `{name}` FETCH_SIZE / WRITE_SIZE (KiB, median of {k['dispatches']}) | {k['fetch_kib']:.0f} / "
                  f"{k['write_kib']:.0f} -> {k['fetch_bytes'] / 1e6:.2f} / {k['write_bytes'] / 1e6:.2f} MB |")
    md.append(f"| traffic per call | {(fetch_b + write_b) / 1e6:.1f} MB (fetch {fetch_b / 1e6:.1f}, "
              f"write {write_b / 1e6:.1f}) |")
    if alg:
        md += [f"| algorithmic bytes per call | {alg / 1e6:.1f} MB |",
               f"| traffic / algorithmic | {(fetch_b + write_b) / alg:.3f} |"]
    md.append("")
    with open(out_prefix + ".md", "w") as f:
        f.write("\n".join(md))
    return res


# SQ counters of one pass each; the derived figures below use these names.
SQ_PASSES = [
    "SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_WAIT_INST_ANY SQ_WAIT_ANY "
    "SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS",
    "SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_INSTS_VALU SQ_INSTS_MFMA SQ_ACTIVE_INST_VMEM SQ_INST_LEVEL_VMEM "
    "SQ_ACTIVE_INST_ANY SQ_CYCLES",
    "SQ_INSTS_SALU SQ_INSTS_SMEM SQ_WAIT_INST_LDS SQ_INST_LEVEL_LDS SQ_LDS_DATA_FIFO_FULL SQ_LDS_CMD_FIFO_FULL "
    "SQ_VALU_MFMA_COEXEC_CYCLES SQ_ACTIVE_INST_MISC",
]
SIMDS = 256 * 4      # MI355X: 256 CUs of 4 SIMDs
SES = 32             # shader engines, over which SQ_BUSY_CYCLES sums


def sq(out_md: str, title: str, workload: str, *dbs: str) -> None:
    """SQ counters per kernel (average per dispatch over all its dispatches).
    SQ_BUSY_CYCLES sums over the shader engines, so the kernel's own cycles
    are SQ_BUSY_CYCLES / 32; MFMA busy is SQ_VALU_MFMA_BUSY_CYCLES over the
    SIMD cycles of that span (1024 SIMDs)."""
    per: dict[str, dict[str, float]] = {}
    for db_path in dbs:
        db = sqlite3.connect(db_path)
        rows = db.execute("select dispatch_id, kernel_name, counter_name, value from counters_collection").fetchall()
        disp: dict[tuple, float] = {}
        names: dict[int, str] = {}
        for d, n, c, v in rows:
            disp[(d, c)] = disp.get((d, c), 0.0) + float(v)
            names[d] = n
        acc: dict[str, dict[str, list[float]]] = {}
        for (d, c), v in disp.items():
            acc.setdefault(_short(names[d]), {}).setdefault(c, []).append(v)
        for k, cs in acc.items():
            if COPY_TAG in k or max(len(v) for v in cs.values()) < 3:   # the copy, set-up kernels
                continue
            for c, vs in cs.items():
                per.setdefault(k, {})[c] = sum(vs) / len(vs)
    lines = [f"# {title}", "", "Commands (repo root on the MI355X box, `TMPDIR=/tmp`), one counter pass each:", ""]
    for i, ctrs in enumerate(SQ_PASSES):
        lines.append(f"    timeout -s KILL 120 rocprofv3 --pmc {ctrs} -d gpurun_out/sq{i} -o p -- "
                     f"python3 -m libstrix_amd.profiling probe {workload}")
    dbargs = " ".join(f"gpurun_out/sq{i}/p_results.db" for i in range(len(SQ_PASSES)))
    lines += [f"    python3 -m libstrix_amd.profiling sq {out_md} '{title}' {workload} {dbargs}", "",
              "Averages per dispatch. busy us = SQ_BUSY_CYCLES / 32 shader engines / 2.4 GHz; MFMA busy = "
              "SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x busy cycles); VALU/MFMA and LDS/MFMA count instructions "
              "(SQ_INSTS_VALU includes the MFMAs); waits are shares of SQ_WAVE_CYCLES.", "",
              "| kernel | busy us | MFMA busy | VALU / MFMA | LDS / MFMA | LDS bank-conflict cycles / LDS inst | "
              "wait (any) | wait (LDS) | VALU+MFMA co-issue / MFMA busy |",
              "|---|---|---|---|---|---|---|---|---|"]
    for k, c in sorted(per.items(), key=lambda kv: -kv[1].get("SQ_BUSY_CYCLES", 0.0)):
        busy = c.get("SQ_BUSY_CYCLES", 0.0) / SES
        if busy <= 0:
            continue
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        mfb = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        wc = c.get("SQ_WAVE_CYCLES", 0.0) or 1.0
        lds = c.get("SQ_INSTS_LDS", 0.0)

        def r(a, b):
            return f"{a / b:.2f}" if b else "-"
        lines.append(
            f"| `{k}` | {busy / 2400:.1f} | {mfb / (SIMDS * busy):.1%} | {r(c.get('SQ_INSTS_VALU', 0.0) - mf, mf)} | "
            f"{r(lds, mf)} | {r(c.get('SQ_LDS_BANK_CONFLICT', 0.0), lds)} | "
            f"{c.get('SQ_WAIT_ANY', 0.0) / wc:.1%} | {c.get('SQ_WAIT_INST_LDS', 0.0) / wc:.1%} | "
            f"{r(c.get('SQ_VALU_MFMA_COEXEC_CYCLES', 0.0), mfb)} |")
    lines.append("")
    with open(out_md, "w") as f:
        f.write("\n".join(lines))


def _short(name: str) -> str:
    name = re.sub(r"^void ", "", name).replace("(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in name:               # drop the parameter list, keep template arguments
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    s = "".join(out)
    return s if len(s) <= 150 else s[:147] + "..."


def stats(db_path: str, out_md: str, title: str, command: str) -> None:
    db = sqlite3.connect(db_path)
    rows = db.execute("select name, duration from kernels").fetchall()
    agg: dict[str, list[float]] = {}
    for name, dur in rows:
        agg.setdefault(_short(name), []).append(dur / 1e3)
    total = sum(sum(v) for v in agg.values()) or 1.0
    lines = [f"# {title}", "", "Command (repo root on the MI355X box):", "", f"    {command}", "",
             "Per-kernel durations from the kernel trace (`kernels` view of the rocprofv3 database):", "",
             "| kernel | calls | avg us | min us | max us | share |", "|---|---|---|---|---|---|"]
    for name, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{name}` | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                     f"{100 * sum(v) / total:.1f} % |")
    lines.append("")
    with open(out_md, "w") as f:
        f.write("\n".join(lines))


def main(argv: list[str]) -> None:
    if not argv:
        raise SystemExit(__doc__)
    if argv[0] == "probe" and len(argv) <= 2:
        probe(*argv[1:])
    elif argv[0] == "traffic" and len(argv) in (4, 5):
        print(json.dumps(traffic(*argv[1:])))
    elif argv[0] == "sq" and len(argv) >= 5:
        sq(*argv[1:])
    elif argv[0] == "stats" and len(argv) == 5:
        stats(*argv[1:])
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
