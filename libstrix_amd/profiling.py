# SPDX-License-Identifier: MIT
"""Measurement helpers behind the `roofline` fields of bench.py's JSON line.

    python -m libstrix_amd.profiling probe
        Launches, on the current stream, a plain copy kernel of known size
        (torch's bitwise_not over 1 GiB of int32: 1 GiB read, 1 GiB written,
        four times the 256 MB Infinity Cache) and then the config-2 headline
        GEMM (FP8-block W8A8, M=4096 N=17408 K=5120), three times each. Meant
        to run under `rocprofv3 --pmc FETCH_SIZE` and again under
        `rocprofv3 --pmc WRITE_SIZE`, one counter pass per run.

    python -m libstrix_amd.profiling traffic FETCH_DB WRITE_DB OUT_PREFIX
        Reads the two rocprofv3 databases, scales each GEMM dispatch's
        FETCH_SIZE / WRITE_SIZE (KiB per dispatch) by what the same counter
        reads for the copy kernel of known size, and writes OUT_PREFIX.json
        (read by bench.py: `bytes_per_launch` becomes roofline.traffic) and
        OUT_PREFIX.md (the figures and the commands).

    python -m libstrix_amd.profiling stats DB OUT_MD TITLE COMMAND
        Per-kernel calls / average / minimum / share of a
        `rocprofv3 --kernel-trace --stats` database as a markdown table.

The counters count L2 (TCC) traffic to the memory fabric, so bytes served by
the Infinity Cache count as traffic too: the figure is what the kernel asks
of the fabric beyond L2, the quantity that re-reads inflate.
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


def probe() -> None:
    import torch

    import libstrix_amd
    from libstrix_amd import workloads

    if not libstrix_amd.library_available():
        raise SystemExit("libstrix_amd/_strix_amd.so is not built")
    S = torch.ops.strix
    src = torch.randint(-2**31, 2**31 - 1, (COPY_ELEMS,), dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    d = workloads.c2_fp8(seed=2, device="cuda", **HEADLINE)
    q, s = S.fp8_quant_group128(d["x"])
    torch.cuda.synchronize()
    for i in range(3):
        torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        print(f"probe: copy {i} done", flush=True)
    for i in range(3):
        S.fp8_w8a8_block_gemm(q, s, d["w"], d["sw"])
        torch.cuda.synchronize()
        print(f"probe: headline gemm {i} done", flush=True)


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


def traffic(fetch_db: str, write_db: str, out_prefix: str) -> dict:
    """One op call of the headline GEMM may launch more than one kernel (the
    256x256 rounds and a 128x128 strip for the leftover columns): per kernel
    the median over calls is taken, and a launch's traffic is their sum."""
    fr = _counter_rows(fetch_db, "FETCH_SIZE")
    wr = _counter_rows(write_db, "WRITE_SIZE")
    cf = [v for vs in _pick(fr, COPY_TAG).values() for v in vs]
    cw = [v for vs in _pick(wr, COPY_TAG).values() for v in vs]
    gf, gw = _pick(fr, GEMM_TAG), _pick(wr, GEMM_TAG)
    if not (cf and cw and gf and gw) or set(gf) != set(gw):
        raise SystemExit(f"missing dispatches: copy {len(cf)}/{len(cw)}, gemm kernels {sorted(gf)} / {sorted(gw)}")
    copy_kib = COPY_BYTES / 1024.0
    f_factor = copy_kib / _med(cf)
    w_factor = copy_kib / _med(cw)
    per_kernel = {name: {"fetch_kib": round(_med(gf[name]), 1), "write_kib": round(_med(gw[name]), 1),
                         "fetch_bytes": int(round(_med(gf[name]) * 1024.0 * f_factor)),
                         "write_bytes": int(round(_med(gw[name]) * 1024.0 * w_factor)), "calls": len(gf[name])}
                  for name in sorted(gf)}
    fetch_b = sum(k["fetch_bytes"] for k in per_kernel.values())
    write_b = sum(k["write_bytes"] for k in per_kernel.values())
    alg = headline_algorithmic_bytes(**HEADLINE)
    res = {
        "kernel": "tiled8_kernel<fp8 block> launches of one config-2 GEMM call (M=4096 N=17408 K=5120)",
        "bytes_per_launch": fetch_b + write_b,
        "fetch_bytes_per_launch": fetch_b,
        "write_bytes_per_launch": write_b,
        "algorithmic_bytes_per_launch": alg,
        "traffic_over_algorithmic": round((fetch_b + write_b) / alg, 3),
        "per_kernel": per_kernel,
        "copy_known_bytes": COPY_BYTES,
        "copy_fetch_kib_raw": [round(v, 1) for v in cf],
        "copy_write_kib_raw": [round(v, 1) for v in cw],
        "fetch_scale": round(f_factor, 4),
        "write_scale": round(w_factor, 4),
    }
    with open(out_prefix + ".json", "w") as f:
        json.dump(res, f, indent=1)
    cmd_f = ("timeout -s KILL 150 rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_fetch -o p -- "
             "python3 -m libstrix_amd.profiling probe")
    cmd_w = cmd_f.replace("FETCH_SIZE", "WRITE_SIZE").replace("pmc_fetch", "pmc_write")
    md = [
        "# HBM-side traffic of the config-2 headline GEMM (FP8-block W8A8, M=4096 N=17408 K=5120)",
        "",
        "Commands (repo root on the MI355X box, `TMPDIR=/tmp`):",
        "",
        f"    {cmd_f}",
        f"    {cmd_w}",
        "    python3 -m libstrix_amd.profiling traffic gpurun_out/pmc_fetch/p_results.db "
        "gpurun_out/pmc_write/p_results.db profiles/fp8_w8a8_block_gemm_m4096_traffic",
        "",
        "Calibration: torch `bitwise_not` over 1 GiB of int32 (1 GiB read + 1 GiB written).",
        "",
        "| quantity | value |",
        "|---|---|",
        f"| copy FETCH_SIZE (KiB, median of {len(cf)}) | {_med(cf):.0f} (known {copy_kib:.0f}) -> scale {f_factor:.4f} |",
        f"| copy WRITE_SIZE (KiB, median of {len(cw)}) | {_med(cw):.0f} (known {copy_kib:.0f}) -> scale {w_factor:.4f} |",
    ]
    for name, k in per_kernel.items():
        md.append(f"| `{name}` FETCH_SIZE / WRITE_SIZE (KiB, median of {k['calls']}) | {k['fetch_kib']:.0f} / "
                  f"{k['write_kib']:.0f} -> {k['fetch_bytes'] / 1e6:.1f} / {k['write_bytes'] / 1e6:.1f} MB |")
    md += [
        f"| traffic per GEMM call | {(fetch_b + write_b) / 1e6:.1f} MB (fetch {fetch_b / 1e6:.1f}, write {write_b / 1e6:.1f}) |",
        f"| algorithmic bytes per GEMM call | {alg / 1e6:.1f} MB |",
        f"| traffic / algorithmic | {(fetch_b + write_b) / alg:.3f} |",
        "",
    ]
    with open(out_prefix + ".md", "w") as f:
        f.write("\n".join(md))
    return res


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
    if argv[0] == "probe":
        probe()
    elif argv[0] == "traffic" and len(argv) == 4:
        print(json.dumps(traffic(*argv[1:])))
    elif argv[0] == "stats" and len(argv) == 5:
        stats(*argv[1:])
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
