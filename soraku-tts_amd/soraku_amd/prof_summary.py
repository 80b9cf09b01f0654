"""Summaries of rocprofv3 output for the decode frame.

    python -m soraku_amd.prof_summary trace OUT/tr_results.db
        per-kernel table of the decode frames in a ``--kernel-trace`` run
        (dispatches after the last prefill kernel, frames delimited by the
        trunk's ``final_norm_kernel`` or the depth step that fuses it)

    python -m soraku_amd.prof_summary prefill OUT/tr_results.db
        per-kernel table of the first batched prefill in the same run

    python -m soraku_amd.prof_summary counters FRAME_FETCH FRAME_WRITE COPY_FETCH COPY_WRITE MIB [KV ...]
        HBM bytes per frame from two ``--pmc`` runs (FETCH_SIZE, then
        WRITE_SIZE; ``*_counter_collection.csv`` under each directory) and the
        same two counters over ``bench.py --copy-probe MIB`` for calibration;
        prints a per-kernel table and the JSON block bench.py reads (with the
        rows' KV lengths KV ... at the counted frame)

A frame is one hipGraph launch of the engine: 28 trunk layers, the trunk's
final norm, then the depth steps; between two consecutive ``final_norm``
dispatches lie exactly one frame's kernels (the depth of one frame and the
trunk of the next).
"""
from __future__ import annotations

import collections
import csv
import glob
import json
import os
import re
import sqlite3
import sys


def short_name(name: str) -> str:
    n = re.sub(r"sk::\(anonymous namespace\)::", "", name)
    n = n.replace("void ", "")
    depth = 0
    for i, ch in enumerate(n):   # cut the argument list, keep template arguments
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return n[:i].strip()
    return n.strip()


PREFILL_MARKERS = ("prefill", "pf_", "gemm_nt_kernel")


def _is_frame_end(n):
    """The frame's last kernel: the trunk's final norm, or on the code-table
    path the depth step that fuses it (``depth_step_kernel<..., 4>``)."""
    return "final_norm_kernel" in n or (n.startswith("depth_step_kernel<") and n.replace(" ", "").endswith(",4>"))


def _frames(names):
    """Index ranges (a, b] of whole frames: between consecutive frame ends
    after the last prefill kernel."""
    last_pf = max((i for i, n in enumerate(names) if any(m in n for m in PREFILL_MARKERS)), default=-1)
    marks = [i for i, n in enumerate(names) if i > last_pf and _is_frame_end(n)]
    return list(zip(marks[:-1], marks[1:]))


def trace(db: str) -> str:
    con = sqlite3.connect(db)
    rows = con.execute("select name, start, end from kernels order by start").fetchall()
    rows = [r for r in rows if "rocclr" not in r[0]]
    names = [short_name(r[0]) for r in rows]
    fr = _frames(names)
    if not fr:
        raise SystemExit("no whole decode frames in the trace")
    agg = collections.OrderedDict()
    for a, b in fr:
        for i in range(a + 1, b + 1):
            s = agg.setdefault(names[i], [0, 0.0])
            s[0] += 1
            s[1] += (rows[i][2] - rows[i][1]) / 1e3
    n = len(fr)
    busy = sum(v[1] for v in agg.values()) / n
    span = (rows[fr[-1][1]][2] - rows[fr[0][1]][2]) / 1e3 / max(1, n - 1)
    out = [f"frames {n}, kernels per frame {sum(v[0] for v in agg.values()) // n}",
           f"per frame: span {span:.1f} us, kernel busy {busy:.1f} us",
           f"{'kernel':58s} {'calls/fr':>8s} {'avg us':>8s} {'us/frame':>9s}"]
    for k, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"{k[:58]:58s} {c / n:8.1f} {t / c:8.2f} {t / n:9.1f}")
    return "\n".join(out)


def prefill(db: str) -> str:
    """Per-kernel table of the first batched prefill in a ``--kernel-trace`` run
    (``pf_rope_table_kernel`` through ``pf_finish_kernel``)."""
    con = sqlite3.connect(db)
    rows = con.execute("select name, start, end from kernels order by start").fetchall()
    names = [short_name(r[0]) for r in rows]
    a = next(i for i, n in enumerate(names) if "pf_rope_table_kernel" in n)
    b = next(i for i, n in enumerate(names) if i > a and "pf_finish_kernel" in n)
    agg = collections.OrderedDict()
    for i in range(a, b + 1):
        s = agg.setdefault(names[i], [0, 0.0])
        s[0] += 1
        s[1] += (rows[i][2] - rows[i][1]) / 1e3
    out = [f"prefill span {(rows[b][2] - rows[a][1]) / 1e3:.0f} us, kernels {sum(v[1] for v in agg.values()):.0f} us",
           f"{'kernel':48s} {'calls':>6s} {'avg us':>8s} {'total us':>9s}"]
    for k, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"{k[:48]:48s} {c:6d} {t / c:8.1f} {t:9.1f}")
    return "\n".join(out)


def _csv(d: str):
    path = glob.glob(os.path.join(d, "*counter_collection.csv"))
    if len(path) != 1:
        raise SystemExit(f"expected one counter_collection.csv under {d}")
    return sorted(csv.DictReader(open(path[0])), key=lambda r: int(r["Dispatch_Id"]))


def _copy_scale(d: str, mib: int) -> tuple[float, float]:
    v = [float(r["Counter_Value"]) for r in _csv(d) if "copyBuffer" in r["Kernel_Name"]]
    if not v:
        raise SystemExit(f"no copy dispatch under {d}")
    kib = sum(v) / len(v)
    return mib * 2**20 / (kib * 1024), kib


def counters(fetch: str, write: str, cfetch: str, cwrite: str, mib: int, kv) -> str:
    fs, fk = _copy_scale(cfetch, mib)
    ws, wk = _copy_scale(cwrite, mib)
    per = []
    for d, scale in ((fetch, fs), (write, ws)):
        rows = _csv(d)
        names = [short_name(r["Kernel_Name"]) for r in rows]
        fr = _frames(names)
        if not fr:
            raise SystemExit(f"no whole decode frames under {d}")
        a, b = fr[-1]
        per.append([(names[i], float(rows[i]["Counter_Value"]) * 1024 * scale) for i in range(a + 1, b + 1)])
        totals = [sum(float(rows[i]["Counter_Value"]) for i in range(x + 1, y + 1)) * 1024 * scale / 1e6
                  for x, y in fr]
        per[-1].append(("__totals__", totals))
    rd, wr = per
    tot_r, tot_w = rd.pop()[1], wr.pop()[1]
    if [n for n, _ in rd] != [n for n, _ in wr]:
        raise SystemExit("the two passes counted different kernel sequences")
    agg = collections.OrderedDict()
    for (n, r), (_, w) in zip(rd, wr):
        s = agg.setdefault(n, [0, 0.0, 0.0])
        s[0] += 1
        s[1] += r
        s[2] += w
    out = [f"copy probe ({mib} MiB): FETCH_SIZE {fk:.0f} KiB, WRITE_SIZE {wk:.0f} KiB per copy -> "
           f"scale FETCH_SIZE x{fs:.3f}, WRITE_SIZE x{ws:.3f}",
           "whole frames counted: read MB " + ", ".join(f"{t:.1f}" for t in tot_r)
           + "; write MB " + ", ".join(f"{t:.1f}" for t in tot_w),
           "",
           "| kernel (last counted frame) | calls | HBM read MB | HBM write MB |",
           "|---|---:|---:|---:|"]
    for k, (c, r, w) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| `{k}` | {c} | {r / 1e6:.2f} | {w / 1e6:.2f} |")
    r_all, w_all = sum(v[1] for v in agg.values()), sum(v[2] for v in agg.values())
    out.append(f"| **frame total** | {len(rd)} | **{r_all / 1e6:.2f}** | **{w_all / 1e6:.2f}** |")
    out += ["", "```json", json.dumps({"read_bytes_per_frame": r_all, "write_bytes_per_frame": w_all,
                                       "fetch_scale": fs, "write_scale": ws, "kv_lens": kv}), "```"]
    return "\n".join(out)


def main(argv):
    if len(argv) >= 2 and argv[0] == "trace":
        print(trace(argv[1]))
    elif len(argv) >= 2 and argv[0] == "prefill":
        print(prefill(argv[1]))
    elif len(argv) >= 6 and argv[0] == "counters":
        print(counters(*argv[1:5], int(argv[5]), [int(k) for k in argv[6:]]))
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
