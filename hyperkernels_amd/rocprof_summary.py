"""Summaries of rocprofv3 CSV output for the kernels of this library.

Usage (after `rocprofv3 ... --output-format csv -d DIR -- python3 bench.py ...`):

    python -m hyperkernels_amd.rocprof_summary stats DIR
        per-kernel dispatch count, average / min / max duration from *_kernel_stats.csv
    python -m hyperkernels_amd.rocprof_summary traffic FETCH_DIR WRITE_DIR COPY_FETCH_DIR \
        COPY_WRITE_DIR COPY_BYTES
        per-kernel HBM traffic per dispatch from FETCH_SIZE / WRITE_SIZE runs (KiB per dispatch),
        each scaled by the factor that makes the same counter read COPY_BYTES for a plain copy
        kernel (torch's elementwise `mul(src, 1, out=dst)` over COPY_BYTES of float32): the
        configs[1] step kernels by name, then every kernel symbol of the runs.

    python -m hyperkernels_amd.rocprof_summary pmc FILTER DIR [DIR ...]
        per kernel whose symbol contains FILTER: dispatches, mean duration and mean value per
        dispatch of every counter found in the `--pmc` runs DIR..., plus derived figures:
          clock_ghz  = GRBM_GUI_ACTIVE / Num_Xcc / duration (GRBM_GUI_ACTIVE is summed over
                       the XCDs; the agent's Num_Xcc and Simd_Count come from *_agent_info.csv);
          mfma_busy  = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / Num_Xcc * Simd_Count), the
                       fraction of SIMD cycles in which the matrix core is busy;
          lds_conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.

The traffic lines (`traffic: <name> fetch_bytes=... write_bytes=... traffic_bytes=...`) are what
bench.py reads back for the `roofline.traffic` field of its dominant kernel.
"""
from __future__ import annotations

import csv
import pathlib
import sys
from collections import defaultdict

# bench.py's step names -> a substring of the kernel symbol rocprofv3 reports
STEP_KERNELS = {
    "gelu_fwd_bf16": "gelu_fwd_vec",
    "gelu_bwd_bf16": "gelu_bwd_vec",
    "ce_fwd": "ce_forward",
    "ce_bwd": "ce_backward",
    "adamw_148": "adam_plan_kernel",
}
COPY_KERNEL = "MulFunctor"


def _csvs(d, suffix):
    files = sorted(pathlib.Path(d).rglob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    return rows


def _short(name, width=90):
    """Kernel symbol without its parameter list and leading `void`."""
    if name.endswith(")"):
        depth = 0
        for i in range(len(name) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(name[i], 0)
            if depth == 0:
                name = name[:i]
                break
    name = name[5:] if name.startswith("void ") else name
    name = name.replace("(anonymous namespace)::", "")
    return name if len(name) <= width else name[:width - 3] + "..."


def kernel_stats(d):
    out = []
    for r in _csvs(d, "kernel_stats.csv"):
        out.append((r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]),
                    float(r["MaxNs"]), float(r["Percentage"])))
    return sorted(out, key=lambda t: -t[1] * t[2])


def counter_per_dispatch(d, counter):
    """Average counter value per dispatch, keyed by kernel symbol."""
    vals = defaultdict(dict)
    for r in _csvs(d, "counter_collection.csv"):
        if r["Counter_Name"] != counter:
            continue
        key = (r.get("Process_Id", ""), r["Dispatch_Id"])
        vals[r["Kernel_Name"]][key] = vals[r["Kernel_Name"]].get(key, 0.0) + float(r["Counter_Value"])
    return {k: sum(v.values()) / len(v) for k, v in vals.items()}


def _match(table, sub):
    hits = [k for k in table if sub in k]
    if not hits:
        return None
    return max(hits, key=lambda k: table[k])


def traffic(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_bytes):
    f, w = counter_per_dispatch(fetch_dir, "FETCH_SIZE"), counter_per_dispatch(write_dir, "WRITE_SIZE")
    cf = counter_per_dispatch(copy_fetch_dir, "FETCH_SIZE")
    cw = counter_per_dispatch(copy_write_dir, "WRITE_SIZE")
    ck_f, ck_w = _match(cf, COPY_KERNEL), _match(cw, COPY_KERNEL)
    if ck_f is None or ck_w is None:
        raise SystemExit("copy kernel not found in the calibration runs")
    f_scale = copy_bytes / (cf[ck_f] * 1024.0)
    w_scale = copy_bytes / (cw[ck_w] * 1024.0)
    lines = [f"copy calibration: {copy_bytes} B read and written; FETCH_SIZE reads "
             f"{cf[ck_f]:.1f} KiB -> scale {f_scale:.4f}; WRITE_SIZE reads {cw[ck_w]:.1f} KiB -> "
             f"scale {w_scale:.4f}"]
    for name, sub in STEP_KERNELS.items():
        kf, kw = _match(f, sub), _match(w, sub)
        if kf is None or kw is None:
            continue
        fb, wb = f[kf] * 1024.0 * f_scale, w[kw] * 1024.0 * w_scale
        lines.append(f"traffic: {name} fetch_bytes={fb:.0f} write_bytes={wb:.0f} "
                     f"traffic_bytes={fb + wb:.0f} raw_fetch_kib={f[kf]:.1f} raw_write_kib={w[kw]:.1f}")
    # every kernel symbol of the runs (the step kernels above again, by symbol), per dispatch
    for k in sorted(set(f) & set(w), key=lambda k: -(f[k] + w[k])):
        fb, wb = f[k] * 1024.0 * f_scale, w[k] * 1024.0 * w_scale
        lines.append(f"kernel {_short(k, 110)}: fetch_bytes={fb:.0f} write_bytes={wb:.0f} "
                     f"traffic_bytes={fb + wb:.0f}")
    return lines


def read_traffic(path):
    """{name: traffic_bytes} from a committed summary's `traffic:` lines (empty if absent)."""
    out = {}
    p = pathlib.Path(path)
    if not p.exists():
        return out
    for line in p.read_text().splitlines():
        if line.startswith("traffic: "):
            parts = line.split()
            kv = dict(x.split("=", 1) for x in parts[2:])
            out[parts[1]] = float(kv["traffic_bytes"])
    return out


def _agent(d):
    """(Num_Xcc, Simd_Count) of the GPU agent of a rocprofv3 output directory."""
    for r in _csvs(d, "agent_info.csv"):
        if r.get("Agent_Type") == "GPU":
            return int(r["Num_Xcc"]), int(r["Simd_Count"])
    raise SystemExit(f"no GPU agent in {d}")


def pmc(filt, dirs):
    """Per-kernel mean counters per dispatch over several `--pmc` runs (one counter set each)."""
    vals = defaultdict(lambda: defaultdict(list))
    durs = defaultdict(list)
    xcc, simds = _agent(dirs[0])
    for d in dirs:
        per = defaultdict(lambda: defaultdict(float))
        span = {}
        for r in _csvs(d, "counter_collection.csv"):
            if filt not in r["Kernel_Name"]:
                continue
            key = (r["Kernel_Name"], r.get("Process_Id", ""), r["Dispatch_Id"])
            per[key][r["Counter_Name"]] += float(r["Counter_Value"])
            span[key] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
        for key, cs in per.items():
            for c, v in cs.items():
                vals[key[0]][c].append(v)
            durs[key[0]].append(span[key])
    lines = []
    for name in sorted(vals, key=lambda n: -sum(durs[n]) / len(durs[n])):
        cs = {c: sum(v) / len(v) for c, v in vals[name].items()}
        dur = sum(durs[name]) / len(durs[name])
        lines.append(f"kernel {_short(name)}: dispatches/run {len(durs[name]) // len(dirs)}, "
                     f"mean duration {dur / 1e3:.1f} us")
        for c in sorted(cs):
            lines.append(f"  {c:30s} {cs[c]:18,.0f}")
        if "GRBM_GUI_ACTIVE" in cs:
            cyc = cs["GRBM_GUI_ACTIVE"] / xcc
            lines.append(f"  {'clock_ghz':30s} {cyc / dur:18.3f}")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in cs:
                lines.append(f"  {'mfma_busy':30s} "
                             f"{cs['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * simds):18.3f}")
        if cs.get("SQ_LDS_IDX_ACTIVE"):
            lines.append(f"  {'lds_conflict':30s} "
                         f"{cs.get('SQ_LDS_BANK_CONFLICT', 0.0) / cs['SQ_LDS_IDX_ACTIVE']:18.3f}")
    return lines


def main(argv):
    if argv[:1] == ["stats"]:
        print(f"{'kernel':90s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'pct':>6s}")
        for n, c, a, lo, hi, pct in kernel_stats(argv[1]):
            print(f"{_short(n):90s} {c:6d} {a / 1e3:10.2f} {lo / 1e3:10.2f} {hi / 1e3:10.2f} {pct:6.2f}")
    elif argv[:1] == ["pmc"] and len(argv) >= 3:
        print("\n".join(pmc(argv[1], argv[2:])))
    elif argv[:1] == ["traffic"]:
        print("\n".join(traffic(argv[1], argv[2], argv[3], argv[4], float(argv[5]))))
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
