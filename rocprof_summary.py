"""Summaries of rocprofv3 output for the MoE block kernels.

    python rocprof_summary.py stats <kernel_trace.csv> [--title TEXT] [--command CMD]
        Markdown table of per-kernel launch counts and durations (from the
        start/end timestamps of a --kernel-trace run), one row per kernel
        and grid shape.

    python rocprof_summary.py traffic --fetch F.csv --write W.csv
            --copy-fetch CF.csv --copy-write CW.csv --copy-bytes N --config NAME
            [--out profiles/traffic.json]
        HBM bytes per forward of each block kernel from two --pmc runs
        (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by the
        factor that makes the same counter read N bytes for a plain device
        copy of N bytes (bench.py --copy-mb).  Merged into the JSON file
        under "<kernel>@<config>", which bench.py reports as roofline.traffic.
"""
import argparse
import collections
import csv
import json
import os

# rocprofv3 kernel name (demangled, without arguments) -> block kernel name
# used by the library's per-kernel timer (tie_hip_profile_read)
_NAMES = (
    ("tie::exact_gu_kernel", "exact_gate_up"),
    ("tie::exact_gu_bf16_kernel", "exact_gate_up"),
    ("tie::exact_down_kernel", "exact_down"),
    ("tie::exact_down_bf16_kernel", "exact_down"),
    ("tie::router_small_kernel", "router"),
    ("tie::router_mid_kernel", "router"),
    ("tie::router_logits_kernel", "router"),
    ("tie::router_topk_kernel", "router"),
    ("tie::router_topk_wave_kernel", "router"),
    ("tie::route_group_kernel", "route_group"),
    ("tie::dispatch_kernel", "dispatch"),
    ("tie::combine_kernel", "combine"),
    ("tie::combine16_kernel", "combine"),
    ("tie::rmsnorm_kernel", "rmsnorm"),
    ("tie::route_bucket_kernel", "router"),
    ("tie::bucket_plan_kernel", "dispatch"),
    ("tie::decode_gu_kernel", "decode_gate_up"),
    ("tie::decode_down_kernel", "decode_down"),
    ("tie::decode_one_kernel", "decode_one"),
    ("tie::recompute_kernel", "recompute"),
    ("tie::combine_fix_kernel", "combine"),
    ("tie::dense_rows_kernel", "dense"),
    ("tie::dense_groups_kernel", "dense"),
    ("tie::dense_stream_kernel", "dense"),
    ("tie::dense_prep_kernel", "dense_mfma"),
    ("tie::dense_fix_kernel", "dense_mfma"),
)


def block_kernel(name):
    """Block kernel a rocprof kernel name belongs to (None: set-up or foreign)."""
    base = name.replace("void ", "").split("(")[0]
    if base.startswith("tie::mfma_experts_kernel"):
        # template arguments <type, down, tile rows>
        args = base[base.index("<") + 1:base.rindex(">")].split(",")
        return "mfma_down" if args[1].strip() == "true" else "mfma_gate_up"
    for prefix, block in _NAMES:
        if base == prefix or base.startswith(prefix + "<"):
            return block
    return None


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def stats(trace_csv):
    agg = collections.OrderedDict()
    for r in _rows(trace_csv):
        name = r["Kernel_Name"].replace("void ", "").split("(")[0]
        if not name.startswith("tie::"):
            continue
        key = (name, r.get("Grid_Size_X", ""), r.get("Grid_Size_Y", ""), r.get("Grid_Size_Z", ""),
               r.get("Workgroup_Size_X", ""))
        agg.setdefault(key, []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return agg


def stats_markdown(trace_csv, title=None, command=None):
    out = []
    if title:
        out.append("# " + title)
        out.append("")
    if command:
        out.append("Command: `%s`" % command)
        out.append("")
    out.append("| kernel | grid (threads) x,y,z | workgroup | launches | avg us | median us | min us |")
    out.append("|---|---|---|---|---|---|---|")
    for (name, gx, gy, gz, wg), v in stats(trace_csv).items():
        v = sorted(v)
        out.append("| %s | %s,%s,%s | %s | %d | %.2f | %.2f | %.2f |" % (
            name, gx, gy, gz, wg, len(v), sum(v) / len(v) / 1e3, v[len(v) // 2] / 1e3, v[0] / 1e3))
    return "\n".join(out) + "\n"


def _per_dispatch(path, counter):
    """{block kernel: [KiB per dispatch]} for one counter of a --pmc run."""
    res = collections.defaultdict(list)
    for r in _rows(path):
        if r["Counter_Name"] != counter:
            continue
        block = block_kernel(r["Kernel_Name"])
        if block is None and r["Kernel_Name"].find("copy") < 0:
            continue
        res[block or "copy"].append(float(r["Counter_Value"]))
    return res


def traffic(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, copy_bytes):
    cf = _per_dispatch(copy_fetch_csv, "FETCH_SIZE")["copy"]
    cw = _per_dispatch(copy_write_csv, "WRITE_SIZE")["copy"]
    # the largest copy dispatch is the timed copy (others are set-up fills)
    f_scale = copy_bytes / (max(cf) * 1024.0)
    w_scale = copy_bytes / (max(cw) * 1024.0)
    fetch = _per_dispatch(fetch_csv, "FETCH_SIZE")
    write = _per_dispatch(write_csv, "WRITE_SIZE")
    # one combine (or, for one token, decode_one / decode_down) dispatch per forward:
    # bytes per forward of a block kernel (some blocks are two kernels,
    # e.g. router logits + selection)
    steps = len(fetch.get("combine") or fetch.get("decode_one") or fetch.get("decode_down") or [])
    if not steps:
        raise ValueError("no combine / decode_one / decode_down dispatches: cannot count forwards")
    res = {}
    for block in fetch:
        if block == "copy" or block not in write:
            continue
        fb = sum(fetch[block]) / steps * 1024.0 * f_scale
        wb = sum(write[block]) / steps * 1024.0 * w_scale
        res[block] = {"bytes": round(fb + wb), "fetch_bytes": round(fb), "write_bytes": round(wb),
                      "dispatches": len(fetch[block]), "forwards": steps}
    return res, {"fetch_scale": f_scale, "write_scale": w_scale}


_DEFAULT_JSON = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


def traffic_markdown(path):
    with open(path) as f:
        t = json.load(f)
    out = ["Kernels are grouped as the library's per-kernel timer groups them: on the matrix-core path router is the "
           "logits kernel plus route_bucket (selection, per-expert selection bytes, and x converted to the gate/up A "
           "operand), dispatch is bucket_plan (per-expert pair lists); decode_one is the whole one-token block; "
           "dense includes its grouping kernel.",
           "",
           "| kernel @ config | fetch MB | write MB | total MB per forward | dispatches | forwards |",
           "|---|---|---|---|---|---|"]
    for k, v in sorted(t["detail"].items(), key=lambda kv: (kv[0].split("@")[1], kv[0])):
        out.append("| %s | %.2f | %.2f | %.2f | %d | %d |" % (k, v["fetch_bytes"] / 1e6, v["write_bytes"] / 1e6,
                                                             v["bytes"] / 1e6, v["dispatches"], v.get("forwards", 0)))
    out.append("")
    out.append("Scale factors (copy bytes / counter bytes): FETCH_SIZE x %.4f, WRITE_SIZE x %.4f." % (
        t["scales"]["fetch_scale"], t["scales"]["write_scale"]))
    return "\n".join(out) + "\n"


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("trace")
    s.add_argument("--title")
    s.add_argument("--command")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--copy-fetch", required=True)
    t.add_argument("--copy-write", required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--config", required=True)
    t.add_argument("--out", default=_DEFAULT_JSON)
    m = sub.add_parser("traffic-md")
    m.add_argument("--json", default=_DEFAULT_JSON)
    a = ap.parse_args()
    if a.cmd == "stats":
        print(stats_markdown(a.trace, a.title, a.command), end="")
        return
    if a.cmd == "traffic-md":
        print(traffic_markdown(a.json), end="")
        return
    res, scales = traffic(a.fetch, a.write, a.copy_fetch, a.copy_write, a.copy_bytes)
    data = {}
    if os.path.exists(a.out):
        with open(a.out) as f:
            data = json.load(f)
    for block, v in res.items():
        data["%s@%s" % (block, a.config)] = v["bytes"]
        data["detail"] = data.get("detail", {})
        data["detail"]["%s@%s" % (block, a.config)] = v
    data["scales"] = scales
    with open(a.out, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
