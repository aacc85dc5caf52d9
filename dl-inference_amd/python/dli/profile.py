"""Reads dli.profile.v1 documents written by dli.ProfileSession (write_json / to_json).

    python -m dli.profile summarize PROFILE.json [--group-by node|op] [--skip-runs N]
    python -m dli.profile compare BEFORE.json AFTER.json [--force]
    python -m dli.profile export PROFILE.json --format csv|json [-o OUT]
    python -m dli.profile trace PROFILE.json -o TRACE.json

The command set, grouping, nearest-rank percentiles and the rule that CPU and GPU times are
never added follow the reference's design (.codex/profiling_design.md, "Analyzer Utility").
Standard library only; the JSON document is the contract, the native runtime is not imported.
"""
from __future__ import annotations

import argparse
import csv
import io
import json
import math
import sys
from collections import OrderedDict

SCHEMA = "dli.profile.v1"
_REQUIRED_EVENT = ("event_id", "run_id", "node_index", "node_name", "op_type", "cpu_start_ns",
                   "cpu_duration_ns", "gpu_duration_ns", "status")
_REQUIRED_RUN = ("run_id", "start_ns", "duration_ns", "status")


class ProfileError(ValueError):
    pass


def load(source) -> dict:
    """Parses and validates a profile (a path, a JSON string or an already parsed dict)."""
    if isinstance(source, dict):
        doc = source
    else:
        text = source if isinstance(source, str) and source.lstrip().startswith("{") else None
        if text is None:
            with open(source) as f:
                text = f.read()
        doc = json.loads(text)
    schema = doc.get("schema")
    if not isinstance(schema, str) or schema.split(".")[:2] != ["dli", "profile"]:
        raise ProfileError(f"not a dli.profile document (schema {schema!r})")
    if schema.split(".")[2:3] != ["v1"]:
        raise ProfileError(f"unsupported major version: {schema}")
    for key in ("metadata", "runs", "events"):
        if key not in doc:
            raise ProfileError(f"missing field {key!r}")
    for r in doc["runs"]:
        for k in _REQUIRED_RUN:
            if k not in r:
                raise ProfileError(f"run without {k!r}")
    for e in doc["events"]:
        for k in _REQUIRED_EVENT:
            if k not in e:
                raise ProfileError(f"event without {k!r}")
    return doc


def nearest_rank(values, q: float):
    """Nearest-rank percentile q in (0, 100] of a non-empty sequence."""
    vals = sorted(values)
    if not vals:
        return None
    rank = max(1, math.ceil(q / 100.0 * len(vals)))
    return vals[rank - 1]


def _stats(values):
    if not values:
        return None
    return {"n": len(values), "total": sum(values), "mean": sum(values) / len(values),
            "p50": nearest_rank(values, 50), "p95": nearest_rank(values, 95), "max": max(values)}


def _peer_events(doc, skip_runs=0):
    """Graph-operator events of the runs kept (nested ranges, if any, are excluded)."""
    run_ids = sorted({r["run_id"] for r in doc["runs"]})
    kept = set(run_ids[skip_runs:])
    return [e for e in doc["events"]
            if e.get("category", "graph_operator") == "graph_operator" and e["run_id"] in kept]


def summarize(doc, group_by: str = "node", skip_runs: int = 0) -> dict:
    """Per group (node: (node_name, op_type); op: op_type): call count, CPU and GPU stats and
    shares of the peer totals, plus run wall times and status counts."""
    doc = load(doc)
    events = _peer_events(doc, skip_runs)
    groups: "OrderedDict[tuple, dict]" = OrderedDict()
    for e in events:
        key = (e["node_name"], e["op_type"]) if group_by == "node" else (e["op_type"],)
        g = groups.setdefault(key, {"calls": 0, "cpu": [], "gpu": [], "failed": 0,
                                    "gpu_unmeasured": 0})
        g["calls"] += 1
        if e["status"] != "ok":
            g["failed"] += 1
        g["cpu"].append(e["cpu_duration_ns"])
        if e["gpu_duration_ns"] is None:
            g["gpu_unmeasured"] += 1
        else:
            g["gpu"].append(e["gpu_duration_ns"])
    cpu_total = sum(sum(g["cpu"]) for g in groups.values())
    gpu_total = sum(sum(g["gpu"]) for g in groups.values())
    rows = []
    for key, g in groups.items():
        cs, gs = _stats(g["cpu"]), _stats(g["gpu"])
        rows.append({"key": list(key), "calls": g["calls"], "failed": g["failed"],
                     "gpu_unmeasured": g["gpu_unmeasured"], "cpu": cs, "gpu": gs,
                     "cpu_pct": 100.0 * cs["total"] / cpu_total if cs and cpu_total else 0.0,
                     "gpu_pct": 100.0 * gs["total"] / gpu_total if gs and gpu_total else 0.0})
    sort_gpu = gpu_total > 0
    rows.sort(key=lambda r: -((r["gpu"] or {}).get("total", 0) if sort_gpu
                              else (r["cpu"] or {}).get("total", 0)))
    run_ids = sorted({r["run_id"] for r in doc["runs"]})[skip_runs:]
    walls = [r["duration_ns"] for r in doc["runs"] if r["run_id"] in set(run_ids)]
    return {"group_by": group_by, "rows": rows, "cpu_total_ns": cpu_total,
            "gpu_total_ns": gpu_total, "runs": len(run_ids), "run_wall": _stats(walls),
            "dropped_events": doc["metadata"].get("dropped_events", 0),
            "failed": sum(r["failed"] for r in rows),
            "gpu_unmeasured": sum(r["gpu_unmeasured"] for r in rows)}


def _us(ns):
    return "-" if ns is None else f"{ns / 1000.0:.1f}"


def format_summary(s: dict) -> str:
    out = [f"runs: {s['runs']}  (percentiles: nearest rank)  CPU = submit time inside "
           f"Operator::compute, GPU = device time between the node's events; never added"]
    if s["run_wall"]:
        w = s["run_wall"]
        out.append(f"run wall: mean {_us(w['mean'])} us  p50 {_us(w['p50'])}  p95 {_us(w['p95'])}")
    if s["runs"] < 3:
        out.append("warning: fewer than 3 runs; percentiles are rough")
    out.append(f"{'group':44s} {'calls':>6s} {'CPU total':>10s} {'CPU p50':>8s} {'CPU%':>6s} "
               f"{'GPU total':>10s} {'GPU p50':>8s} {'GPU p95':>8s} {'GPU%':>6s}  (us)")
    for r in s["rows"]:
        name = " / ".join(r["key"])
        name = name if len(name) <= 44 else name[:41] + "..."
        c, g = r["cpu"] or {}, r["gpu"] or {}
        out.append(f"{name:44s} {r['calls']:6d} {_us(c.get('total')):>10s} {_us(c.get('p50')):>8s} "
                   f"{r['cpu_pct']:6.1f} {_us(g.get('total')):>10s} {_us(g.get('p50')):>8s} "
                   f"{_us(g.get('p95')):>8s} {r['gpu_pct']:6.1f}")
    out.append(f"unmeasured GPU: {s['gpu_unmeasured']}  failed: {s['failed']}  "
               f"dropped: {s['dropped_events']}")
    return "\n".join(out)


def compare(before, after, force: bool = False) -> dict:
    """Joins (node_name, op_type) rows and reports the change of median CPU and GPU time.
    Refuses (ProfileError) when the runs are not comparable: different devices or shape
    signatures, or a sample count that differs by more than 2x, unless force."""
    a, b = load(before), load(after)
    if not force:
        dev_a = sorted({e.get("device") for e in a["events"]})
        dev_b = sorted({e.get("device") for e in b["events"]})
        if dev_a != dev_b:
            raise ProfileError(f"device sets differ ({dev_a} vs {dev_b}); use force")
        sh_a = {(e["node_name"], e.get("shapes")) for e in a["events"] if e.get("shapes")}
        sh_b = {(e["node_name"], e.get("shapes")) for e in b["events"] if e.get("shapes")}
        if sh_a and sh_b and sh_a != sh_b:
            raise ProfileError("shape signatures differ; use force")
        na, nb = len(a["events"]), len(b["events"])
        if min(na, nb) == 0 or max(na, nb) > 2 * min(na, nb):
            raise ProfileError(f"sample counts not comparable ({na} vs {nb}); use force")
    sa = {tuple(r["key"]): r for r in summarize(a)["rows"]}
    sb = {tuple(r["key"]): r for r in summarize(b)["rows"]}
    rows = []
    for key in list(sa) + [k for k in sb if k not in sa]:
        ra, rb = sa.get(key), sb.get(key)
        row = {"key": list(key), "status": "both" if ra and rb else ("removed" if ra else "added")}
        for kind in ("cpu", "gpu"):
            va = (ra or {}).get(kind) and ra[kind]["p50"]
            vb = (rb or {}).get(kind) and rb[kind]["p50"]
            row[f"{kind}_p50_before"], row[f"{kind}_p50_after"] = va, vb
            row[f"{kind}_change_ns"] = vb - va if va is not None and vb is not None else None
            row[f"{kind}_change_pct"] = (100.0 * (vb - va) / va
                                         if va and vb is not None else None)
        rows.append(row)
    return {"rows": rows}


def export(doc, fmt: str = "csv") -> str:
    doc = load(doc)
    if fmt == "json":
        return json.dumps(doc, indent=1)
    buf = io.StringIO()
    cols = ["event_id", "run_id", "node_index", "node_name", "op_type", "cpu_start_ns",
            "cpu_duration_ns", "gpu_duration_ns", "device", "stream", "status", "shapes"]
    w = csv.writer(buf)
    w.writerow(cols)
    for e in doc["events"]:
        w.writerow(["" if e.get(c) is None else e.get(c) for c in cols])
    return buf.getvalue()


def trace(doc) -> dict:
    """Chrome Trace Event Format (Perfetto). CPU spans at their host timestamps on one track
    per host thread; GPU spans on one track per (device, stream), laid end to end in event order
    starting with each run's first CPU start: their durations are exact, their host alignment
    approximate (said in the metadata)."""
    doc = load(doc)
    events = []
    pid = doc["metadata"].get("process_id", 0)
    gpu_cursor = {}
    for e in sorted(doc["events"], key=lambda e: e["event_id"]):
        args = {"run_id": e["run_id"], "node_index": e["node_index"], "status": e["status"]}
        events.append({"name": e["node_name"], "cat": f"cpu,{e['op_type']}", "ph": "X",
                       "pid": pid, "tid": str(e.get("host_thread_id", 0)),
                       "ts": e["cpu_start_ns"] / 1000.0, "dur": e["cpu_duration_ns"] / 1000.0,
                       "args": args})
        if e["gpu_duration_ns"] is not None:
            track = f"gpu {e.get('device')} stream {e.get('stream')}"
            start = max(gpu_cursor.get(track, 0.0), e["cpu_start_ns"] / 1000.0)
            events.append({"name": e["node_name"], "cat": f"gpu,{e['op_type']}", "ph": "X",
                           "pid": pid, "tid": track, "ts": start,
                           "dur": e["gpu_duration_ns"] / 1000.0, "args": args})
            gpu_cursor[track] = start + e["gpu_duration_ns"] / 1000.0
    return {"traceEvents": events, "displayTimeUnit": "ns",
            "metadata": {"source": SCHEMA, "gpu_alignment": "approximate (durations exact)"}}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m dli.profile")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("summarize")
    s.add_argument("profile")
    s.add_argument("--group-by", choices=("node", "op"), default="node")
    s.add_argument("--skip-runs", type=int, default=0)
    c = sub.add_parser("compare")
    c.add_argument("before")
    c.add_argument("after")
    c.add_argument("--force", action="store_true")
    x = sub.add_parser("export")
    x.add_argument("profile")
    x.add_argument("--format", choices=("csv", "json"), default="csv")
    x.add_argument("-o", "--output")
    t = sub.add_parser("trace")
    t.add_argument("profile")
    t.add_argument("-o", "--output", required=True)
    args = ap.parse_args(argv)
    try:
        if args.cmd == "summarize":
            print(format_summary(summarize(args.profile, args.group_by, args.skip_runs)))
        elif args.cmd == "compare":
            res = compare(args.before, args.after, args.force)
            print(f"{'group':44s} {'status':8s} {'CPU p50 change':>16s} {'GPU p50 change':>16s}")
            for r in res["rows"]:
                def fmt(kind):
                    v, p = r[f"{kind}_change_ns"], r[f"{kind}_change_pct"]
                    return "-" if v is None else f"{v / 1000.0:+.1f}us" + (
                        "" if p is None else f" ({p:+.0f}%)")
                print(f"{' / '.join(r['key'])[:44]:44s} {r['status']:8s} {fmt('cpu'):>16s} "
                      f"{fmt('gpu'):>16s}")
        elif args.cmd == "export":
            text = export(args.profile, args.format)
            if args.output:
                with open(args.output, "w") as f:
                    f.write(text)
            else:
                sys.stdout.write(text)
        else:
            with open(args.output, "w") as f:
                json.dump(trace(args.profile), f)
    except ProfileError as err:
        print(f"error: {err}", file=sys.stderr)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main())
