"""Operator profiling (dli.ProfileSession + Engine.run(profile=)) and the dli.profile analyzer,
after the reference's .codex/profiling_design.md (validation plan items 1-5: CPU spans,
disabled path, schema round trip, aggregation on fixed durations, limits and errors)."""
from __future__ import annotations

import csv
import io
import json

import pytest
import torch

import dli
from dli import profile as prof


def _graph(nodes):
    return dli.Graph.from_json(json.dumps({
        "format": "dli.graph.v1", "model_type": "profile_test", "inputs": ["x"],
        "outputs": [nodes[-1]["outputs"][0]], "nodes": nodes}))


RELU_NEG = [
    {"name": "relu", "op": "aten", "inputs": ["x"], "outputs": ["y"], "attrs": {"name": "aten::relu"}},
    {"name": "neg", "op": "aten", "inputs": ["y"], "outputs": ["z"], "attrs": {"name": "aten::neg"}},
]


def test_cpu_spans_runs_and_schema_round_trip(tmp_path):
    e, g = dli.Engine(), _graph(RELU_NEG)
    p = dli.ProfileSession(record_shapes=True)
    x = torch.randn(3, 4)
    for _ in range(3):
        out = e.run(g, {"x": x}, profile=p)["z"]
        assert torch.equal(out, -torch.relu(x))  # profiling does not change results
    p.finalize()
    assert p.finalized
    path = tmp_path / "p.json"
    p.write_json(str(path))
    doc = prof.load(str(path))
    assert doc == json.loads(p.to_json())
    assert doc["schema"] == "dli.profile.v1"
    assert [r["run_id"] for r in doc["runs"]] == [0, 1, 2]
    assert all(r["status"] == "ok" and r["duration_ns"] > 0 for r in doc["runs"])
    ev = doc["events"]
    assert [(x["run_id"], x["node_index"], x["node_name"], x["op_type"]) for x in ev] == [
        (r, i, n, "aten") for r in range(3) for i, n in enumerate(("relu", "neg"))]
    assert [x["event_id"] for x in ev] == list(range(6))
    for x in ev:
        assert x["cpu_duration_ns"] > 0 and x["gpu_duration_ns"] is None
        assert x["device"] == -1 and x["status"] == "ok"
        assert x["shapes"] == "in:[float32 cpu [3,4]] -> out:[float32 cpu [3,4]]"
    # a node starts after the previous one ended, and inside its run
    for a, b in zip(ev, ev[1:]):
        if a["run_id"] == b["run_id"]:
            assert b["cpu_start_ns"] >= a["cpu_start_ns"] + a["cpu_duration_ns"]
    for x in ev:
        run = doc["runs"][x["run_id"]]
        assert run["start_ns"] <= x["cpu_start_ns"]
        assert x["cpu_start_ns"] + x["cpu_duration_ns"] <= run["start_ns"] + run["duration_ns"]


def test_unprofiled_run_is_unchanged():
    e, g = dli.Engine(), _graph(RELU_NEG)
    x = torch.randn(5)
    assert torch.equal(e.run(g, {"x": x})["z"], e.run(g, {"x": x}, profile=None)["z"])


def test_failing_node_is_recorded_and_the_error_propagates():
    e = dli.Engine()
    g = _graph([RELU_NEG[0], {"name": "bad", "op": "aten", "inputs": ["y"], "outputs": ["z"],
                              "attrs": {"name": "aten::no_such_operator"}}])
    p = dli.ProfileSession()
    with pytest.raises(Exception):
        e.run(g, {"x": torch.randn(2)}, profile=p)
    p.finalize()
    doc = json.loads(p.to_json())
    assert doc["runs"][0]["status"] == "error"
    assert [x["status"] for x in doc["events"]] == ["ok", "error"]


def test_event_limit_drops_and_counts():
    e, g = dli.Engine(), _graph(RELU_NEG)
    p = dli.ProfileSession(max_events=3)
    for _ in range(3):
        e.run(g, {"x": torch.randn(2)}, profile=p)
    p.finalize()
    doc = json.loads(p.to_json())
    assert len(doc["events"]) == 3 and doc["metadata"]["dropped_events"] == 3


def test_lifecycle_errors():
    e, g = dli.Engine(), _graph(RELU_NEG)
    p = dli.ProfileSession()
    e.run(g, {"x": torch.randn(2)}, profile=p)
    with pytest.raises(Exception):
        p.to_json()  # before finalize
    p.finalize()
    p.finalize()  # harmless
    with pytest.raises(Exception):
        e.run(g, {"x": torch.randn(2)}, profile=p)  # after finalize


# ---- analyzer on fixed durations ---------------------------------------------------------

def _fixture(gpu=(10, 20, 30, 40), cpu=(1, 2, 3, 4), device=0, shapes=None):
    runs = [{"run_id": r, "start_ns": 1000 * r, "duration_ns": 500 + r, "status": "ok"}
            for r in range(4)]
    events = []
    for r in range(4):
        for i, (name, op) in enumerate((("a", "linear"), ("b", "linear"), ("c", "attention"))):
            k = len(events)
            events.append({"event_id": k, "run_id": r, "parent_id": None,
                           "category": "graph_operator", "node_index": i, "node_name": name,
                           "op_type": op, "host_thread_id": 1,
                           "cpu_start_ns": 1000 * r + 10 * i, "cpu_duration_ns": cpu[r] * (i + 1),
                           "gpu_duration_ns": None if name == "c" and r == 0 else gpu[r] * (i + 1),
                           "device": device, "stream": "0x0", "status": "ok",
                           **({"shapes": shapes} if shapes else {})})
    return {"schema": "dli.profile.v1", "clock": "steady_clock",
            "metadata": {"dropped_events": 0}, "runs": runs, "events": events}


def test_nearest_rank():
    assert prof.nearest_rank([5, 1, 4, 2, 3], 50) == 3
    assert prof.nearest_rank([10, 20, 30, 40], 50) == 20
    assert prof.nearest_rank([10, 20, 30, 40], 95) == 40
    assert prof.nearest_rank([7], 1) == 7


def test_summarize_groups_totals_percentiles():
    s = prof.summarize(_fixture())
    rows = {tuple(r["key"]): r for r in s["rows"]}
    b = rows[("b", "linear")]
    assert b["calls"] == 4
    assert b["gpu"]["total"] == 2 * (10 + 20 + 30 + 40) and b["gpu"]["p50"] == 40
    assert b["cpu"]["total"] == 2 * 10 and b["cpu"]["p95"] == 8
    c = rows[("c", "attention")]
    assert c["gpu_unmeasured"] == 1 and c["gpu"]["n"] == 3
    assert abs(sum(r["gpu_pct"] for r in s["rows"]) - 100.0) < 1e-9
    assert s["rows"][0]["key"] == ["c", "attention"]  # sorted by GPU total
    assert s["run_wall"]["p50"] == 501 and s["gpu_unmeasured"] == 1
    by_op = {tuple(r["key"]): r for r in prof.summarize(_fixture(), group_by="op")["rows"]}
    assert by_op[("linear",)]["calls"] == 8
    skipped = prof.summarize(_fixture(), skip_runs=2)
    assert skipped["runs"] == 2 and {r["calls"] for r in skipped["rows"]} == {2}
    assert "nearest rank" in prof.format_summary(s)


def test_compare_and_refusals():
    before, after = _fixture(), _fixture(gpu=(20, 40, 60, 80))
    after["events"] = [e for e in after["events"] if e["node_name"] != "a"]
    res = {tuple(r["key"]): r for r in prof.compare(before, after, force=True)["rows"]}
    assert res[("a", "linear")]["status"] == "removed"
    assert res[("b", "linear")]["gpu_change_ns"] == 40 and res[("b", "linear")]["gpu_change_pct"] == 100.0
    assert res[("b", "linear")]["cpu_change_ns"] == 0
    with pytest.raises(prof.ProfileError):
        prof.compare(_fixture(device=0), _fixture(device=1))
    with pytest.raises(prof.ProfileError):
        prof.compare(_fixture(shapes="in:[a]"), _fixture(shapes="in:[b]"))
    assert prof.compare(_fixture(), _fixture())["rows"]


def test_export_trace_and_validation(tmp_path):
    doc = _fixture()
    rows = list(csv.DictReader(io.StringIO(prof.export(doc, "csv"))))
    assert len(rows) == 12 and rows[0]["node_name"] == "a" and rows[2]["gpu_duration_ns"] == ""
    t = prof.trace(doc)
    cpu = [x for x in t["traceEvents"] if x["cat"].startswith("cpu")]
    gpu = [x for x in t["traceEvents"] if x["cat"].startswith("gpu")]
    assert len(cpu) == 12 and len(gpu) == 11
    for a, b in zip(gpu, gpu[1:]):  # one track, spans end to end
        assert b["ts"] >= a["ts"] + a["dur"] - 1e-9
    with pytest.raises(prof.ProfileError):
        prof.load({"schema": "dli.profile.v2", "metadata": {}, "runs": [], "events": []})
    with pytest.raises(prof.ProfileError):
        prof.load({"schema": "dli.profile.v1", "metadata": {}, "runs": [], "events": [{}]})
    path = tmp_path / "f.json"
    path.write_text(json.dumps(doc))
    assert prof.main(["summarize", str(path)]) == 0
    assert prof.main(["trace", str(path), "-o", str(tmp_path / "t.json")]) == 0
    assert json.loads((tmp_path / "t.json").read_text())["traceEvents"]
    assert prof.main(["compare", str(path), str(path)]) == 0
