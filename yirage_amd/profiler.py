"""Per-task profile of the persistent kernel as a Perfetto trace.

The device writes, per task, {start, inputs ready, end, worker, four stage
stamps} in 10 ns ticks of the GPU's constant clock (yr_pk_set_profiler).
export_to_perfetto_trace() turns one launch's records into a trace with one
track per worker and one slice per task, named like the reference's trace
(python/yirage/profiler_persistent.py:89-136: "<TASK_TYPE>_<n>"), with the
wait for inputs and the stage stamps as slice arguments.  The file is the
JSON trace-event format, which ui.perfetto.dev and trace_processor open
directly; the reference writes the same slices through the tg4perfetto
protobuf writer, a dependency this package does not have.
"""
from __future__ import annotations

import json

import numpy as np

# this backend's task types (csrc/pk_types.h) -> the reference's task names
# (include/yirage/persistent_kernel/runtime_header.h:62-124)
TASK_NAMES = {
    1: "TASK_EMBEDDING",
    2: "TASK_LINEAR",
    3: "TASK_RMS_NORM_LINEAR",
    4: "TASK_RMS_NORM_LINEAR_SILU_MUL",
    5: "TASK_PAGED_ATTENTION_1",
    6: "TASK_RMS_NORM_LINEAR_ARGMAX",
    7: "TASK_PREPARE_NEXT_BATCH",
}
STAGES = ("stage4", "stage5", "stage6", "stage7")


def trace_events(profile: np.ndarray, task_table: np.ndarray) -> list:
    """Trace events (one complete slice per executed task) from the
    [tasks, 8] profile and the [tasks, 10] task table of PersistentKernel."""
    prof = np.asarray(profile, dtype=np.int64).reshape(-1, 8)
    ran = prof[:, 0] > 0
    if not ran.any():
        return []
    t0 = int(prof[ran, 0].min())
    workers = sorted(set(int(w) for w in prof[ran, 3]))
    ev = [{"name": "process_name", "ph": "M", "pid": 0, "args": {"name": "persistent kernel"}}]
    for w in workers:
        ev.append({"name": "thread_name", "ph": "M", "pid": 0, "tid": w, "args": {"name": f"worker_{w}"}})
    counts: dict = {}
    for t in np.nonzero(ran)[0]:
        rec = prof[t]
        op, ty = int(task_table[t][0]), int(task_table[t][1])
        base = TASK_NAMES.get(ty, f"TASK_{ty}")
        n = counts.get(op, 0)
        counts[op] = n + 1
        start, ready, end = int(rec[0]), int(rec[1]), int(rec[2])
        args = {"task": int(t), "op": op, "wait_us": max(0, ready - start) / 100.0 if ready else None}
        for k, name in enumerate(STAGES):
            v = int(rec[4 + k])
            if v:
                args[name + "_us"] = (v - start) / 100.0
        ev.append({"name": f"{base}_{op}", "cat": base, "ph": "X", "pid": 0, "tid": int(rec[3]),
                   "ts": (start - t0) / 100.0, "dur": max(0, end - start) / 100.0, "args": args})
    return ev


def export_to_perfetto_trace(profile, file_name: str, task_table) -> int:
    """Write the trace of one launch; returns the number of task slices."""
    if hasattr(profile, "cpu"):
        profile = profile.cpu().numpy()
    ev = trace_events(profile, task_table)
    with open(file_name, "w") as f:
        json.dump({"traceEvents": ev, "displayTimeUnit": "ns"}, f)
    return sum(1 for e in ev if e["ph"] == "X")
