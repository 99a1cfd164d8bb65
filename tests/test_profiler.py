"""Perfetto export of the persistent kernel's per-task profile
(python/yirage/profiler_persistent.py:89-136 of the reference): the trace
has one track per worker and one slice per executed task, named
<TASK_TYPE>_<op>, with microsecond timestamps from the 10 ns device clock."""
import json

import numpy as np
import pytest
import torch

from yirage_amd.profiler import export_to_perfetto_trace, trace_events


def test_trace_events_from_a_synthetic_profile(tmp_path):
    prof = np.zeros((4, 8), np.int64)
    # task: start, ready, end, worker, stage stamps
    prof[0] = [1000, 1100, 1500, 0, 1200, 1400, 0, 0]
    prof[1] = [1000, 1000, 1300, 1, 0, 0, 0, 0]
    prof[2] = [1600, 1700, 2600, 0, 0, 0, 0, 0]
    # task 3 never ran (all zero)
    table = np.zeros((4, 10), np.int64)
    table[:, 0] = [0, 0, 1, 2]
    table[:, 1] = [3, 3, 5, 6]
    ev = trace_events(prof, table)
    sl = [e for e in ev if e["ph"] == "X"]
    assert [e["name"] for e in sl] == ["TASK_RMS_NORM_LINEAR_0", "TASK_RMS_NORM_LINEAR_0", "TASK_PAGED_ATTENTION_1_1"]
    assert [e["tid"] for e in sl] == [0, 1, 0]
    assert [e["ts"] for e in sl] == [0.0, 0.0, 6.0] and [e["dur"] for e in sl] == [5.0, 3.0, 10.0]
    assert sl[0]["args"]["wait_us"] == 1.0 and sl[0]["args"]["stage4_us"] == 2.0
    assert {e["args"]["name"] for e in ev if e["name"] == "thread_name"} == {"worker_0", "worker_1"}
    f = tmp_path / "t.perfetto-trace"
    assert export_to_perfetto_trace(prof, str(f), table) == 3
    assert len(json.loads(f.read_text())["traceEvents"]) == len(ev)


@pytest.mark.gpu
def test_persistent_kernel_profiler_tensor_writes_a_trace(tmp_path):
    """PersistentKernel(profiler_tensor=..., trace_name=...) exports after
    every launch, as the reference's __call__ does."""
    from yirage_amd.llama import LlamaConfig, LlamaDecodeModel

    cfg = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096)
    model = LlamaDecodeModel(cfg, batch=1, kv_len=100, seed=1)
    pk = model.pk
    n = pk.graph_info()["tasks"]
    pk.profiler_tensor = torch.zeros(n * 8, dtype=torch.int64, device="cuda")
    pk.trace_name = str(tmp_path / "decode")
    pk.enable_profiler(tensor=pk.profiler_tensor)
    model.set_input_tokens([5])
    model.step()
    torch.cuda.synchronize()
    data = json.loads((tmp_path / "decode.perfetto-trace").read_text())
    sl = [e for e in data["traceEvents"] if e["ph"] == "X"]
    print(f"[profiler] {len(sl)} task slices of {n}", flush=True)
    assert len(sl) == n
    assert all(e["dur"] >= 0 for e in sl)
    ops = {e["args"]["op"] for e in sl}
    assert ops == set(range(pk.graph_info()["ops"]))
    # tasks of one worker do not overlap
    by_w = {}
    for e in sl:
        by_w.setdefault(e["tid"], []).append((e["ts"], e["ts"] + e["dur"]))
    for spans in by_w.values():
        spans.sort()
        assert all(a[1] <= b[0] + 1e-3 for a, b in zip(spans, spans[1:]))
