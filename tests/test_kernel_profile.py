"""gemma_hip.kernel_profile's summariser on a synthetic rocprofv3 counter CSV
(CPU): dispatches split at the separator kernel, counters averaged per
segment, byte counters scaled by the calibration copy."""
from __future__ import annotations

import csv
import json

from gemma_hip import kernel_profile as kp

COLS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size", "Kernel_Id",
        "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count",
        "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def _write(path, seq, counter):
    path.mkdir(parents=True)
    with open(path / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(COLS)
        for i, (name, v) in enumerate(seq, 1):
            w.writerow([i, i, "Agent 1", 1, 1, 1, 256, 1, name, 256, 0, 0, 8, 0, 32, counter, v, 1000 * i, 1000 * i + 500])


def test_summarize_splits_at_separators_and_calibrates(tmp_path, capsys):
    sep = "gh::k_stream_read(void const*, unsigned int, unsigned int, float*)"
    mv = "void gh::k_matvec<0, 3, 2, gh::ProResid<2, false>, gh::EpiPartial>(gh::DMat, int, gh::ProResid<2, false>, gh::EpiPartial)"
    at = "void gh::k_attn_step<256, 4>(gh::AttnArgs)"
    seq = [("k_prompt", 5.0)] * 3 + [(sep, 1.0), (sep, 1.0)] + [(mv, 100.0), (mv, 110.0)] + [(sep, 1.0)] * 2 \
        + [(at, 40.0)] * 4 + [(sep, 1.0)] * 2 + [("__amd_rocclr_fillBufferAligned", 0.0),
                                                 ("__amd_rocclr_copyBuffer", 4096.0)]
    _write(tmp_path / "fetch", seq, "FETCH_SIZE")
    man = {"config": "gemma3-1b", "position": 8, "copy_bytes": 8 << 20,
           "segments": [{"name": "gate_up", "reps": 1, "launches_per_step": 2, "bytes_per_launch": 210 * 2048},
                        {"name": "attention", "reps": 1, "launches_per_step": 4, "bytes_per_launch": 40 * 2048}]}
    (tmp_path / "m.json").write_text(json.dumps(man))
    kp.main(["summarize", "--manifest", str(tmp_path / "m.json"), "--fetch", str(tmp_path / "fetch")])
    out = capsys.readouterr().out
    # factor = 8 MiB / 4096 KiB-units = 2048 bytes per unit; gate_up averages 105 units
    assert "FETCH_SIZE 2048.00000" in out
    assert "| gate_up | 2 | 430,080 | 215,040 |" in out
    assert "| attention | 4 | 81,920 | 81,920 |" in out


def test_summarize_assigns_decode_dispatches_by_their_place_in_the_step(tmp_path, capsys):
    """A decode segment (eager steps in the step's launch order): each
    dispatch takes its kernel kind from its index modulo the recorded step
    sequence, and a segment whose count is not whole steps is refused."""
    import pytest
    sep = "gh::k_stream_read(void const*, unsigned int, unsigned int, float*)"
    a, b, c = "k_a(int)", "k_b(int)", "k_c(int)"
    step = [(a, 10.0), (b, 20.0), (a, 30.0), (c, 8.0)]
    seq = [(sep, 1.0), (sep, 1.0)] + step + step + [(sep, 1.0)] * 2 + [("__amd_rocclr_copyBuffer", 4096.0)]
    _write(tmp_path / "fetch", seq, "FETCH_SIZE")
    man = {"config": "gemma3-1b", "position": None, "copy_bytes": 8 << 20,
           "segments": [{"name": "decode", "steps": 2, "positions": [224, 225], "sequence": ["x", "y", "x", "z"],
                         "kinds": {"x": {"bytes_per_launch": 20 * 2048, "event_avg_us": 0.5},
                                   "y": {"bytes_per_launch": 20 * 2048, "event_avg_us": 0.5},
                                   "z": {"bytes_per_launch": 8 * 2048, "event_avg_us": 0.5}}}]}
    (tmp_path / "m.json").write_text(json.dumps(man))
    kp.main(["summarize", "--manifest", str(tmp_path / "m.json"), "--fetch", str(tmp_path / "fetch")])
    out = capsys.readouterr().out
    assert "| x | 4 | 40,960 | 40,960 |" in out  # (10 + 30) / 2 units of 2048 B
    assert "| y | 2 | 40,960 | 40,960 |" in out
    assert "| z | 2 | 16,384 | 16,384 |" in out
    man["segments"][0]["steps"] = 3
    (tmp_path / "m.json").write_text(json.dumps(man))
    with pytest.raises(SystemExit):
        kp.main(["summarize", "--manifest", str(tmp_path / "m.json"), "--fetch", str(tmp_path / "fetch")])
