"""The rocprofv3 summariser (triton-fa2-forward_amd/rocprof_summary.py) on a committed fixture.

tests/golden/rocprof/ holds the CSVs of one real profiling run of C3 on MI355X (the kernel trace,
cut to the dispatches the summary reads, and the FETCH_SIZE, WRITE_SIZE, SQ and utilisation
counter runs, whole) and the fields of that run's bench.py line. The expected figures are the ones
the previous summaries committed for that very run, computed then by a separate script: the L2-miss
bytes per launch and their copy calibration, the MFMA-busy fraction and instruction mix, the
per-unit busy fractions, and the per-step kernel times of the timed dispatches. The reference
tests its Nsight summariser the same way, on a saved export (tests/test_ncu_summary.py).
"""

import json
import os

import pytest

import rocprof_summary as rs

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rocprof")


def test_copy_calibration_and_l2_miss_bytes():
    fetch, write = rs.pmc(os.path.join(FIX, "C3_fetch")), rs.pmc(os.path.join(FIX, "C3_write"))
    fs, ws = rs.copy_scales(fetch, write)
    # the calibration copy moved 1 GiB each way; FETCH_SIZE read half of it (64-byte requests
    # counted in 32-byte units), WRITE_SIZE all of it
    assert fs == pytest.approx(1.999900107604851, rel=1e-12)
    assert ws == 1.0
    t = rs.traffic(fetch, write)
    assert len(t["fetch_kib_each"]) == len(t["write_kib_each"]) == 3   # three attention launches
    assert t["fetch_kib"] == pytest.approx(130341.10416666667, rel=1e-12)
    assert t["write_kib"] == pytest.approx(65556.10416666667, rel=1e-12)
    assert abs(t["bytes"] - 334054699) <= 1      # the committed figure for this run


def test_key_norm_dispatches_are_not_attention():
    fetch = rs.pmc(os.path.join(FIX, "C3_fetch"))
    assert len(rs.values(fetch, rs.KEY_NORM, "FETCH_SIZE")) == 3
    assert all(v > 8000 for v in rs.values(fetch, rs.KEY_NORM, "FETCH_SIZE"))   # K once: 8 MiB/2
    assert all(v > 129000 for v in rs.values(fetch, rs.ATTN, "FETCH_SIZE"))


def test_sq_and_utilisation_readings():
    sq = rs.first_attn(rs.pmc(os.path.join(FIX, "C3_sq")))
    busy = sq["SQ_VALU_MFMA_BUSY_CYCLES"] / rs.SIMDS / (sq["GRBM_GUI_ACTIVE"] / rs.XCDS)
    assert round(100 * busy, 1) == 68.5
    assert round(sq["SQ_INSTS_MFMA"] / sq["SQ_WAVES"]) == 1943
    assert sq["SQ_LDS_BANK_CONFLICT"] == 0
    u = rs.utilisation(rs.first_attn(rs.pmc(os.path.join(FIX, "C3_util"))))
    got = {k: round(100 * u[k], 1) for k in ("mfma_busy", "valu_busy", "lds_busy", "salu_busy")}
    assert got == {"mfma_busy": 68.6, "valu_busy": 51.2, "lds_busy": 34.5, "salu_busy": 15.6}
    assert round(100 * u["mfma_with_valu"]) == 38
    assert u["exp_insts"] == pytest.approx(1.7e7, rel=0.01)


def test_kernel_trace_steps():
    d = os.path.join(FIX, "C3_trace")
    stats = rs.kernel_stats(d)
    assert "attn_fwd_kernel" in stats[0][0] and stats[0][1] == 4511 and round(stats[0][2]) == 454675
    b = rs.bench_line(d + ".log")
    K = b["steps"]
    attn, kn = rs.dispatches(d, rs.ATTN), rs.dispatches(d, rs.KEY_NORM)
    timed, ktimed = attn[-2 * K:-K], kn[-2 * K:-K]
    t_attn = sum(e - s for s, e in timed) / K
    t_kn = sum(e - s for s, e in ktimed) / K
    # the committed summary of this run: key-norm 4.8 us + attention 454.4 us = 459.2 us per step
    assert (round(t_kn / 1e3, 1), round(t_attn / 1e3, 1), round((t_kn + t_attn) / 1e3, 1)) == (4.8, 454.4, 459.2)


def test_writers_produce_the_summaries(tmp_path):
    """The four writers run end to end on the fixture into a scratch folder; the JSON entry is
    the one bench.py reads (profiles/l2_miss_traffic.json's layout)."""
    j = str(tmp_path / "l2.json")
    assert os.path.exists(rs.write_trace(FIX, "C3", str(tmp_path)))
    path, t = rs.write_traffic(FIX, "C3", str(tmp_path), j, "fixture")
    text = open(path).read()
    assert "334054699 bytes" in text.replace(",", "") and "1.99x" in text
    entry = json.load(open(j))["configs"]["C3"]
    assert abs(entry["bytes"] - 334054699) <= 1 and entry["kernel_build"] == "fixture"
    assert entry["algorithmic_bytes"] == 167772160
    assert "68.5%" in open(rs.write_sq(FIX, "C3", str(tmp_path))).read()
    upath, u = rs.write_util(FIX, ["C3"], str(tmp_path))
    assert "68.6%" in open(upath).read()
    trace = open(str(tmp_path / "attn_fwd_kernel_C3_kernel_trace.md")).read()
    assert "key-norm pass 4.8 us + attention kernel 454.4 us = 459.2 us" in trace
