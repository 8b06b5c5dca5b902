"""The rocprof harness (kda_bt16/profiling.py) on the CPU: the pass commands
it would run, and the reduction of rocprofv3's CSV files to the profiles/
summaries, on synthetic CSVs written here, read back through bench.py's own
readers."""

from __future__ import annotations

import csv
import json

import pytest

from kda_bt16 import profiling


def _write_csv(path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(header)
        w.writerows(rows)


K1 = "void kda::(anonymous namespace)::k1_kernel<0, true, true>(kda::Params)"
K2 = "void kda::(anonymous namespace)::k2_kernel<0>(kda::Params)"
COPY = "__amd_rocclr_copyBuffer"
TORCH = "void at::native::vectorized_elementwise_kernel<4, float>(int, float, float)"
CC_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
             "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
             "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
             "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def _counters(path, dispatches):
    """dispatches: [(kernel name, {counter: value})] in dispatch order."""
    rows = []
    for i, (name, vals) in enumerate(dispatches, 1):
        for c, v in vals.items():
            rows.append([i, i, "Agent 1", 1, 1, 1, 512, 7, name, 256, 0, 0, 8, 0, 32, c, v, 10 * i,
                         10 * i + 5])
    _write_csv(path, CC_HEADER, rows)


def _agent(path):
    _write_csv(path, ["Node_Id", "Agent_Type", "Cu_Count", "Num_Xcc", "Simd_Per_Cu", "Name"],
               [[0, "CPU", 0, 1, 0, "AMD EPYC"], [1, "GPU", 256, 8, 4, "gfx950"]])


def _fake_run(d):
    manifest = {"workload": "config", "config": "c2", "prefix": "kda_fwd_B1_T8192_H32",
                "bench": "python3 bench.py --steps 10 --warmup 3 --copy-calibration --workload config --config c2",
                "passes": {p: {"rocprofv3": f"rocprofv3 {' '.join(profiling.PASSES[p])} -- python3 bench.py",
                               "rc": 0} for p in ("trace", "fetch", "write", "mfma", "lds")}}
    d.mkdir(parents=True, exist_ok=True)
    (d / "manifest.json").write_text(json.dumps(manifest))
    _write_csv(d / "trace" / "run_kernel_stats.csv",
               ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"],
               [[K2, 3, 450000, 150000.0, 50.0, 140000, 160000, 1.0],
                [K1, 3, 330000, 110000.0, 40.0, 100000, 120000, 1.0],
                [TORCH, 1, 1000, 1000.0, 1.0, 1000, 1000, 0.0]])
    _write_csv(d / "trace" / "run_kernel_trace.csv",
               ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"],
               [["KERNEL_DISPATCH", i, K2 if i % 2 else K1, 1000 * i, 1000 * i + dur]
                for i, dur in enumerate([160000, 120000, 140000, 100000, 150000, 110000], 1)])
    _agent(d / "trace" / "run_agent_info.csv")
    copies = [(COPY, {"FETCH_SIZE": 131072.0}), (COPY, {"FETCH_SIZE": 131072.0}),
              (COPY, {"FETCH_SIZE": 131072.0})]
    # an input upload later in the run, larger than the calibration copy:
    # only the first three copies calibrate
    _counters(d / "fetch" / "run_counter_collection.csv",
              copies + [(COPY, {"FETCH_SIZE": 9e9}), (K1, {"FETCH_SIZE": 1000.0}),
                        (K1, {"FETCH_SIZE": 3000.0}), (K2, {"FETCH_SIZE": 500.0}),
                        (TORCH, {"FETCH_SIZE": 7.0})])
    _counters(d / "write" / "run_counter_collection.csv",
              [(COPY, {"WRITE_SIZE": 262144.0})] * 3 + [(K1, {"WRITE_SIZE": 100.0}),
                                                        (K2, {"WRITE_SIZE": 200.0})])
    mf = {"SQ_INSTS_VALU_MFMA_MOPS_BF16": 1000.0, "SQ_INSTS_VALU_MFMA_MOPS_F32": 10.0,
          "SQ_VALU_MFMA_BUSY_CYCLES": 4096.0, "GRBM_GUI_ACTIVE": 8000.0}
    _counters(d / "mfma" / "run_counter_collection.csv", [(K1, mf), (K2, mf), (K2, mf)])
    _agent(d / "mfma" / "run_agent_info.csv")
    _counters(d / "lds" / "run_counter_collection.csv",
              [(K2, {"SQ_INSTS_LDS": 10.0, "SQ_LDS_BANK_CONFLICT": 0.0, "SQ_WAIT_INST_LDS": 4.0,
                     "SQ_WAVES": 768.0, "GRBM_GUI_ACTIVE": 8000.0})])


def test_kernel_roles():
    r = profiling.kernel_role
    assert r(K1) == "k1" and r(K2) == "k2"
    assert r("void kda::(anonymous namespace)::k2_kernel<3>(kda::Params)") == "k2"
    assert r("void kda::(anonymous namespace)::k2w_kernel<4, 1>(kda::Params)") == "k2"
    assert r("void kda::(anonymous namespace)::k2s_kernel<2>(kda::Params)") == "k2"
    assert r("void kda::(anonymous namespace)::gate_segment_kernel(kda::Params)") == "gate_segment"
    assert r("void kda::(anonymous namespace)::gate_reduce_kernel(kda::Params)") == "gate_reduce"
    assert r("void kda::(anonymous namespace)::k1_kernel<2, false, true>(kda::Params)") == "k1_train_fwd"
    assert r("void kda::(anonymous namespace)::k2_kernel<2>(kda::Params)") == "k2_bwd_chain"
    assert r("void kda::(anonymous namespace)::k2_kernel<4>(kda::Params)") == "k2_train_fwd"
    assert r("void kda::(anonymous namespace)::fused_kernel<true>(kda::Params)") == "fused"
    assert r("void kda::(anonymous namespace)::k1_dout_kernel(kda::Params)") == "k1_dout"
    assert r("void kda::(anonymous namespace)::recurrent_kernel<true, true>(kda::Params)") == "recurrent"
    assert r(COPY) == "copy" and r(TORCH) is None


def test_pass_commands_put_the_program_after_the_separator(tmp_path):
    bench = profiling.bench_args("config", "c3", 10, 3)
    assert bench[-4:] == ["--workload", "config", "--config", "c3"] and "--copy-calibration" in bench
    for p in profiling.PASSES:
        cmd = profiling.pass_command(p, tmp_path, bench, "python3")
        assert cmd[:4] == ["timeout", "-s", "KILL", str(profiling.PASS_LIMIT_S)]
        assert cmd[4] == "rocprofv3"
        sep = cmd.index("--")
        assert cmd[sep + 1] == "python3" and cmd[sep + 2].endswith("bench.py")
        opts = cmd[5:sep]
        # counters never share a run with tracing domains
        assert not ({"--pmc"} & set(opts) and {"--kernel-trace", "-s", "--sys-trace"} & set(opts))
    assert profiling.profile_prefix("config", "c4") == "kda_fwd_B16_T2048_H32"
    assert profiling.profile_prefix("headline") == "kda_fwd_B1_T8192_H32"


def test_pass_counter_sets_fit_one_run():
    """At most 8 SQ, 4 TCC (FETCH_SIZE 3, WRITE_SIZE 2), 4 TCP, 2 TA, 2 TD
    and 2 GRBM counters per rocprofv3 run."""
    limits = {"SQ": 8, "TCC": 4, "TCP": 4, "TA": 2, "TD": 2, "GRBM": 2}
    cost = {"FETCH_SIZE": ("TCC", 3), "WRITE_SIZE": ("TCC", 2)}
    for p, opts in profiling.PASSES.items():
        if "--pmc" not in opts:
            continue
        used = {}
        for c in opts[opts.index("--pmc") + 1:]:
            block, n = cost.get(c, (c.split("_")[0], 1))
            used[block] = used.get(block, 0) + n
        for block, n in used.items():
            assert n <= limits[block], (p, block, n)


def test_summarize_writes_what_bench_reads(tmp_path, monkeypatch):
    run = tmp_path / "run"
    _fake_run(run)
    prof = tmp_path / "profiles"
    assert profiling.main(["summarize", "--dir", str(run), "--profiles", str(prof), "--last", "2"]) == 0
    t = json.loads((prof / "kda_fwd_B1_T8192_H32_traffic.json").read_text())
    assert t["fetch_scale"] == pytest.approx(2.0) and t["write_scale"] == pytest.approx(1.0)
    assert t["kernels"]["k1"]["FETCH_SIZE_KiB"] == 2000.0 and t["kernels"]["k1"]["dispatches"] == 2
    assert t["kernels"]["k1"]["hbm_bytes"] == int((2000.0 * 2 + 100.0) * 1024)
    assert set(t["kernels"]) == {"k1", "k2"}
    m = json.loads((prof / "kda_fwd_B1_T8192_H32_mfma.json").read_text())
    assert (m["cus"], m["xcds"], m["simds_per_cu"]) == (256, 8, 4)
    assert m["kernels"]["k2"]["dispatches"] == 2
    md = (prof / "kda_fwd_B1_T8192_H32_kernel_stats.md").read_text()
    assert "`k2_kernel<0>`" in md and "150.0" in md and "vectorized" not in md
    ks = json.loads((prof / "kda_fwd_B1_T8192_H32_kernel_stats.json").read_text())
    k2 = next(r for r in ks["kernels"] if r["role"] == "k2")
    assert k2["last_n"] == 2 and k2["last_avg_us"] == pytest.approx(145.0)
    c = json.loads((prof / "kda_fwd_B1_T8192_H32_counters.json").read_text())
    assert c["lds"]["kernels"]["k2"]["SQ_INSTS_LDS"] == 10.0
    # bench.py's readers of the committed summaries
    import bench

    monkeypatch.setattr(bench, "ROOT", tmp_path)
    tr = bench.measured_traffic(1, 8192, 32)
    assert tr["k1"] == t["kernels"]["k1"]["hbm_bytes"]
    mf = bench.measured_mfma({"k1": {"ms": 0.1}, "k2": {"ms": 0.2}}, 1, 8192, 32)
    assert mf["k1"]["bf16_flops"] == 1000 * 512
    assert mf["k2"]["mfma_busy_frac"] == pytest.approx(4096.0 / (8000.0 / 8 * 256 * 4), abs=1e-5)


def test_missing_calibration_is_an_error(tmp_path):
    run = tmp_path / "run"
    _fake_run(run)
    _counters(run / "fetch" / "run_counter_collection.csv", [(K1, {"FETCH_SIZE": 1.0})])
    with pytest.raises(ValueError, match="calibration copy"):
        profiling.main(["summarize", "--dir", str(run), "--profiles", str(tmp_path / "p")])
