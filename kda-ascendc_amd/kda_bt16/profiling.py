"""rocprofv3 harness of the KDA BT=16 kernels: run the counter passes over a
``bench.py`` workload on the GPU box, then reduce rocprofv3's CSV output to
the summaries under ``profiles/`` that ``bench.py`` reads.

It has the role of the reference's profiler driver
(``/root/reference/tools/msprof_op_kda.py:1-14``) and of its CSV-to-summary
reducer (``/root/reference/tools/parse_msop_pipeutilization.py:1-13``).

Standard library only: run it as a script, so the process that starts the
profiler never touches the GPU itself::

    # on the GPU box: one rocprofv3 run per pass, the program after `--`
    python3 kda-ascendc_amd/kda_bt16/profiling.py run --workload config --config c2 \\
        --out gpurun_out/prof_c2 [--passes trace,fetch,write,mfma] [--steps 10 --warmup 3]

    # anywhere: the CSVs to profiles/<prefix>_{kernel_stats.md,traffic.json,mfma.json,
    # counters.json,counters.md}
    python3 kda-ascendc_amd/kda_bt16/profiling.py summarize --dir gpurun_out/prof_c2 \\
        --profiles profiles

Passes (``PASSES``): ``trace`` (``--kernel-trace --stats``), ``fetch``
(``FETCH_SIZE``), ``write`` (``WRITE_SIZE``), ``mfma`` (matrix-op counts and
busy cycles), ``texture`` (the per-CU vector-memory path), ``lds`` (LDS
instructions, bank conflicts and waits), ``l2write`` (L1-to-L2 and L2-to-HBM
write requests), ``waves`` (where the waves' cycles go: waiting, issuing,
by instruction kind).  Each pass is its own process under ``timeout -s KILL``,
with at most the counters one rocprofv3 run can collect.

HBM bytes: rocprofv3's ``FETCH_SIZE`` / ``WRITE_SIZE`` (KiB per dispatch)
are scaled by what they read for a plain device copy of known size, the
256 MiB copy that ``bench.py --copy-calibration`` runs first (its first three
``copyBuffer`` dispatches), so that bytes = FETCH_SIZE x fetch_scale +
WRITE_SIZE x write_scale, in KiB.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import shlex
import subprocess
import sys
import time
from collections import defaultdict
from pathlib import Path

REPO = Path(__file__).resolve().parents[2]
BENCH = REPO / "bench.py"

# rocprofv3 arguments of each pass.  One run holds at most 8 SQ, 4 TCC
# (FETCH_SIZE takes 3, WRITE_SIZE 2), 4 TCP, 2 TA, 2 TD and 2 GRBM counters.
PASSES = {
    "trace": ["--kernel-trace", "--stats"],
    "fetch": ["--pmc", "FETCH_SIZE"],
    "write": ["--pmc", "WRITE_SIZE"],
    "mfma": ["--pmc", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F32",
             "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"],
    "texture": ["--pmc", "TA_TA_BUSY_sum", "TD_TD_BUSY_sum", "TCP_PENDING_STALL_CYCLES_sum",
                "TCP_TCC_READ_REQ_sum", "TCP_TCC_READ_REQ_LATENCY_sum", "GRBM_GUI_ACTIVE"],
    "lds": ["--pmc", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_WAIT_INST_LDS", "SQ_WAVES",
            "GRBM_GUI_ACTIVE"],
    "l2write": ["--pmc", "TCP_TCC_WRITE_REQ_sum", "TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum",
                "GRBM_GUI_ACTIVE"],
    "waves": ["--pmc", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
              "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_MISC",
              "GRBM_GUI_ACTIVE"],
}
DEFAULT_PASSES = ("trace", "fetch", "write", "mfma")
PASS_LIMIT_S = 180

# (B, T, H) of bench.py's BASELINE configs.
CONFIG_SHAPES = {"c0": (2, 1024, 4), "c1": (2, 4096, 8), "c2": (1, 8192, 32),
                 "c3": (1, 8192, 96), "c4": (16, 2048, 32)}

CALIBRATION_KIB = 262144.0  # the 256 MiB copy of bench.py --copy-calibration, each way


def profile_prefix(workload: str, config: str = "c2") -> str:
    """File-name prefix of a workload's summaries under profiles/."""
    if workload in ("headline", "config"):
        b, t, h = CONFIG_SHAPES["c2" if workload == "headline" else config]
        return f"kda_fwd_B{b}_T{t}_H{h}"
    return {"varlen": "kda_varlen_T8192_N16_H32", "train": "kda_train_B1_T8192_H32",
            "decode": "kda_decode_B128_H32"}[workload]


# Roles of the stage kernels' record modes (kda_k1_chunk.h K1Mode,
# kda_k2.hip K2Mode): the forward's, the training forward's (which keeps its
# state), and the backward's.
_K1_MODES = {"0": "k1", "1": "k1_bwd_recompute", "2": "k1_train_fwd"}
_K2_MODES = {"0": "k2", "3": "k2", "1": "k2_bwd_recompute", "2": "k2_bwd_chain",
             "4": "k2_train_fwd"}
# The backward's kernels when it starts from the saved state (bench.py
# --workload train reads their traffic).
BACKWARD_ROLES = ["k1_dout", "k2_bwd_chain", "bwd_chunk", "gate_segment", "gate_reduce"]


def kernel_role(name: str) -> str | None:
    """The role of a kernel in the summaries, from its (demangled) name:
    k1 (stage 1), k2 (stage 2, one or several value tiles or sequences per
    work-group), fused, recurrent, the training and backward kernels by
    mode, or copy (the calibration copy); None for anything else (torch's
    own kernels)."""
    m = re.search(r"\bk1_kernel<(\d+)", name)
    if m:
        return _K1_MODES.get(m.group(1), "k1_mode" + m.group(1))
    m = re.search(r"\bk2_kernel<(\d+)", name)
    if m:
        return _K2_MODES.get(m.group(1), "k2_mode" + m.group(1))
    for key, role in (("fused_kernel", "fused"), ("k1_dout_kernel", "k1_dout"),
                      ("k2w_kernel", "k2"), ("k2s_kernel", "k2"), ("recurrent_kernel", "recurrent"),
                      ("bwd_chunk_kernel", "bwd_chunk"), ("gate_segment_kernel", "gate_segment"),
                      ("gate_reduce_kernel", "gate_reduce"),
                      ("copyBuffer", "copy")):
        if key in name:
            return role
    return None


# ----------------------------------------------------------------------------
# run (on the GPU box)


def bench_args(workload: str, config: str, steps: int, warmup: int) -> list[str]:
    a = ["--steps", str(steps), "--warmup", str(warmup), "--copy-calibration"]
    if workload == "config":
        a += ["--workload", "config", "--config", config]
    elif workload == "headline":
        a += ["--no-cpu-baseline"]
    else:
        a += ["--workload", workload]
    return a


def pass_command(pass_name: str, out_dir: Path, bench: list[str], python: str) -> list[str]:
    """The rocprofv3 command of one pass: the profiler under a hard time
    limit, the Python program itself after `--`."""
    return ["timeout", "-s", "KILL", str(PASS_LIMIT_S), "rocprofv3", *PASSES[pass_name],
            "-d", str(out_dir / pass_name), "-o", "run", "--output-format", "csv", "--",
            python, str(BENCH), *bench]


def run(args) -> int:
    out = Path(args.out).resolve()
    out.mkdir(parents=True, exist_ok=True)
    passes = [p for p in args.passes.split(",") if p]
    for p in passes:
        if p not in PASSES:
            raise SystemExit(f"unknown pass {p!r}; choose from {sorted(PASSES)}")
    bench = bench_args(args.workload, args.config, args.steps, args.warmup)
    manifest = {"workload": args.workload, "config": args.config,
                "prefix": profile_prefix(args.workload, args.config),
                "bench": "python3 bench.py " + " ".join(bench), "passes": {}}
    env = dict(os.environ, TMPDIR="/tmp")
    for p in passes:
        cmd = pass_command(p, out, bench, args.python)
        print(f"== pass {p}: {shlex.join(cmd)}", flush=True)
        t0 = time.time()
        with open(out / f"{p}.log", "w") as log:
            rc = subprocess.run(cmd, cwd="/tmp", env=env, stdout=log, stderr=subprocess.STDOUT).returncode
        print(f"   rc {rc} in {time.time() - t0:.1f} s", flush=True)
        lines = (out / f"{p}.log").read_text(errors="replace").splitlines()
        # rocprofv3 can end with a segmentation fault after the program has
        # finished and its results are whole: keep such a pass when the
        # program's JSON line came out and the CSVs are there
        done = any(ln.startswith("{") for ln in lines) and bool(_csvs(out / p))
        if rc != 0 and not (rc in (139, -11) and done):
            print(f"   pass {p} failed; see {out / (p + '.log')}", flush=True)
            return rc
        manifest["passes"][p] = {
            "rocprofv3": "rocprofv3 " + " ".join(PASSES[p]) + f" -d <out>/{p} -o run --output-format csv"
                         f" -- python3 <repo>/bench.py " + " ".join(bench),
            "rc": rc}
        (out / "manifest.json").write_text(json.dumps(manifest, indent=1))
    return 0


def _csvs(d: Path) -> list[str]:
    return glob.glob(str(d / "**" / "*.csv"), recursive=True)


# ----------------------------------------------------------------------------
# summarize (anywhere)


def _find(d: Path, suffix: str) -> Path | None:
    hits = sorted(glob.glob(str(d / "**" / f"*{suffix}"), recursive=True))
    return Path(hits[0]) if hits else None


def read_counters(d: Path) -> tuple[dict, list]:
    """{(role, counter): [value per dispatch]} from a pass's
    counter_collection.csv, and the copy dispatches in order as
    [(dispatch id, counter, value)]."""
    f = _find(d, "counter_collection.csv")
    if f is None:
        raise FileNotFoundError(f"no counter_collection.csv under {d}")
    vals = defaultdict(list)
    copies = []
    with open(f, newline="") as fh:
        for r in csv.DictReader(fh):
            role = kernel_role(r["Kernel_Name"])
            if role is None:
                continue
            v = float(r["Counter_Value"])
            vals[(role, r["Counter_Name"])].append(v)
            if role == "copy":
                copies.append((int(r["Dispatch_Id"]), r["Counter_Name"], v))
    return vals, copies


def read_agent(d: Path) -> dict:
    """CUs, XCDs and SIMDs per CU of the GPU agent (agent_info.csv)."""
    f = _find(d, "agent_info.csv")
    out = {"cus": 256, "xcds": 8, "simds_per_cu": 4}
    if f is None:
        return out
    with open(f, newline="") as fh:
        for r in csv.DictReader(fh):
            if r.get("Agent_Type") == "GPU":
                out = {"cus": int(r["Cu_Count"]), "xcds": int(r["Num_Xcc"]),
                       "simds_per_cu": int(r["Simd_Per_Cu"])}
                if r.get("Name"):
                    out["gfx"] = r["Name"]
                break
    return out


def calibration_scale(copies: list, counter: str) -> tuple[float, float]:
    """(scale, KiB read) from the first three dispatches of the calibration
    copy: CALIBRATION_KIB over the mean value of `counter` on them."""
    first = sorted({c[0] for c in copies if c[1] == counter})[:3]
    vals = [v for i, c, v in copies if c == counter and i in first]
    if len(vals) < 3:
        raise ValueError(f"calibration copy not found for {counter} (run bench.py with --copy-calibration)")
    mean = sum(vals) / len(vals)
    return CALIBRATION_KIB / mean, mean


def _mean(xs: list) -> float:
    return sum(xs) / len(xs)


def traffic_summary(fetch_dir: Path, write_dir: Path, manifest: dict) -> dict:
    f, fc = read_counters(fetch_dir)
    w, wc = read_counters(write_dir)
    fs, fk = calibration_scale(fc, "FETCH_SIZE")
    ws, wk = calibration_scale(wc, "WRITE_SIZE")
    kernels = {}
    for role in sorted({r for r, c in f if r != "copy"}):
        if (role, "WRITE_SIZE") not in w:
            continue
        fe, wr = f[(role, "FETCH_SIZE")], w[(role, "WRITE_SIZE")]
        kernels[role] = {"FETCH_SIZE_KiB": round(_mean(fe), 1), "WRITE_SIZE_KiB": round(_mean(wr), 1),
                         "dispatches": len(fe),
                         "hbm_bytes": int(round((_mean(fe) * fs + _mean(wr) * ws) * 1024))}
    out = {
        "workload": manifest.get("bench", ""),
        "source": "; ".join(manifest["passes"][p]["rocprofv3"] for p in ("fetch", "write")
                            if p in manifest.get("passes", {})),
        "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
        "calibration": f"256 MiB device copy (copyBuffer, first 3 dispatches): FETCH_SIZE {fk:.1f} KiB, "
                       f"WRITE_SIZE {wk:.1f} KiB for {CALIBRATION_KIB:.0f} KiB moved each way",
        "kernels": kernels,
    }
    if manifest.get("workload") == "train":
        out["backward_kernels"] = [r for r in BACKWARD_ROLES if r in kernels]
    return out


def counter_summary(d: Path, manifest: dict, pass_name: str) -> dict:
    vals, _ = read_counters(d)
    kernels = defaultdict(dict)
    for (role, counter), xs in vals.items():
        if role == "copy":
            continue
        kernels[role][counter] = round(_mean(xs), 1)
        kernels[role]["dispatches"] = len(xs)
    out = {"workload": manifest.get("bench", ""),
           "source": manifest.get("passes", {}).get(pass_name, {}).get("rocprofv3", ""),
           "units": "means per dispatch of each kernel role; *_sum counters summed over the "
                    "GPU's units; GRBM_GUI_ACTIVE summed over the XCDs",
           "kernels": dict(sorted(kernels.items()))}
    out.update(read_agent(d))
    return out


def kernel_stats(trace_dir: Path, last: int = 20) -> list[dict]:
    """Per kernel of the library (and the calibration copy): calls and
    average / min / max µs from kernel_stats.csv, and the mean of its last
    `last` dispatches from kernel_trace.csv (the timed forwards and the
    latency loop run last)."""
    rows = []
    f = _find(trace_dir, "kernel_stats.csv")
    if f is None:
        raise FileNotFoundError(f"no kernel_stats.csv under {trace_dir}")
    tail = defaultdict(list)
    t = _find(trace_dir, "kernel_trace.csv")
    if t is not None:
        with open(t, newline="") as fh:
            for r in csv.DictReader(fh):
                tail[r["Kernel_Name"]].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    with open(f, newline="") as fh:
        for r in csv.DictReader(fh):
            role = kernel_role(r["Name"])
            if role is None:
                continue
            d = tail.get(r["Name"], [])[-last:]
            rows.append({"kernel": r["Name"], "role": role, "calls": int(r["Calls"]),
                         "avg_us": float(r["AverageNs"]) / 1e3, "min_us": float(r["MinNs"]) / 1e3,
                         "max_us": float(r["MaxNs"]) / 1e3,
                         "last_avg_us": (sum(d) / len(d) / 1e3) if d else None,
                         "last_n": len(d)})
    return rows


def _short(name: str) -> str:
    return name.replace("void ", "").replace("kda::(anonymous namespace)::", "").replace("(kda::Params)", "")


def kernel_stats_md(rows: list[dict], manifest: dict, agent: dict) -> str:
    cmd = manifest.get("passes", {}).get("trace", {}).get("rocprofv3", "")
    lines = [f"# rocprofv3 kernel trace: {manifest.get('bench', '')}", "",
             "Made by `kda-ascendc_amd/kda_bt16/profiling.py` (pass `trace`), on the GPU box from /tmp "
             "with TMPDIR=/tmp:", "", f"    {cmd}", "",
             f"GPU: {agent.get('gfx', 'gfx950')}, {agent['cus']} CUs, {agent['xcds']} XCDs. "
             "Every dispatch of the run (precision checks, stage timing loops, warmup, timed and "
             "latency loops) counts in `calls`; `last N avg` is the mean of the kernel's last N "
             "dispatches, which are the timed and latency forwards.", "",
             "| kernel | role | calls | avg µs | min µs | max µs | last N avg µs (N) |",
             "|---|---|---:|---:|---:|---:|---:|"]
    for r in sorted(rows, key=lambda r: -r["avg_us"] * r["calls"]):
        last = "" if r["last_avg_us"] is None else f"{r['last_avg_us']:.1f} ({r['last_n']})"
        lines.append(f"| `{_short(r['kernel'])}` | {r['role']} | {r['calls']} | {r['avg_us']:.1f} | "
                     f"{r['min_us']:.1f} | {r['max_us']:.1f} | {last} |")
    return "\n".join(lines) + "\n"


def counters_md(summaries: dict, manifest: dict) -> str:
    lines = [f"# rocprofv3 counters: {manifest.get('bench', '')}", "",
             "Made by `kda-ascendc_amd/kda_bt16/profiling.py`, one rocprofv3 run per pass "
             "(on the GPU box from /tmp with TMPDIR=/tmp). Means per dispatch of each kernel role.", ""]
    for p, s in summaries.items():
        lines += [f"## {p}", "", f"    {s.get('source', '')}", ""]
        names = sorted({c for k in s["kernels"].values() for c in k if c != "dispatches"})
        lines.append("| role | dispatches | " + " | ".join(names) + " |")
        lines.append("|---|---:|" + "---:|" * len(names))
        for role, k in s["kernels"].items():
            lines.append(f"| {role} | {k.get('dispatches', '')} | "
                         + " | ".join(f"{k.get(n, float('nan')):.1f}" for n in names) + " |")
        lines.append("")
    return "\n".join(lines)


def summarize(args) -> int:
    d = Path(args.dir).resolve()
    manifest = json.loads((d / "manifest.json").read_text())
    prof = Path(args.profiles).resolve()
    prof.mkdir(parents=True, exist_ok=True)
    prefix = args.prefix or manifest["prefix"]
    passes = manifest.get("passes", {})
    written = []
    if "trace" in passes:
        agent = read_agent(d / "trace")
        rows = kernel_stats(d / "trace", args.last)
        (prof / f"{prefix}_kernel_stats.md").write_text(kernel_stats_md(rows, manifest, agent))
        (prof / f"{prefix}_kernel_stats.json").write_text(json.dumps(
            {"workload": manifest.get("bench", ""), "source": passes["trace"]["rocprofv3"],
             "kernels": rows}, indent=1) + "\n")
        written += [f"{prefix}_kernel_stats.md", f"{prefix}_kernel_stats.json"]
    if "fetch" in passes and "write" in passes:
        t = traffic_summary(d / "fetch", d / "write", manifest)
        (prof / f"{prefix}_traffic.json").write_text(json.dumps(t, indent=1) + "\n")
        written.append(f"{prefix}_traffic.json")
    if "mfma" in passes:
        m = counter_summary(d / "mfma", manifest, "mfma")
        (prof / f"{prefix}_mfma.json").write_text(json.dumps(m, indent=1) + "\n")
        written.append(f"{prefix}_mfma.json")
    extra = {p: counter_summary(d / p, manifest, p) for p in ("texture", "lds", "l2write", "waves")
             if p in passes}
    if extra:
        (prof / f"{prefix}_counters.json").write_text(json.dumps(extra, indent=1) + "\n")
        (prof / f"{prefix}_counters.md").write_text(counters_md(extra, manifest))
        written += [f"{prefix}_counters.json", f"{prefix}_counters.md"]
    for w in written:
        print(prof / w)
    return 0


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run", help="profile a bench.py workload (on the GPU box)")
    r.add_argument("--workload", default="config",
                   choices=("headline", "config", "varlen", "train", "decode"))
    r.add_argument("--config", default="c2", choices=sorted(CONFIG_SHAPES))
    r.add_argument("--out", required=True)
    r.add_argument("--passes", default=",".join(DEFAULT_PASSES))
    r.add_argument("--steps", type=int, default=10)
    r.add_argument("--warmup", type=int, default=3)
    r.add_argument("--python", default=sys.executable or "python3")
    s = sub.add_parser("summarize", help="reduce a run's CSVs to the profiles/ summaries")
    s.add_argument("--dir", required=True)
    s.add_argument("--profiles", default=str(REPO / "profiles"))
    s.add_argument("--prefix", default=None)
    s.add_argument("--last", type=int, default=20)
    a = ap.parse_args(argv)
    return run(a) if a.cmd == "run" else summarize(a)


if __name__ == "__main__":
    sys.exit(main())
