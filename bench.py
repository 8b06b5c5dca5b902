"""Benchmark of the KDA BT=16 forward on one MI355X.

Workload (the headline): BASELINE configs[2], B=1 T=8192 H=32 K=V=128, bf16
q/k/v/g/beta, A_log = log U(1,16), dt_bias ~N(0, 0.1), zero initial state,
final state returned, all in-kernel flags on (lower_bound -5, scale
128^-0.5).  A step is one kda_bt16_fwd over that batch with inputs already
resident in HBM.

Prints ONE JSON line with the throughput (tokens/s), the roofline of the
forward's dominant kernel (the forward's algorithmic bytes over that
kernel's mean launch time from HIP events on its stream, and its HBM bytes
per launch), the same for the whole forward and per kernel (with the
matrix-op work that rocprofv3 counters measured), the precision of o and ht
against the fp32 token recurrence, and the CPU restatement of the reference
chunked path timed on this host.

  python bench.py [--gpus 1] [--steps 200] [--warmup 50] [--no-cpu-baseline]

More workloads, each printing its own line in the same format (not the
headline metric):
  --workload config --config c0..c4
                      any BASELINE config (c0 B=2 T=1024 H=4, c1 B=2
                      T=4096 H=8 with h0, c2 the headline, c3 B=1 T=8192
                      H=96, c4 B=16 T=2048 H=32 with h0 and g_raw std 2);
  --workload train    one training step of the op (forward, then the
                      backward through autograd) at the headline shape;
  --workload varlen   the same 8192 tokens and 32 heads as 16 packed
                      sequences of uneven lengths (cu_seqlens);
  --workload decode   one decode step (T = 1, state updated in place) for
                      B = 128 sequences of 32 heads: the token recurrence,
                      bound by reading and writing the fp32 states.
  --workload dispatch the forward at shapes around its dispatch boundaries
                      (40-224 (sequence, head) pairs), every choice forced
                      and the library's own; a table, not a metric line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kda-ascendc_amd"))

from kda_bt16 import (  # noqa: E402
    forward_choice, kda_bt16_fwd, kda_bt16_stage_launchers, kda_decode_step, kda_recurrent_fwd)

METRIC = "KDA fwd tokens/sec and ms at B=1 T=8192 H=32 bf16; % HBM/MFMA roofline"
B, T, H, D = 1, 8192, 32, 128
LOWER_BOUND = -5.0
SCALE = D ** -0.5
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3
# Published reference latency for this shape (Ascend 910B3, README.md:53): 20.5 ms.
REF_MS = 20.5

# shape, initial state (None: not passed; "zeros": a
# zero tensor passed; a float: ~N(0, std)) and the std of g_raw.
CONFIGS = {
    "c0": dict(B=2, T=1024, H=4, h0="zeros", g_std=1.0),
    "c1": dict(B=2, T=4096, H=8, h0=0.05, g_std=1.0),
    "c2": dict(B=1, T=8192, H=32, h0=None, g_std=1.0),
    "c3": dict(B=1, T=8192, H=96, h0=None, g_std=1.0),
    "c4": dict(B=16, T=2048, H=32, h0=0.05, g_std=2.0),
}


def make_inputs(seed: int = 42, cfg: dict | None = None):
    """BASELINE.json generators on the CPU: seed 42, order q, k, v, g_raw,
    beta_raw (N(0,1), g_raw std ``g_std``, stored bf16), A_log = log U(1,16),
    dt_bias ~N(0,0.1), then h0 ~N(0, std) when the config has one."""
    c = CONFIGS["c2"] if cfg is None else cfg
    b, t, h = c["B"], c["T"], c["H"]
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, t, h, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, t, h, D, generator=gen).to(torch.bfloat16)
    g = (torch.randn(b, t, h, D, generator=gen) * c["g_std"]).to(torch.bfloat16)
    beta = torch.randn(b, t, h, generator=gen).to(torch.bfloat16)
    A_log = torch.log(torch.rand(h, generator=gen) * 15.0 + 1.0)
    dt_bias = torch.randn(h * D, generator=gen) * 0.1
    if cfg is None:
        return q, k, v, g, beta, A_log, dt_bias
    h0 = None
    if c["h0"] == "zeros":
        h0 = torch.zeros(b, h, D, D)
    elif c["h0"] is not None:
        h0 = torch.randn(b, h, D, D, generator=gen) * c["h0"]
    return q, k, v, g, beta, A_log, dt_bias, h0


def algorithmic_bytes(n_states: int = B, b: int = B, t: int = T, h: int = H, h0: bool = False):
    """Algorithmic HBM bytes of one forward, split by the kernel that moves
    them: stage 1 reads q, k, v (2 B), g (2 B), beta (2 B) per token-head
    element plus A_log/dt_bias; stage 2 reads the fp32 initial state (when
    one is passed) and writes o (2 B) and the fp32 final state of each of
    ``n_states`` sequences.  Total = 1282 B per token-head + states."""
    nth = b * t * h
    k1 = nth * (3 * D * 2 + D * 2 + 2) + h * (4 + 4 * D)
    k2 = nth * D * 2 + n_states * h * D * D * 4 * (1 + int(h0))
    return k1, k2


def matmul_flops(n_chunks: int | None = None, b: int = B, t: int = T, h: int = H):
    """Matrix-op FLOPs of one forward per kernel: stage 1 the two fp32 grams
    and the two bf16 products of w and u; stage 2 w @ hc^T, qg @ hc^T,
    kg^T @ v_new and Aqk @ v_new."""
    nch = b * h * math.ceil(t / 16) if n_chunks is None else h * n_chunks
    k1 = nch * 4 * (2 * 16 * 16 * D)
    k2 = nch * (3 * (2 * 16 * D * D) + 2 * 16 * 16 * D)
    return k1, k2


TRAIN_TRAFFIC_FILE = ROOT / "profiles" / "kda_train_B1_T8192_H32_traffic.json"


def _profile(kind: str, b: int, t: int, h: int):
    """A committed rocprofv3 summary (profiles/kda_fwd_B{b}_T{t}_H{h}_{kind}.json),
    or None."""
    try:
        return json.loads((ROOT / "profiles" / f"kda_fwd_B{b}_T{t}_H{h}_{kind}.json").read_text())
    except (OSError, ValueError):
        return None


def measured_traffic(b: int = B, t: int = T, h: int = H):
    """HBM bytes per launch of each kernel from the committed rocprofv3 PMC
    summary (FETCH_SIZE x fetch scale + WRITE_SIZE x write scale, KiB), or
    None when no summary is present."""
    d = _profile("traffic", b, t, h)
    if d is None:
        return None
    out = {}
    for name, kb in d.get("kernels", {}).items():
        out[name] = int(round((kb["FETCH_SIZE_KiB"] * d["fetch_scale"]
                               + kb["WRITE_SIZE_KiB"] * d["write_scale"]) * 1024))
    return out


def measured_mfma(kern: dict, b: int = B, t: int = T, h: int = H):
    """Matrix-op work of each kernel from the committed rocprofv3 counter
    summary: SQ_INSTS_VALU_MFMA_MOPS_BF16 / _F32 count 512 FLOPs each, so
    FLOPs per launch = MOPS x 512; divided by the kernel's time measured
    here, that is the achieved rate and its fraction of the dense peak.
    SQ_VALU_MFMA_BUSY_CYCLES (summed over every SIMD) over the kernel's cycles
    times the SIMD count (GRBM_GUI_ACTIVE, summed over the XCDs, / XCDs x
    CUs x 4) is the fraction of the matrix pipes' time they were busy.  None
    when no summary is present."""
    d = _profile("mfma", b, t, h)
    if d is None:
        return None
    out = {}
    for name, c in d.get("kernels", {}).items():
        if name not in kern:
            continue
        ms = kern[name]["ms"]
        bf = c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512
        f32 = c["SQ_INSTS_VALU_MFMA_MOPS_F32"] * 512
        out[name] = {
            "bf16_flops": int(bf), "f32_flops": int(f32),
            "bf16_tflops": round(bf / ms / 1e9, 2),
            "bf16_frac": round(bf / ms / 1e9 / BF16_PEAK_TFLOPS, 5),
            "f32_tflops": round(f32 / ms / 1e9, 2),
            "f32_frac": round(f32 / ms / 1e9 / F32_PEAK_TFLOPS, 5),
            "mfma_busy_frac": round(c["SQ_VALU_MFMA_BUSY_CYCLES"]
                                    / (c["GRBM_GUI_ACTIVE"] / d["xcds"] * d["cus"]
                                       * d["simds_per_cu"]), 5),
        }
    return out


STAGE_REPS = 100  # minimum launches when a stage is timed on its own


def time_events(fn, reps: int) -> float:
    """Average ms per call over ``reps`` calls, HIP events on the current stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def cpu_baseline(inputs, min_seconds: float = 10.0, max_reps: int = 30) -> dict:
    """The CPU restatement of the reference chunked path (oracle/kda_oracle.py),
    timed on this host's cores over the full workload, repeated until about
    ``min_seconds`` of CPU work (at most ``max_reps`` forwards); the value is
    the median repetition."""
    sys.path.insert(0, str(ROOT / "oracle"))
    from kda_oracle import chunked_reference  # checker/baseline only, never the product

    q, k, v, g, beta, A_log, dt_bias = inputs
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    # warm up on a small slice
    chunked_reference(q[:, :64, :2], k[:, :64, :2], v[:, :64, :2], g[:, :64, :2].float(),
                      beta[:, :64, :2].float(), SCALE, A_log=A_log[:2], dt_bias=dt_bias[:2 * D],
                      lower_bound=LOWER_BOUND)
    times = []
    while sum(times) < min_seconds and len(times) < max_reps:
        t0 = time.perf_counter()
        chunked_reference(q, k, v, g.float(), beta.float(), SCALE, A_log=A_log, dt_bias=dt_bias,
                          lower_bound=LOWER_BOUND)
        times.append(time.perf_counter() - t0)
    dt = statistics.median(times)
    cpu_model = platform.processor() or ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": B * T / dt,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full workload B={B} T={T} H={H}: {len(times)} forwards in "
                  f"{sum(times):.1f} s, median {dt:.3f} s; torch CPU fp32 with the reference's "
                  f"bf16 rounding points; {cpu_model}",
    }


VARLEN_N = 16


def varlen_offsets(seed: int = 7) -> list[int]:
    """16 sequences over the 8192 tokens, lengths uneven (16 cut points drawn
    uniformly, so most lengths are not multiples of 16)."""
    gen = torch.Generator().manual_seed(seed)
    cuts = sorted(set(torch.randint(1, T, (VARLEN_N - 1,), generator=gen).tolist()))
    while len(cuts) < VARLEN_N - 1:  # distinct cut points
        cuts = sorted(set(cuts + torch.randint(1, T, (1,), generator=gen).tolist()))
    return [0] + cuts + [T]


KERNEL_LABELS = {
    "k1": "stage 1 (k1_kernel)",
    "k2": "stage 2 (k2_kernel, or k2s_kernel / k2w_kernel where one-tile work-groups would "
          "outnumber the CUs)",
    "fused": "fused_kernel (stage 1's records kept in LDS), the forward's one launch",
}


def _dominant_roofline(kern, traffic, alg_bytes, flops, fwd_ms, fused, launches: int = 1) -> dict:
    """The roofline of the forward's dominant (longest) kernel: the
    algorithmic bytes of one of its launches over its mean launch time, HIP
    events on the stream it runs on (stage launches timed on their own just
    before the timed region; a fused forward is its one launch), and its
    HBM bytes per launch from rocprof's FETCH_SIZE / WRITE_SIZE scaled by the
    copy calibration.  A forward whose two stages run in `launches` chunk
    ranges launches each stage that many times, each launch over 1/launches
    of the chunks and of the algorithmic bytes; `kern` then holds one
    launch's time.  The same figures for the whole forward (all its launches
    over the timed region's mean forward time) are under ``forward``."""
    dom = max(kern, key=lambda n: kern[n]["ms"])
    dom_ms = kern[dom]["ms"]
    achieved = alg_bytes / launches / dom_ms / 1e6
    fwd_achieved = alg_bytes / fwd_ms / 1e6
    have = traffic is not None and all(n in traffic for n in kern)
    return {
        "bound": "hbm",
        "kernel": KERNEL_LABELS[dom],
        "achieved": round(achieved, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 5),
        "traffic": traffic.get(dom) if traffic else None,
        "kernel_ms_events": round(dom_ms, 5),
        "launches_per_forward": launches,
        "alg_bytes": alg_bytes,
        "rule": "achieved = the forward's algorithmic bytes / launches per forward / the dominant "
                "kernel's mean launch time (HIP events); traffic = that kernel's HBM bytes per "
                "launch (rocprof)",
        "forward": {
            "kernels": (KERNEL_LABELS["fused"] if fused else
                        "stage 1 then stage 2, one launch each" if launches == 1 else
                        f"stage 1 then stage 2 on each of {launches} chunk ranges"),
            "ms_events": round(fwd_ms, 5),
            "achieved": round(fwd_achieved, 2),
            "frac": round(fwd_achieved / HBM_PEAK_GBS, 5),
            "traffic": launches * sum(traffic[n] for n in kern) if have else None,
            "matmul_flops": flops,
            "alg_tflops": round(flops / fwd_ms / 1e9, 2),
            "alg_mfma_frac": round(flops / fwd_ms / 1e9 / BF16_PEAK_TFLOPS, 5),
        },
        "kernels": {n: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                        for kk, vv in d.items()} for n, d in kern.items()},
    }


def _kernel_roofline(k1_ms, k2_ms, wall_ms, by, fl):
    by1, by2 = by
    fl1, fl2 = fl
    kern = {
        "k1": {"ms": k1_ms, "alg_bytes": by1, "alg_gbs": by1 / k1_ms / 1e6,
               "tflops": fl1 / k1_ms / 1e9},
        "k2": {"ms": k2_ms, "alg_bytes": by2, "alg_gbs": by2 / k2_ms / 1e6,
               "tflops": fl2 / k2_ms / 1e9},
    }
    dom = "k1" if k1_ms >= k2_ms else "k2"
    return kern, dom


def run_varlen(args, dev, inputs_cpu) -> dict:
    q, k, v, g, beta, A_log, dt_bias = (x.to(dev) for x in inputs_cpu)
    offs = varlen_offsets()
    cu = torch.tensor(offs, dtype=torch.int64, device=dev)
    kw = dict(scale=SCALE, output_final_state=True, use_qk_l2norm_in_kernel=True,
              use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
              lower_bound=LOWER_BOUND, A_log=A_log, dt_bias=dt_bias)

    def step():
        return kda_bt16_fwd(q, k, v, g, beta, cu_seqlens=cu, **kw)

    k1, k2, _, _ = kda_bt16_stage_launchers(q, k, v, g, beta, output_final_state=True,
                                            A_log=A_log, dt_bias=dt_bias,
                                            lower_bound=LOWER_BOUND, cu_seqlens=cu)
    k1(); k2()
    reps = max(args.steps, STAGE_REPS)
    k1_ms, k2_ms = time_events(k1, reps), time_events(k2, reps)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    fwd_ms = ev0.elapsed_time(ev1) / args.steps
    lens = [b - a for a, b in zip(offs[:-1], offs[1:])]
    n_chunks = sum(math.ceil(n / 16) for n in lens)
    by = algorithmic_bytes(VARLEN_N)
    fl = matmul_flops(n_chunks)
    kern, _ = _kernel_roofline(k1_ms, k2_ms, wall_ms, by, fl)
    fused = k1.forward_plan == "fused"
    stage_ms = None
    if fused:
        stage_ms = {n: round(d["ms"], 4) for n, d in kern.items()}
        kern = {"fused": {"ms": fwd_ms, "alg_bytes": sum(by), "alg_gbs": sum(by) / fwd_ms / 1e6,
                          "tflops": sum(fl) / fwd_ms / 1e9}}
    traffic = None
    try:
        t = json.loads((ROOT / "profiles" / "kda_varlen_T8192_N16_H32_traffic.json").read_text())
        traffic = {n: int(round((kb["FETCH_SIZE_KiB"] * t["fetch_scale"]
                                 + kb["WRITE_SIZE_KiB"] * t["write_scale"]) * 1024))
                   for n, kb in t["kernels"].items()}
    except (OSError, ValueError, KeyError):
        pass
    roofline = _dominant_roofline(kern, traffic, sum(by), sum(fl), fwd_ms, fused)
    if fused:
        # the two stages on the same inputs, each timed on its own (the
        # forward does not run them here)
        roofline["two_stage_kernels_ms"] = stage_ms
    return {
        "metric": "KDA varlen fwd tokens/sec, 8192 tokens in 16 packed sequences, H=32 bf16",
        "value": round(T / (wall_ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"kda_bt16_fwd cu_seqlens, {VARLEN_N} sequences over T={T}, "
                               f"H={H}, lengths {lens}", "seq_len": T, "heads": H,
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline,
    }


def bwd_algorithmic_bytes():
    """Algorithmic HBM bytes of one backward: it reads q, k, v, g, beta and
    dO (2 B per element, 2 B of beta) and writes dq, dk, dv, dg (2 B) and
    dbeta (2 B) per token-head, plus A_log / dt_bias and their gradients:
    2308 B per token-head."""
    nth = B * T * H
    return nth * (5 * D * 2 + 2 + 4 * D * 2 + 2) + 2 * H * (4 + 4 * D)


def bwd_matmul_flops():
    """Matrix-op FLOPs of one backward per chunk-head: the recompute (the
    forward's 1,900,544), the state-gradient chain (Aqk^T dO, kg dh', and the
    32-deep update of dh: 1,638,400) and the per-chunk products (dO h^T,
    dv_new h^T, v_new dh'^T, dO v_new^T, and the fp32 grams and 16-deep
    products of the intra-chunk gradients: 1,900,544)."""
    nch = B * H * math.ceil(T / 16)
    recompute = 4 * (2 * 16 * 16 * D) + 3 * (2 * 16 * D * D) + 2 * 16 * 16 * D
    chain = 2 * 16 * 16 * D + 2 * 16 * D * D + 2 * D * 32 * D
    chunk = 3 * (2 * 16 * D * D) + 2 * 16 * 16 * D + 3 * (2 * 16 * 16 * D) + 5 * (2 * 16 * 16 * D)
    return nch * (recompute + chain + chunk)


def run_train(args, dev, inputs_cpu) -> dict:
    """One training step of the op: kda_bt16_fwd with inputs that require
    grad (the training forward, which keeps the per-chunk state), then the
    backward through autograd (from that state: the state-gradient chain,
    the per-chunk gradients).  The step with the recompute policy
    (set_backward_recompute) is timed beside it."""
    from kda_bt16 import set_backward_recompute

    ins = [x.to(dev) for x in inputs_cpu]
    leaves = [t.detach().clone().requires_grad_(True) for t in ins]
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(B, T, H, D, generator=gen).to(torch.bfloat16).to(dev)
    flags = dict(scale=SCALE, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                 use_beta_sigmoid_in_kernel=True, lower_bound=LOWER_BOUND)

    def step():
        for t in leaves:
            t.grad = None
        o, _ = kda_bt16_fwd(*leaves[:5], A_log=leaves[5], dt_bias=leaves[6], **flags)
        o.backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    reps = max(args.steps, 10)
    # the two halves, with HIP events: the training forward, and the
    # backward over one saved state (torch.autograd.grad: no accumulation)
    fwd = lambda: kda_bt16_fwd(*leaves[:5], A_log=leaves[5], dt_bias=leaves[6], **flags)
    fwd_ms = time_events(fwd, reps)
    o, _ = fwd()
    bwd_ms = time_events(lambda: torch.autograd.grad(o, leaves, do, retain_graph=True), reps)
    del o
    try:
        set_backward_recompute(True)
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            step()
        torch.cuda.synchronize()
        recompute_ms = (time.perf_counter() - t0) * 1e3 / reps
    finally:
        set_backward_recompute(False)
    by = bwd_algorithmic_bytes()
    fl = bwd_matmul_flops()
    achieved = by / bwd_ms / 1e6
    # HBM bytes of one saved-state backward (its five launches), from the
    # FETCH_SIZE / WRITE_SIZE runs scaled by the copy calibration
    traffic = None
    if TRAIN_TRAFFIC_FILE.exists():
        t = json.loads(TRAIN_TRAFFIC_FILE.read_text())
        traffic = round(sum((t["kernels"][n]["FETCH_SIZE_KiB"] * t["fetch_scale"]
                             + t["kernels"][n]["WRITE_SIZE_KiB"] * t["write_scale"]) * 1024
                            for n in t["backward_kernels"]))
    return {
        "metric": "KDA training step (fwd + bwd) tokens/sec at B=1 T=8192 H=32 bf16",
        "value": round(B * T / (wall_ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"kda_bt16_fwd + autograd backward B={B} T={T} H={H} K=V={D}, "
                               "zero h0, all in-kernel flags, dO ~N(0,1)",
                   "global_batch": B, "seq_len": T, "heads": H, "parallelism": "none (1 GPU)"},
        "recompute_ms_per_step": round(recompute_ms, 4),
        "roofline": {"bound": "hbm",
                     "kernel": "backward from the saved state (kda_bt16_bwd_saved_hip, 5 launches)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic,
                     "bwd_ms": round(bwd_ms, 4), "fwd_ms": round(fwd_ms, 4),
                     "bwd_alg_bytes": by, "bwd_matmul_flops": fl,
                     "bwd_tflops": round(fl / bwd_ms / 1e9, 2),
                     "bwd_mfma_frac": round(fl / bwd_ms / 1e9 / BF16_PEAK_TFLOPS, 5)},
    }


DEC_B = 128


def run_decode(args, dev) -> dict:
    """One decode step for DEC_B sequences x H heads, the state updated in
    place (kda_decode_step).  Algorithmic bytes per (sequence, head): the
    fp32 state read and written (2 x 64 KiB), q, k, v, o (4 x 256 B), g
    (512 B fp32), beta (4 B)."""
    gen = torch.Generator().manual_seed(11)
    q = torch.randn(DEC_B, 1, H, D, generator=gen).bfloat16().to(dev)
    k = torch.randn(DEC_B, 1, H, D, generator=gen).bfloat16().to(dev)
    v = torch.randn(DEC_B, 1, H, D, generator=gen).bfloat16().to(dev)
    g = torch.randn(DEC_B, 1, H, D, generator=gen).to(dev)
    beta = torch.randn(DEC_B, 1, H, generator=gen).to(dev)
    A_log = torch.log(torch.rand(H, generator=gen) * 15.0 + 1.0).to(dev)
    dt_bias = (torch.randn(H * D, generator=gen) * 0.1).to(dev)
    state = (torch.randn(DEC_B, H, D, D, generator=gen) * 0.05).to(dev)
    kw = dict(scale=SCALE, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=LOWER_BOUND, A_log=A_log,
              dt_bias=dt_bias)

    def step():
        return kda_decode_step(q, k, v, g, beta, state, **kw)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ev_ms = time_events(step, max(args.steps, 10))
    per = 2 * D * D * 4 + 4 * D * 2 + D * 4 + 4
    alg = DEC_B * H * per
    achieved = alg / ev_ms / 1e6
    return {
        "metric": "KDA decode step tokens/sec, B=128 sequences x H=32, fp32 state in place",
        "value": round(DEC_B / (wall_ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"kda_decode_step B={DEC_B} T=1 H={H} K=V={D}, V-first fp32 "
                               "state updated in place, all in-kernel flags",
                   "global_batch": DEC_B, "seq_len": 1, "heads": H,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "recurrent", "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": None,
                     "kernel_ms": round(ev_ms, 5), "alg_bytes": alg},
    }


# (B, T, H) shapes around the forward's dispatch boundaries: stage-2 value
# tiles per work-group (1, 2, 4, 8) and fused against two stages.
DISPATCH_SHAPES = [(1, 4096, 40), (1, 4096, 48), (1, 4096, 64), (1, 4096, 80), (1, 4096, 128),
                   (1, 4096, 160), (1, 4096, 192), (1, 4096, 224), (1, 2048, 160), (1, 2048, 224)]


def run_dispatch(args, dev) -> dict:
    """The forward at each DISPATCH_SHAPES shape with every choice forced
    through ``forward_choice`` (the C ABI's ``KDA_BT16_TWO_STAGE`` flag and
    ``k2_tiles`` field: 1, 2, 4 or 8 value tiles per stage-2 work-group;
    ``KDA_BT16_FUSED_KERNEL`` for the fused kernel) and with the library's
    own choice, HIP events over ``steps`` calls after ``warmup`` (µs per
    call), the faster of two rounds.  Every choice gives the same bits; this
    only measures which is fastest."""
    rows = []
    for B, T, Hs in DISPATCH_SHAPES:
        gen = torch.Generator(device=dev).manual_seed(3)
        q, k, v, g = (torch.randn(B, T, Hs, D, device=dev, generator=gen).bfloat16()
                      for _ in range(4))
        beta = torch.randn(B, T, Hs, device=dev, generator=gen).bfloat16()
        A_log = torch.log(torch.rand(Hs, device=dev, generator=gen) * 15.0 + 1.0)
        dt_bias = torch.randn(Hs * D, device=dev, generator=gen) * 0.1
        kw = dict(scale=SCALE, output_final_state=True, use_qk_l2norm_in_kernel=True,
                  use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                  lower_bound=LOWER_BOUND, A_log=A_log, dt_bias=dt_bias)

        def timed(**choice):
            fn = lambda: kda_bt16_fwd(q, k, v, g, beta, **kw)  # noqa: E731
            with forward_choice(**choice):
                for _ in range(args.warmup):
                    fn()
                return round(time_events(fn, args.steps) * 1e3, 1)

        row = {"B": B, "T": T, "H": Hs, "pairs": B * Hs}
        # two rounds over the choices, the faster of each choice's two timings:
        # a two-stage timing taken right after the fused kernel reads a few
        # percent slow, so the fused kernel comes last in each round
        choices = [(f"two_stage_{t}_tiles_us", dict(fused=False, k2_tiles=t)) for t in (1, 2, 4, 8)]
        choices += [("library_choice_us", {}), ("fused_us", dict(fused=True))]
        for _ in range(2):
            for key, choice in choices:
                t_us = timed(**choice)
                row[key] = min(row.get(key, t_us), t_us)
        rows.append(row)
        print(f"# {row}", file=sys.stderr, flush=True)
        del q, k, v, g, beta
    return {"workload": "forward dispatch: stage-2 value tiles and fused against two stages, "
                        "K=V=128 bf16, all in-kernel flags",
            "steps": args.steps, "warmup": args.warmup, "unit": "us per forward", "rows": rows,
            "varlen_rows": run_dispatch_varlen(args, dev)}


# Packed sequences (cu_seqlens, 32 heads) at or above the CU count of
# (sequence, head) pairs: one long sequence among short ones, and equal
# lengths.
DISPATCH_VARLEN = [("one_long", [16384] + [1024] * 7), ("equal", [2944] * 8),
                   ("one_long_16", [8192] + [512] * 15)]


def run_dispatch_varlen(args, dev) -> list:
    """The varlen forward at each DISPATCH_VARLEN batch: the two stages and
    the fused kernel forced, and the library's own choice without and with
    the ``max_seqlen`` hint (which the fused-or-not choice weighs against
    the longest sequence).  HIP events, µs per call, the faster of two
    rounds."""
    rows = []
    Hs = 32
    for name, lens in DISPATCH_VARLEN:
        cu_list = [0]
        for n in lens:
            cu_list.append(cu_list[-1] + n)
        T = cu_list[-1]
        gen = torch.Generator(device=dev).manual_seed(5)
        q, k, v, g = (torch.randn(1, T, Hs, D, device=dev, generator=gen).bfloat16()
                      for _ in range(4))
        beta = torch.randn(1, T, Hs, device=dev, generator=gen).bfloat16()
        A_log = torch.log(torch.rand(Hs, device=dev, generator=gen) * 15.0 + 1.0)
        dt_bias = torch.randn(Hs * D, device=dev, generator=gen) * 0.1
        cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
        kw = dict(scale=SCALE, output_final_state=True, use_qk_l2norm_in_kernel=True,
                  use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                  lower_bound=LOWER_BOUND, A_log=A_log, dt_bias=dt_bias, cu_seqlens=cu)

        def timed(choice, **over):
            fn = lambda: kda_bt16_fwd(q, k, v, g, beta, **kw, **over)  # noqa: E731
            with forward_choice(**choice):
                for _ in range(args.warmup):
                    fn()
                return round(time_events(fn, args.steps) * 1e3, 1)

        row = {"name": name, "lengths": lens, "T": T, "H": Hs, "pairs": len(lens) * Hs}
        choices = [("two_stage_us", dict(fused=False), {}),
                   ("library_choice_us", {}, {}),
                   ("library_choice_max_seqlen_us", {}, {"max_seqlen": max(lens)}),
                   ("fused_us", dict(fused=True), {})]
        for _ in range(2):
            for key, choice, over in choices:
                t_us = timed(choice, **over)
                row[key] = min(row.get(key, t_us), t_us)
        best = min(row["two_stage_us"], row["fused_us"])
        row["hinted_choice_within_3pct_of_best"] = row["library_choice_max_seqlen_us"] <= 1.03 * best
        rows.append(row)
        print(f"# {row}", file=sys.stderr, flush=True)
        del q, k, v, g, beta
    return rows


def precision_vs_recurrence(fwd_out, ins, kw) -> dict:
    """Max-abs error of o and ht against the token recurrence in fp32 on the
    GPU (kda_recurrent_fwd with an fp32 o: no rounding between tokens, the
    role of the reference tests' fused_recurrent_kda gold,
    tests/test_kda_bt16.py:26-38).  The tests check that recurrence against
    the CPU gold; the bar they apply at this shape is 1.5x the reference
    chunked path's own error (about 1.05e-3 for o and 6.1e-3 for ht at B=1
    T=8192 H=32)."""
    o, ht = fwd_out
    o_g, ht_g = kda_recurrent_fwd(*ins, output_dtype=torch.float32, **kw)
    return {
        "gold": "kda_recurrent_fwd, fp32 state and o, same inputs",
        "o_maxabs": float((o.float() - o_g).abs().max()),
        "ht_maxabs": float((ht - ht_g).abs().max()),
        "o_rel_rms": float((o.float() - o_g).pow(2).mean().sqrt() / o_g.pow(2).mean().sqrt()),
        "ht_rel_rms": float((ht - ht_g).pow(2).mean().sqrt() / ht_g.pow(2).mean().sqrt()),
    }


def run_forward(args, dev, name: str, *, cpu: bool, inputs_cpu=None) -> dict:
    """One BASELINE config: precision against the fp32 recurrence, the two
    stages timed with HIP events, then ``warmup`` forwards and exactly
    ``steps`` timed forwards (synchronized on both sides; HIP events on the
    launch stream bracket the same region)."""
    c = CONFIGS[name]
    b, t, h = c["B"], c["T"], c["H"]
    ins_cpu = make_inputs(cfg=c)
    q, k, v, g, beta, A_log, dt_bias, h0 = (None if x is None else x.to(dev) for x in ins_cpu)
    flags = dict(scale=SCALE, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                 use_beta_sigmoid_in_kernel=True, lower_bound=LOWER_BOUND, A_log=A_log,
                 dt_bias=dt_bias)
    kw = dict(initial_state=h0, output_final_state=True, **flags)

    def step():
        return kda_bt16_fwd(q, k, v, g, beta, **kw)

    # Untimed measurements first: precision, then each stage on its own.
    precision = precision_vs_recurrence(step(), (q, k, v, g, beta), kw)
    k1, k2, _, _ = kda_bt16_stage_launchers(q, k, v, g, beta, initial_state=h0,
                                            output_final_state=True, A_log=A_log,
                                            dt_bias=dt_bias, lower_bound=LOWER_BOUND)
    fused = k1.forward_plan == "fused"
    # A forward whose two stages run in chunk ranges launches each stage once
    # per range: time the first range's launches (the ranges are equal when
    # the chunks divide evenly), as the forward runs them.
    launches = max(1, k1.forward_segments)
    if launches > 1:
        rows = 16 * (((t + 15) // 16) // launches)  # the first range's tokens (16 a chunk)
        part = lambda x: x[:, :rows].contiguous()
        k1, k2, _, _ = kda_bt16_stage_launchers(part(q), part(k), part(v), part(g), part(beta),
                                                initial_state=h0, output_final_state=True,
                                                A_log=A_log, dt_bias=dt_bias,
                                                lower_bound=LOWER_BOUND)
    k1(); k2()
    # Each stage over at least 100 launches: a steadier figure than a few,
    # and ~30 ms of this work has run by the time the forward's own warmup
    # starts (with 20 launches each, a 20-step run measured the forward ~3 %
    # slower than a 50- or 200-step run).
    reps = max(args.steps, STAGE_REPS)
    k1_ms = time_events(k1, reps)
    k2_ms = time_events(k2, reps)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: synchronize on both sides, exactly `steps` forwards
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    fwd_ms = ev0.elapsed_time(ev1) / args.steps
    # per-call latency distribution with HIP events
    lat = sorted(time_events(step, 1) for _ in range(min(max(args.steps, 5), 50)))

    by1, by2 = algorithmic_bytes(b, b, t, h, h0 is not None)
    fl1, fl2 = matmul_flops(None, b, t, h)
    # per launch (1/launches of the forward's chunks)
    stage_kern = {
        "k1": {"ms": k1_ms, "alg_bytes": by1 / launches, "alg_gbs": by1 / launches / k1_ms / 1e6,
               "alg_tflops": fl1 / launches / k1_ms / 1e9},
        "k2": {"ms": k2_ms, "alg_bytes": by2 / launches, "alg_gbs": by2 / launches / k2_ms / 1e6,
               "alg_tflops": fl2 / launches / k2_ms / 1e9},
    }
    # The forward's kernels: one fused launch, or the two stages.
    kern = ({"fused": {"ms": fwd_ms, "alg_bytes": by1 + by2, "alg_gbs": (by1 + by2) / fwd_ms / 1e6,
                       "alg_tflops": (fl1 + fl2) / fwd_ms / 1e9}} if fused else stage_kern)
    traffic = measured_traffic(b, t, h)
    if traffic:
        for n in kern:
            if n in traffic:
                kern[n]["hbm_bytes"] = traffic[n]
                kern[n]["hbm_gbs"] = traffic[n] / kern[n]["ms"] / 1e6
    mfma = measured_mfma(kern, b, t, h)
    if mfma:
        for n, m in mfma.items():
            kern[n]["mfma"] = m
    tot_bytes = by1 + by2
    roofline = _dominant_roofline(kern, traffic, tot_bytes, fl1 + fl2, fwd_ms, fused,
                                  1 if fused else launches)
    roofline["alg_bytes_rule"] = "B*T*H*1282 + 65536*B*H*(h0 passed + ht) + 516*H"
    if fused:
        # the two stages on the same inputs, each timed on its own (the
        # forward does not run them here)
        roofline["two_stage_kernels_ms"] = {n: round(d["ms"], 4) for n, d in stage_kern.items()}
    h0_txt = {None: "no initial state", "zeros": "zero initial state passed"}.get(
        c["h0"], f"initial state ~N(0,{c['h0']})")
    result = {
        "metric": METRIC if name == "c2" else
        f"KDA fwd tokens/sec and ms at B={b} T={t} H={h} bf16 (BASELINE {name})",
        "value": round(b * t / (wall_ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"kda_bt16_fwd B={b} T={t} H={h} K=V={D} (BASELINE configs[{name[1]}]), "
                        f"{h0_txt}, g_raw std {c['g_std']}, final state out, all in-kernel flags",
            "global_batch": b,
            "seq_len": t,
            "heads": h,
            "parallelism": "none (1 GPU)",
        },
        # everything that runs on the GPU before the timed region: the
        # precision check (one forward and the fp32 recurrence), each stage
        # timed on its own (1 + reps launches each), then the warmup forwards
        "pre_timed_launches": {"forwards": 1 + args.warmup, "fp32_recurrence": 1,
                               "stage1": 1 + reps, "stage2": 1 + reps},
        "latency_ms": {"p20": round(lat[len(lat) // 5], 4),
                       "median": round(statistics.median(lat), 4),
                       "p80": round(lat[(4 * len(lat)) // 5], 4)},
        "roofline": roofline,
        "precision": {kk: (float(f"{vv:.4g}") if isinstance(vv, float) else vv)
                      for kk, vv in precision.items()},
    }
    if name == "c2":
        result["vs_baseline"] = round((b * t / (wall_ms / 1e3)) / (b * t / (REF_MS / 1e3)), 2)
        result["baseline_ref"] = ("reference kda_bt16_fwd 20.5 ms at this shape on Ascend "
                                  "910B3 (README.md:53)")
    if cpu:
        result["cpu_baseline"] = cpu_baseline(inputs_cpu if inputs_cpu is not None
                                              else make_inputs())
    return result


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 200 forwards are ~60 ms of timed work; 50 warmups bring the GPU to its
    # steady clocks first (20 steps after 5 warmups read ~6% slow).
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (3 launches), the reference "
                         "kernel for scaling rocprof FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--workload",
                    choices=("headline", "config", "varlen", "decode", "train", "dispatch"),
                    default="headline")
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c2",
                    help="BASELINE config of --workload config")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the forward shards over (batch, head) with no "
              "communication, so every GPU runs this same single-GPU workload on its share; "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.workload == "decode":
        print(json.dumps(run_decode(args, dev)), flush=True)
        return
    if args.workload == "dispatch":
        print(json.dumps(run_dispatch(args, dev)), flush=True)
        return
    inputs_cpu = make_inputs()
    if args.workload == "varlen":
        print(json.dumps(run_varlen(args, dev, inputs_cpu)), flush=True)
        return
    if args.workload == "train":
        print(json.dumps(run_train(args, dev, inputs_cpu)), flush=True)
        return
    if args.workload == "config":
        print(json.dumps(run_forward(args, dev, args.config, cpu=False)), flush=True)
        return
    print(json.dumps(run_forward(args, dev, "c2", cpu=not args.no_cpu_baseline,
                                 inputs_cpu=inputs_cpu)), flush=True)


if __name__ == "__main__":
    main()
