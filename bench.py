"""Benchmark of the INT8 DenseNet169 encoder on one MI355X (BASELINE.json metric: 512 px DenseNet169 INT8
slices/s on 1 MI355X; 24-slice study latency in ms).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (`value`): configuration 5, sustained throughput.  A step = one synthetic study: 2 seeded
DenseNet169 weight sets x 2 crops x 24 slices of 3 x 512 x 512 uint8 with flip TTA = one pass of 96
encoded images per seed (48 slices + their mirrors, the flip fused in the stem), i.e. 192 encoded
slices per step.  Inputs are resident in HBM: 50 distinct seeded studies (`synthetic.c5_study`, seeds
1234..1283), step k encoding study k mod 50 (K = 50 by default: every study once); each encoder
call replays its HIP graph.  value = 192 K / T slices/s.  `c5_all_studies`: the 50 studies once each,
back to back, after the timed steps.
`study_latency_ms`: configuration 4, one 24-slice study through one encoder (batch 24, one pass) and the
1664 -> 8 linear head on the device (`d8s_linear`), to the logits.
The two seeds' passes of a step run from two streams (`--serial`: one after the other).
`roofline`: the dominant kernel family: its launches of a configuration-5 pass recorded R times in a HIP
graph and replayed between HIP events on the encoder's stream (algorithmic bytes of a launch / the
average launch time); `frac_in_pass` the same family's share of a whole pass (the pass's graph against
the pass's graph without the family's launches, per launch), `in_schedule` what the family's launches
add to the two-stream pair of passes (partly filled by the other seed's work, so no roofline fraction
is derived from it); `roofline_runner_up`: the second family by time (the
band layers of block 0 and the chained launches of block 2 take about as long, so either can lead),
against HBM and the int8 MFMA peak; `step_hbm_frac`: both passes' algorithmic bytes over the timed
step time.  `roofline_c4`: configuration 4's dominant launch (the 32 x 32 banded block)
against the int8 MFMA peak.  `kernels`: configurations 2 and 3 case by case (`--path kernels` alone).
`cpu_baseline`: the float32 DenseNet169 forward (`oracle/fp32.py`) on the host cores at batch 1
(slices/s) and at batch 24 (one study, `study_latency_ms`).
`mfma_probe`: the int8 MFMA rate measured on the GPU (`d8s_micro_mfma`), beside the 5.0 POP/s datasheet
figure; `family_int8_frac_of_measured_peak` quotes each family's int8 rate against it.
`fp32_agreement`: max-abs, rel_l2 and minimum cosine of the configuration-4 study's INT8 features (and
of a seeded 1664 -> 8 linear head's logits) against the fp32 DenseNet169 forward of the same weights
(the package's `densenet` module in float32 on the GPU), with the reference's gate; under "c5" the
same for configuration 5's outputs (study 0, both seeds, plain and mirrored images).
`reference_study`: ms per study at the reference's own headline shape (88 images at 288 px, one
encoder, graph replay) beside the 34 ms the reference quotes for it on one T4.
`prep`: the upstream preparation (raw uint16 crops -> the uint8 volume of a study, `d8s_prep`) on the
same GPU, studies/s with the payloads resident in HBM.
One JSON line on stdout.

    python bench.py --path prep [--steps K] [--warmup W] [--no-cpu]

The preparation alone, one study per step (4 series x 2 crops x 24 slices at 512 px, slices 0:23),
with its own `roofline` (bytes of the whole d8s_prep launch sequence per study) and `cpu_baseline`
(the oracle's chain on one study).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import platform
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from rsna_knee_efficiency_amd import dense8s, densenet, synthetic  # noqa: E402
from rsna_knee_efficiency_amd import head as head_mod  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
I8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA, published
IMG = 512
SLICES = 24
C5_BLOCKS = [{"c0": 64, "h": 128, "w": 128, "L": 6, "trans": True},      # DenseNet169 at 512 px
             {"c0": 128, "h": 64, "w": 64, "L": 12, "trans": True},
             {"c0": 256, "h": 32, "w": 32, "L": 32, "trans": True},
             {"c0": 640, "h": 16, "w": 16, "L": 32, "trans": False}]
C5_STUDIES = 50                 # configuration 5 streams over 50 synthetic studies


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_encoder(seed: int, nb: int, dev: torch.device) -> tuple[dense8s.Dense8SEncoder, dense8s.SPlan]:
    model = densenet.seeded_densenet169(seed).to(dev)
    cal_x = synthetic.study_u8(64, IMG, seed=7)
    with torch.no_grad():
        cal = dense8s.calibrate(model, [synthetic.normalise(torch.from_numpy(c).to(dev))
                                        for c in np.split(cal_x, 8)])
    plan = dense8s.make_plan(model.cpu(), cal, IMG)
    enc = dense8s.Dense8SEncoder(dense8s.make_pack(plan, nb, input_kind="u8"), dev.index or 0, nb)
    return enc, plan


def agree(a: np.ndarray, b: np.ndarray) -> dict:
    """max-abs, rel_l2 and the minimum per-row cosine of a against b."""
    cos = (a * b).sum(1) / np.maximum(np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1), 1e-30)
    return {"max_abs": round(float(np.abs(a - b).max()), 5),
            "rel_l2": round(float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)), 5),
            "cos_min": round(float(cos.min()), 6)}


def kernel_bytes(meta: dict, n: int, kinds: dict | None = None) -> dict[str, list[float]]:
    """Algorithmic HBM bytes of every launch of a pass of n images, per kernel family: compulsory reads
    of the activations and writes of the outputs, plus the weights and tables (read once).  `kinds`
    {block: "conv" | "chain" | "tile" | "img" | "parts"} (`Dense8SEncoder.fused`): a fused layer
    ("dense") has no bottleneck in memory; a chained launch ("chain": conv2 of a layer and conv1 of the
    next) does not read the new layer's channels back; a whole block ("block") reads its input and
    writes its layers' outputs once."""
    kinds = kinds or {}
    out: dict[str, list[float]] = {"stem": [], "conv1": [], "conv2": [], "chain": [], "dense": [],
                                   "block": [], "trans": [], "final": []}
    img = meta["img"]
    out["stem"].append(n * 3 * img * img + n * 64 * (img // 4) ** 2 + 64 * 168 * 2 + 3 * 256 * 2)
    for bi, b in enumerate(meta["blocks"]):
        hw = b["h"] * b["w"]
        M = n * hw
        kind = str(kinds.get(bi, "conv")).split(":")[0]
        wts = 0
        for li in range(b["L"]):
            cin = b["c0"] + 32 * li
            w = 128 * cin + cin * 4 + 128 * 12 + 36864 + 32 * 8
            wts += w
            c1 = M * cin + M * 128 + 128 * cin + cin * 4 + 128 * 12
            c2 = M * 128 + M * 32 + 36864 + 32 * 8
            if kind == "tile":
                out["dense"].append(M * cin + M * 32 + w)
            elif kind == "conv":
                out["conv1"].append(c1)
                out["conv2"].append(c2)
            elif kind == "chain":
                # conv1 of layer 0, then per launch conv2 of layer li - 1 with conv1 of layer li (which
                # takes the 32 new channels from registers: M * 32 fewer bytes read), conv2 of the last
                if li == 0:
                    out["conv1"].append(c1)
                else:
                    out["chain"].append(M * 128 + M * 32 + 36864 + 32 * 8 + c1 - M * 32)
                if li == b["L"] - 1:
                    out["conv2"].append(c2)
        if kind in ("img", "parts"):
            out["block"].append(M * b["c0"] + M * 32 * b["L"] + wts)
        ctot = b["c0"] + 32 * b["L"]
        if b["trans"]:
            cout = ctot // 2
            out["trans"].append(M * ctot + (M // 4) * cout + cout * ctot + ctot * 4 + cout * 12)
        else:
            out["final"].append(M * ctot + n * ctot * 4 + ctot * 8)
    return {k: v for k, v in out.items() if v}


def kernel_ops(meta: dict, n: int, kinds: dict | None = None) -> dict[str, float]:
    """int8 MFMA operations (2 per MAC) of a pass, per family (the transition at quarter resolution)."""
    kinds = kinds or {}
    img = meta["img"]
    ops = {"stem": 2.0 * n * 64 * 147 * (img // 2) ** 2, "conv1": 0.0, "conv2": 0.0, "chain": 0.0,
           "dense": 0.0, "block": 0.0, "trans": 0.0}
    for bi, b in enumerate(meta["blocks"]):
        M = n * b["h"] * b["w"]
        kind = str(kinds.get(bi, "conv")).split(":")[0]
        for li in range(b["L"]):
            o1 = 2.0 * M * (b["c0"] + 32 * li) * 128
            o2 = 2.0 * M * 1152 * 32
            if kind == "conv":
                ops["conv1"] += o1
                ops["conv2"] += o2
            elif kind == "chain":
                ops["conv1" if li == 0 else "chain"] += o1
                ops["conv2" if li == b["L"] - 1 else "chain"] += o2
            else:
                ops["dense" if kind == "tile" else "block"] += o1 + o2
        if b["trans"]:
            ctot = b["c0"] + 32 * b["L"]
            ops["trans"] += 2.0 * (M // 4) * ctot * (ctot // 2)
    return {k: v for k, v in ops.items() if v}


def family_times(enc: dense8s.Dense8SEncoder, x: torch.Tensor, reps: int, mode) -> dict[str, float]:
    """Summed ms per kernel family of one pass (mean over reps), from HIP events between launches."""
    prof = enc.profile(x, reps=reps, flip=mode)
    fam: dict[str, float] = {}
    for tag, ms in prof.items():
        key = tag.rstrip("0123456789").rstrip("_")
        key = {"trans": "trans", "conv1": "conv1", "conv2": "conv2", "stem": "stem",
               "final": "final"}.get(key, key)
        fam[key] = fam.get(key, 0.0) + ms
    return fam


def copy_probe(dev: torch.device, mib: int = 1024, reps: int = 5) -> dict:
    """d8s_micro_copy over `mib` MiB (read + write): the practical HBM bandwidth, and the plain copy of
    known size that calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    from rsna_knee_efficiency_amd import hip
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    hip.call("d8s_micro_copy", src.data_ptr(), dst.data_ptr(), n, st)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        hip.call("d8s_micro_copy", src.data_ptr(), dst.data_ptr(), n, st)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return {"bytes_per_launch": 2 * n, "ms": round(ms, 4), "gbs": round(2 * n / (ms * 1e-3) / 1e9, 1)}


FAMILY = {"k_conv1": "conv1", "k_conv1p": "conv1", "k_conv2": "conv2", "k_c21": "chain", "k_dense": "dense",
          "k_band": "dense", "k_dblock": "block", "k_dparts": "block", "k_trans": "trans", "k_stem": "stem",
          "k_stem_rows": "stem", "k_final": "final", "k_copy": "copy", "k_prep_setup": "prep_setup",
          "k_prep_hist": "prep_hist", "k_prep_select": "prep_select", "k_prep_norm": "prep_norm",
          "k_prep_resize": "prep_resize"}


def _family(name: str) -> str | None:
    for k, v in FAMILY.items():
        if k + "<" in name or k + "(" in name:
            return v
    return None


def rocprof_summary(d: str) -> str:
    """Markdown summary of a rocprofv3 CSV output directory (kernel stats and/or counter collection),
    this library's kernels only."""
    import csv
    import glob
    lines = []
    for path in sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)):
        rows = [r for r in csv.DictReader(open(path)) if _family(r["Name"])]
        lines += [f"### kernel stats ({os.path.basename(path)})", "",
                  "| kernel | calls | avg us | total ms |", "|---|---|---|---|"]
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
            lines.append(f"| `{r['Name']}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                         f"{float(r['TotalDurationNs']) / 1e6:.3f} |")
        lines.append("")
    for path in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
        acc: dict = {}
        for r in csv.DictReader(open(path)):
            fam = _family(r.get("Kernel_Name", ""))
            if not fam:
                continue
            key = (r["Kernel_Name"], r["Counter_Name"])
            v = acc.setdefault(key, [0, 0.0])
            v[0] += 1
            v[1] += float(r["Counter_Value"])
        lines += [f"### counters ({os.path.basename(path)})", "",
                  "| kernel | counter | dispatches | mean per dispatch |", "|---|---|---|---|"]
        for (name, ctr), (cnt, tot) in sorted(acc.items()):
            lines.append(f"| `{name}` | {ctr} | {cnt} | {tot / cnt:.1f} |")
        lines.append("")
    for path in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
        lines += family_run_summary(path)
    return "\n".join(lines)


def family_run_summary(path: str) -> list[str]:
    """From a kernel trace of a bench.py run: the dispatches of the per-family timing (each family's
    launches of a configuration-5 pass replayed back to back, `Dense8SEncoder.time_families`): runs of
    consecutive dispatches of one family on one queue longer than any run of that family within a pass
    (a pass of the default kinds at 96 images, `kernel_bytes`), the first dispatch of each run not
    counted.  (A pass's own runs, e.g. the 31 chained launches of the 32 x 32 block, are left out: the
    two seeds' passes run concurrently.)  Runs are summed per family and the set of kernels (name and
    template arguments) they hold, so the 64 x 64 chain of the 24-image study does not mix into the
    32 x 32 chain of the 96-image pass.  Their mean duration is the average launch time behind
    bench.py's roofline."""
    import csv
    nb = 4 * SLICES
    per_pass = {k: len(v) for k, v in kernel_bytes({"img": IMG, "blocks": C5_BLOCKS}, nb,
                                                   dense8s.fused_blocks({"blocks": C5_BLOCKS, "n": nb})).items()}
    rows = [r for r in csv.DictReader(open(path)) if _family(r["Kernel_Name"])]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    runs: dict = {}                                   # queue -> [family, [durations], {kernels}]
    acc: dict = {}

    def close(run):
        fam, ds, names = run
        if fam != "copy" and len(ds) > per_pass.get(fam, 1):
            a = acc.setdefault((fam, ", ".join(f"`{k}`" for k in sorted(names))), [0, 0.0])
            a[0] += len(ds) - 1
            a[1] += sum(ds[1:])

    for r in rows:
        name = r["Kernel_Name"]
        fam = _family(name)
        q = r["Queue_Id"]
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        run = runs.get(q)
        if run is None or run[0] != fam:
            if run is not None:
                close(run)
            run = runs[q] = [fam, [], set()]
        run[1].append(us)
        run[2].add(name.split("(")[0].replace("void ", "").strip())
    for run in runs.values():
        close(run)
    out = [f"### family timing dispatches ({os.path.basename(path)})", "",
           "Runs of dispatches of one family on one queue longer than the family's runs within a pass "
           "(the back-to-back replays of the per-family timing; the first launch of each run not "
           "counted), by the kernels a run holds.", "", "| family | kernels | dispatches | mean us |",
           "|---|---|---|---|"]
    for (fam, kerns), (n, us) in sorted(acc.items()):
        out.append(f"| {fam} | {kerns} | {n} | {us / n:.2f} |")
    return out + [""]


TRAFFIC_FILE = ROOT / "profiles" / "encoder_c5_hbm_traffic.md"


def traffic_summary(fetch_dir: str, write_dir: str, passes: int, copy_bytes: int = 1 << 30) -> str:
    """HBM bytes per launch of every kernel family from two counter runs of `bench.py --pmc-passes P
    --copy-probe` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the counter
    reads for k_copy (1 GiB read + 1 GiB written per dispatch)."""
    import csv
    import glob

    def collect(d: str, counter: str) -> dict:
        acc: dict = {}
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                fam = _family(r.get("Kernel_Name", ""))
                if fam and r["Counter_Name"] == counter:
                    v = acc.setdefault(fam, [0, 0.0])
                    v[0] += 1
                    v[1] += float(r["Counter_Value"]) * 1024
        return acc

    fe, wr = collect(fetch_dir, "FETCH_SIZE"), collect(write_dir, "WRITE_SIZE")
    kf = copy_bytes / (fe["copy"][1] / fe["copy"][0])
    kw = copy_bytes / (wr["copy"][1] / wr["copy"][0])
    nb = 4 * SLICES
    meta_blocks = C5_BLOCKS
    alg = kernel_bytes({"img": IMG, "blocks": meta_blocks}, nb,
                       dense8s.fused_blocks({"blocks": meta_blocks, "n": nb}))
    lines = [f"Calibration: k_copy moves {copy_bytes} B read + {copy_bytes} B written per dispatch; "
             f"FETCH_SIZE scale {kf:.3f}, WRITE_SIZE scale {kw:.3f}.", "",
             "| family | launches per pass | HBM read MB/launch | HBM write MB/launch | traffic MB/launch "
             "| algorithmic MB/launch | traffic / algorithmic |", "|---|---|---|---|---|---|---|"]
    machine = []
    for fam in ("conv1", "conv2", "chain", "dense", "block", "trans", "stem", "final"):
        if fam not in fe or fam not in wr or fam not in alg:
            continue
        n = len(alg[fam])
        rd = fe[fam][1] * kf / (passes * n)
        wt = wr[fam][1] * kw / (passes * n)
        a = sum(alg[fam]) / n
        lines.append(f"| {fam} | {n} | {rd / 1e6:.2f} | {wt / 1e6:.2f} | {(rd + wt) / 1e6:.2f} | "
                     f"{a / 1e6:.2f} | {(rd + wt) / a:.3f} |")
        machine.append(f"traffic_per_launch[{fam}] = {int(rd + wt)}")
    return "\n".join(lines + ["", "```", *machine, "```"])


def mfma_summary(pmc_dir: str, passes: int) -> str:
    """MFMA use per kernel family from one counter run of `bench.py --pmc-passes P` with
    `--pmc MfmaUtil GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_INSTS_VALU_MFMA_MOPS_F16`:
    MfmaUtil (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs, per dispatch) averaged with the
    dispatches' GRBM_GUI_ACTIVE as weights, and the MFMA operations issued (MOPS x 512) against the
    algorithmic int8 operations of the family (`kernel_ops`): above 1 where K steps are padded."""
    import csv
    import glob

    per: dict = {}
    for path in glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            fam = _family(r.get("Kernel_Name", ""))
            if not fam:
                continue
            d = per.setdefault(fam, {}).setdefault(r.get("Dispatch_Id", r.get("Correlation_Id", "")), {})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    nb = 4 * SLICES
    meta_blocks = C5_BLOCKS
    kinds = dense8s.fused_blocks({"blocks": meta_blocks, "n": nb})
    alg = kernel_ops({"img": IMG, "blocks": meta_blocks}, nb, kinds)
    lines = ["| family | dispatches | MFMA busy (% of SIMD cycles, weighted) | MFMA ops issued per pass (G) "
             "| algorithmic int8 ops per pass (G) | issued / algorithmic |", "|---|---|---|---|---|---|"]
    for fam in ("conv1", "conv2", "chain", "dense", "block", "trans", "stem"):
        if fam not in per:
            continue
        ds = list(per[fam].values())
        w = sum(d.get("GRBM_GUI_ACTIVE", 0.0) for d in ds)
        util = sum(d.get("MfmaUtil", 0.0) * d.get("GRBM_GUI_ACTIVE", 0.0) for d in ds) / w if w else 0.0
        ops = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0) + d.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0)
                  for d in ds) * 512 / passes
        a = alg.get(fam, 0.0)
        lines.append(f"| {fam} | {len(ds)} | {util:.1f} | {ops / 1e9:.1f} | {a / 1e9:.1f} | "
                     f"{ops / a if a else float('nan'):.3f} |")
    return "\n".join(lines)


def family_roofline(f: str, fam: dict, byts: dict, ops: dict) -> dict:
    """HBM and int8 MFMA roofline figures of a kernel family from its per-pass time (`time_families`),
    bytes (`kernel_bytes`) and operations (`kernel_ops`)."""
    launches = len(byts[f])
    avg_ms = fam[f] / launches
    gbs = sum(byts[f]) / launches / (avg_ms * 1e-3) / 1e9
    tops = ops.get(f, 0.0) / (fam[f] * 1e-3) / 1e12
    return {"kernel": f"d8s_{f} (all {launches} launches of a pass)", "bound": "hbm",
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "avg_launch_ms": round(avg_ms, 5), "algorithmic_bytes_per_launch": int(sum(byts[f]) / launches),
            "int8_tops": round(tops, 1), "frac_mfma_datasheet": round(tops / I8_PEAK_TOPS, 4)}


def c4_summary(trace_csv: str) -> str:
    """Per-pass kernel times of a configuration-4 kernel trace (`rocprofv3 --kernel-trace` of
    `bench.py --c4-passes P`): the trace split into passes at every stem dispatch, the segments holding
    one final-features dispatch and a transition kept (whole passes of the graph replays), then per
    kernel the median over passes of its launches and microseconds."""
    import csv
    import statistics

    rows = [r for r in csv.DictReader(open(trace_csv)) if _family(r["Kernel_Name"])]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    segs, cur = [], None
    for r in rows:
        fam = _family(r["Kernel_Name"])
        if fam == "stem":
            cur = []
            segs.append(cur)
        if cur is not None:
            cur.append(r)
    passes = [sg for sg in segs if sum(_family(r["Kernel_Name"]) == "final" for r in sg) == 1
              and any(_family(r["Kernel_Name"]) == "trans" for r in sg)]
    if not passes:
        return "no whole pass in the trace"
    per: dict = {}
    spans = []
    for sg in passes:
        spans.append((int(sg[-1]["End_Timestamp"]) - int(sg[0]["Start_Timestamp"])) / 1e3)
        acc: dict = {}
        for r in sg:
            k = r["Kernel_Name"].split("(")[0].replace("void ", "")
            a = acc.setdefault(k, [0, 0.0])
            a[0] += 1
            a[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        for k, (n, us) in acc.items():
            per.setdefault(k, []).append((n, us))
    lines = [f"{len(passes)} whole passes; median pass span {statistics.median(spans):.1f} us", "",
             "| kernel | family | launches per pass | us per pass |", "|---|---|---|---|"]
    tot = 0.0
    for k, v in sorted(per.items(), key=lambda kv: -statistics.median(us for _, us in kv[1])):
        med = statistics.median(us for _, us in v)
        tot += med
        lines.append(f"| `{k}` | {_family(k + '(')} | {int(statistics.median(n for n, _ in v))} | {med:.1f} |")
    lines += ["", f"sum of the per-kernel medians: {tot:.1f} us per pass"]
    return "\n".join(lines)


def _dispatch_counters(d: str) -> dict:
    """{(kernel base name, dispatch id): {counter: value}} of every library dispatch in a rocprofv3
    counter-collection output directory."""
    import csv
    import glob
    out: dict = {}
    for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            name = r.get("Kernel_Name", "")
            if not _family(name):
                continue
            key = (name.split("(")[0].replace("void ", ""), r.get("Dispatch_Id", r.get("Correlation_Id", "")))
            c = out.setdefault(key, {})
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def c4_counter_summary(fetch_dir: str, write_dir: str, mfma_dir: str, wave_dir: str, passes: int,
                       copy_bytes: int = 1 << 30) -> str:
    """Configuration 4's banded whole-block launches (k_dparts, blocks 2 and 3 of a 24-image pass) from
    four counter runs of `bench.py --pmc-passes P --pmc-nb 24 --copy-probe` (FETCH_SIZE; WRITE_SIZE;
    MfmaUtil GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_I8; WAVE_COUNTERS): per kernel the HBM bytes per
    launch (scaled by k_copy's reading, as `traffic_summary`) against the algorithmic bytes
    (`block_work`), the MFMA busy fraction and issued operations against the algorithmic ones, and
    where the waves' cycles go."""
    fe, wr, mf, wv = (_dispatch_counters(d) for d in (fetch_dir, write_dir, mfma_dir, wave_dir))

    def per_kernel(tab: dict, counter: str) -> dict:
        acc: dict = {}
        for (k, _), c in tab.items():
            if counter in c:
                a = acc.setdefault(k, [0, 0.0])
                a[0] += 1
                a[1] += c[counter]
        return acc

    cf, cw = per_kernel(fe, "FETCH_SIZE"), per_kernel(wr, "WRITE_SIZE")
    kf = copy_bytes / (cf["k_copy"][1] * 1024 / cf["k_copy"][0])
    kw = copy_bytes / (cw["k_copy"][1] * 1024 / cw["k_copy"][0])
    n = SLICES
    kinds = dense8s.fused_blocks({"blocks": C5_BLOCKS, "n": n})
    work = {}
    for bi, b in enumerate(C5_BLOCKS):
        if str(kinds[bi]).startswith("parts:"):
            pt = b["h"] // int(kinds[bi].split(":")[1]) * b["w"] // 32
            work[f"k_dparts<{pt}>"] = (bi, kinds[bi]) + block_work(b, n)
    lines = [f"Calibration: k_copy moves {copy_bytes} B read + {copy_bytes} B written per dispatch; "
             f"FETCH_SIZE scale {kf:.3f}, WRITE_SIZE scale {kw:.3f}.", "",
             "| kernel | block (kind) | launches | HBM read MB | HBM write MB | traffic / algorithmic "
             "| MFMA busy % | MFMA ops issued (G) | algorithmic ops (G) | waiting % | ready, not issued % "
             "| issuing % | VALU issuing % |", "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for k, (bi, kind, byts, ops) in sorted(work.items()):
        if k not in cf or k not in cw:
            continue
        cnt = cf[k][0]
        rd = cf[k][1] * 1024 * kf / cnt
        wt = cw[k][1] * 1024 * kw / cw[k][0]
        ds = [c for (kk, _), c in mf.items() if kk == k]
        w = sum(c.get("GRBM_GUI_ACTIVE", 0.0) for c in ds)
        util = sum(c.get("MfmaUtil", 0.0) * c.get("GRBM_GUI_ACTIVE", 0.0) for c in ds) / w if w else 0.0
        issued = sum(c.get("SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0) for c in ds) * 512 / max(len(ds), 1)
        wsum: dict = {}
        for (kk, _), c in wv.items():
            if kk == k:
                for name, v in c.items():
                    wsum[name] = wsum.get(name, 0.0) + v
        cyc = wsum.get("SQ_WAVE_CYCLES", 0.0) or float("nan")
        pct = lambda c: 100.0 * wsum.get(c, 0.0) / cyc  # noqa: E731
        lines.append(f"| `{k}` | {bi} ({kind}) | {cnt} | {rd / 1e6:.2f} | {wt / 1e6:.2f} | {(rd + wt) / byts:.3f} "
                     f"| {util:.1f} | {issued / 1e9:.1f} | {ops / 1e9:.1f} | {pct('SQ_WAIT_ANY'):.1f} "
                     f"| {pct('SQ_WAIT_INST_ANY'):.1f} | {pct('SQ_ACTIVE_INST_ANY'):.1f} "
                     f"| {pct('SQ_ACTIVE_INST_VALU'):.1f} |")
    return "\n".join(lines)


WAVE_COUNTERS = ("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
                 "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_INSTS_VALU")


def wave_summary(pmc_dir: str) -> str:
    """Where the waves' cycles go, per kernel family, from one counter run of `bench.py --pmc-passes 1`
    with `--pmc` WAVE_COUNTERS: every counter summed over the family's dispatches; the percentages
    are of SQ_WAVE_CYCLES (the waves' resident cycles)."""
    import csv
    import glob

    per: dict = {}
    for path in glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            fam = _family(r.get("Kernel_Name", ""))
            if not fam or fam == "copy":
                continue
            f = per.setdefault(fam, {"dispatches": set()})
            f["dispatches"].add(r.get("Dispatch_Id", r.get("Correlation_Id", "")))
            f[r["Counter_Name"]] = f.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    lines = ["| family | dispatches | waves | cycles per wave | waiting on memory/counters (SQ_WAIT_ANY) "
             "| ready, not issued (SQ_WAIT_INST_ANY) | issuing (SQ_ACTIVE_INST_ANY) "
             "| VALU issuing (SQ_ACTIVE_INST_VALU) | VALU instructions per wave |",
             "|---|---|---|---|---|---|---|---|---|"]
    for fam in ("stem", "dense", "conv1", "conv2", "chain", "trans", "block", "final"):
        f = per.get(fam)
        if not f or not f.get("SQ_WAVES") or not f.get("SQ_WAVE_CYCLES"):
            continue
        wc = f["SQ_WAVE_CYCLES"]
        pct = lambda c: f"{100.0 * f.get(c, 0.0) / wc:.1f} %"  # noqa: E731
        lines.append(f"| {fam} | {len(f['dispatches'])} | {int(f['SQ_WAVES'])} | {wc / f['SQ_WAVES']:.0f} | "
                     f"{pct('SQ_WAIT_ANY')} | {pct('SQ_WAIT_INST_ANY')} | {pct('SQ_ACTIVE_INST_ANY')} | "
                     f"{pct('SQ_ACTIVE_INST_VALU')} | {f.get('SQ_INSTS_VALU', 0.0) / f['SQ_WAVES']:.0f} |")
    return "\n".join(lines)


def committed_traffic(family: str) -> int | None:
    """HBM bytes per launch of `family` from the committed counter summary (None if absent)."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith(f"traffic_per_launch[{family}] = "):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def cpu_baseline(reps: int = 5, warmup: int = 2, study_reps: int = 3) -> dict:
    """The float32 DenseNet169 forward (`oracle/fp32.py`) on the host cores: batch 1 (slices/s, the
    `value`) and one 24-slice study at batch 24 (`study_latency_ms`, configuration 4's shape)."""
    from oracle import fp32
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cores = min(cores or 1, int(os.environ.get("OMP_NUM_THREADS", cores or 1)))
    torch.set_num_threads(cores)
    model = densenet.seeded_densenet169(0)
    sd = model.state_dict()
    study = torch.from_numpy(synthetic.c5_study(0)[:SLICES])
    x = synthetic.normalise(study[:1])
    for _ in range(warmup):
        fp32.forward(sd, x)
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fp32.forward(sd, x)
        ts.append(time.perf_counter() - t)
    med = float(np.median(ts))
    xs = synthetic.normalise(study)
    fp32.forward(sd, xs)
    tb = []
    for _ in range(study_reps):
        t = time.perf_counter()
        fp32.forward(sd, xs)
        tb.append(time.perf_counter() - t)
    med24 = float(np.median(tb))
    cpu = platform.processor() or ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(1.0 / med, 4), "unit": "slices/s", "cores": cores, "kind": "port",
            "study_latency_ms": round(med24 * 1e3, 1),
            "study_slices_per_s": round(SLICES / med24, 3),
            "sample": f"fp32 DenseNet169 forward (oracle/fp32.py) at 512 px: batch 1, {warmup} warm-up + "
                      f"{reps} timed, median {med * 1e3:.0f} ms; batch {SLICES} (one study), 1 warm-up + "
                      f"{study_reps} timed, median {med24 * 1e3:.0f} ms; CPU {cpu}"}


def mfma_probe(dev: torch.device, blocks: int = 2048, iters: int = 4096, reps: int = 3) -> dict:
    """Measured int8 MFMA rate: `d8s_micro_mfma` (every wave issues independent
    v_mfma_i32_32x32x32_i8 back to back, 4 waves per workgroup, 8 workgroups per CU) between HIP
    events on the current stream; the ceiling the MFMA fractions are also quoted against."""
    import ctypes
    from rsna_knee_efficiency_amd import hip
    sink = torch.zeros(blocks, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    launch = lambda: hip.call("d8s_micro_mfma", blocks, iters, ctypes.c_void_p(sink.data_ptr()),  # noqa: E731
                              ctypes.c_void_p(st))
    launch()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        launch()
    e1.record()
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / reps
    ops = blocks * 4 * iters * 4 * (32 * 32 * 32 * 2)
    tops = ops / (ms * 1e-3) / 1e12
    return {"i8_tops": round(tops, 1), "datasheet_i8_tops": I8_PEAK_TOPS,
            "frac_of_datasheet": round(tops / I8_PEAK_TOPS, 4), "ms": round(ms, 4),
            "sample": f"{blocks} workgroups x 4 waves x {iters} rounds of 4 independent "
                      f"v_mfma_i32_32x32x32_i8"}


def graph_ms(fn, reps: int, stream) -> float:
    """ms per call of `fn` (which launches on `stream`): `reps` calls in one HIP graph, one warm replay,
    then the median of three timed replays."""
    with torch.cuda.stream(stream):
        fn()
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            for _ in range(reps):
                fn()
        g.replay()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record(stream)
        for e in ev[1:]:
            g.replay()
            e.record(stream)
        stream.synchronize()
    return sorted(a.elapsed_time(b) for a, b in zip(ev, ev[1:]))[1] / reps


def bench_kernels(dev: torch.device, reps: int = 20, peak_tops: float | None = None) -> dict:
    """Configurations 2 and 3 case by case: the 12 fused-prologue 1 x 1 GEMMs (`d8s_conv1`) and the 4
    3 x 3 convs (`d8s_conv2`) at batch 24 on the benchmark's own inputs (`synthetic.c2_case` /
    `c3_case`, seeds 11/12 and 21/22), each timed alone (`graph_ms`): ms, algorithmic GB/s (conv1:
    M C_in + M 128 + its tables; conv2: M 128 + M 32 + 36 KB of weights), int8 TOP/s (2 per MAC) and
    the fractions of 8 TB/s, of the 5.0 POP/s datasheet peak and of `peak_tops` (the rate measured on
    the box by `mfma_probe`)."""
    import ctypes
    from rsna_knee_efficiency_amd import hip
    stream = torch.cuda.Stream(dev)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731

    def row(case: dict, ms: float, byts: float, ops: float) -> dict:
        gbs, tops = byts / (ms * 1e-3) / 1e9, ops / (ms * 1e-3) / 1e12
        r = {**case, "ms": round(ms, 5), "gbs": round(gbs, 1), "int8_tops": round(tops, 1),
             "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "frac_mfma_datasheet": round(tops / I8_PEAK_TOPS, 4)}
        if peak_tops:
            r["frac_mfma_measured"] = round(tops / peak_tops, 4)
        return r

    c2 = []
    for S, cin in synthetic.C2_CASES:
        d = synthetic.c2_case(S, cin)
        M = d["N"] * S * S
        t = {k: T(d[k]) for k in ("in0", "seg", "w1", "abh", "gdu", "w1sum")}
        bott = torch.empty(4 * M * 32, dtype=torch.uint8, device=dev)
        args = hip.GemmArgs(t["in0"].data_ptr(), t["seg"].data_ptr(), t["w1"].data_ptr(), t["abh"].data_ptr(),
                            t["gdu"].data_ptr(), t["w1sum"].data_ptr(), bott.data_ptr(), d["G0"], d["G"],
                            d["N"], S * S, S, M, 128, 0)
        ms = graph_ms(lambda: hip.call("d8s_conv1", ctypes.byref(args), stream.cuda_stream), reps, stream)
        byts = M * cin + M * 128 + 128 * cin + cin * 4 + 128 * 12
        c2.append(row({"S": S, "C_in": cin, "batch": d["N"]}, ms, byts, 2.0 * M * cin * 128))
        del t, bott
    c3 = []
    for S in synthetic.C3_SIDES:
        d = synthetic.c3_case(S)
        M = d["N"] * S * S
        t = {k: T(d[k]) for k in ("bott", "w2k", "c2u", "w2sum")}
        slot = torch.empty(M * 32, dtype=torch.int8, device=dev)
        args = hip.Conv2Args(t["bott"].data_ptr(), t["w2k"].data_ptr(), t["c2u"].data_ptr(),
                             t["w2sum"].data_ptr(), slot.data_ptr(), d["N"], S, S, 0)
        ms = graph_ms(lambda: hip.call("d8s_conv2", ctypes.byref(args), stream.cuda_stream), reps, stream)
        byts = M * 128 + M * 32 + 36864 + 32 * 8
        c3.append(row({"S": S, "batch": d["N"]}, ms, byts, 2.0 * M * 1152 * 32))
        del t, slot
    return {"config": "C2: fused BN + ReLU prologue 1x1 INT8 GEMM -> u8 bottleneck (d8s_conv1); C3: 3x3 "
                      "pad-1 INT8 conv 128 -> 32 into a store slot (d8s_conv2); batch 24, each case alone, "
                      f"{reps} launches per HIP graph, median of 3 replays",
            "c2_cases": c2, "c3_cases": c3}


def block_work(b: dict, n: int) -> tuple[float, float]:
    """(algorithmic bytes, int8 operations) of a whole dense block of n images in one launch: its input
    read once, its layers' outputs written once, the weights read once."""
    M = n * b["h"] * b["w"]
    byts, ops = M * b["c0"] + M * 32 * b["L"], 0.0
    for li in range(b["L"]):
        cin = b["c0"] + 32 * li
        byts += 128 * cin + cin * 4 + 128 * 12 + 36864 + 32 * 8
        ops += 2.0 * M * cin * 128 + 2.0 * M * 1152 * 32
    return byts, ops


def c4_roofline(enc, reps: int, peak_tops: float | None) -> dict:
    """Configuration 4's dominant launch, a whole banded block (`time_layers` of the block launches on the
    study's store; the other launches of the pass are shorter, `profiles/encoder_c4_kernel_trace.md`):
    its int8 rate against the MFMA peak (thousands of operations per byte, far right of the ridge, so the
    bound is the matrix cores) and its algorithmic GB/s."""
    layers = enc.time_layers(reps=reps, families=("block",))
    label = max(layers, key=layers.get)
    ms = layers[label]
    out = {"kernel": label, "ms": round(ms, 5), "block_launch_ms": layers}
    if label.startswith("blk b"):
        bi = int(label[5:])
        byts, ops = block_work(enc.meta["blocks"][bi], enc.nb)
        tops = ops / (ms * 1e-3) / 1e12
        out.update({"entry": "d8s_dense_block_parts" if enc.fused[bi].startswith("parts") else "d8s_dense_block",
                    "kind": enc.fused[bi], "bound": "mfma", "achieved": round(tops, 1), "peak": I8_PEAK_TOPS,
                    "unit": "TOP/s", "frac": round(tops / I8_PEAK_TOPS, 4),
                    "gbs": round(byts / (ms * 1e-3) / 1e9, 1), "algorithmic_bytes": int(byts), "ops": ops})
        if peak_tops:
            out["frac_of_measured_peak"] = round(tops / peak_tops, 4)
    return out


def family_in_pass(encs, x, reps: int, family: str, bytes_per_launch: float, concurrent: bool) -> dict:
    """One family's share of a whole configuration-5 pass of seed 0 as the timed steps run it, a HIP graph
    replay: the pass against the same pass without the family's launches (`Dense8SEncoder.pass_share`,
    medians over `reps` replays of each), the difference / launches, and the algorithmic bytes per launch
    over it against 8 TB/s.  `concurrent`: seed 1's pass replays its graph on its own stream from the
    same start (the two then share the GPU as in the two-stream step); the difference is then what the
    family adds to the pair's time, which the other pass's work partly fills, so it is reported per
    launch without a bandwidth or roofline fraction."""
    enc = encs[0]
    if not any(s.family == family for s in enc.program):
        return {}
    sh = enc.pass_share(x, family, reps=reps, flip="tta", beside=encs[1] if concurrent else None)
    ms = sh["share_ms"] / sh["launches"]
    if concurrent:
        return {"family": family, "launches": sh["launches"], "share_ms_per_launch": round(ms, 5),
                "pair_ms": round(sh["pass_ms"], 4), "pair_without_ms": round(sh["without_ms"], 4),
                "timed": "seed 0's pass and seed 1's on two streams from the same start, with and without "
                         "seed 0's launches of the family (HIP graphs)"}
    gbs = bytes_per_launch / (ms * 1e-3) / 1e9
    return {"family": family, "launches": sh["launches"], "avg_launch_ms": round(ms, 5), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "pass_ms": round(sh["pass_ms"], 4),
            "without_ms": round(sh["without_ms"], 4),
            "timed": "seed 0's pass alone, with and without the family's launches (HIP graphs)"}


def bench_c4(dev: torch.device, passes: int, reps: int) -> dict:
    """Configuration 4 alone: one encoder (seed 0, batch 24), the 24-slice study of study 0 replayed
    from its graph `passes` times (wall latency per replay, median), then the per-family kernel times
    of its pass (`Dense8SEncoder.time_families`, batch 24)."""
    enc, _ = build_encoder(0, SLICES, dev)
    hw, hb = synthetic.linear_head(1664, 8, seed=99)
    lin = head_mod.LinearHead(hw, hb, dev)
    x = torch.from_numpy(synthetic.c5_study(0)[:SLICES]).to(dev)
    enc.capture(SLICES)
    for _ in range(3):
        lin(enc(x))
    torch.cuda.synchronize()
    lat = []
    for _ in range(passes):
        t = time.perf_counter()
        lin(enc(x))
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t)
    fam = enc.time_families(x, reps=reps)
    byts = kernel_bytes(enc.meta, SLICES, enc.fused)
    ops = kernel_ops(enc.meta, SLICES, enc.fused)
    return {"config": "C4: one 24-slice study, batch 24, seed 0, HIP graph replay, then the 1664 -> 8 "
                      "linear head on the device",
            "passes": passes, "study_latency_ms": round(float(np.median(lat)) * 1e3, 3),
            "pass_ms_kernels": round(sum(fam.values()), 3),
            "family_ms": {k: round(v, 4) for k, v in fam.items()},
            "launches_per_pass": {k: len(v) for k, v in byts.items()},
            "family_gbs": {k: round(sum(byts[k]) / (fam[k] * 1e-3) / 1e9, 1) for k in byts if fam.get(k)},
            "family_int8_tops": {k: round(ops[k] / (fam[k] * 1e-3) / 1e12, 1) for k in ops if fam.get(k)},
            "blocks": {str(k): v for k, v in enc.fused.items()}}


PREP_READ_SLICES = (0, 23)      # the final submission's KNEE_READ_SLICES (raw_crop.py:71-76)


def prep_bytes(payload: dict, img: int, n_scales: int, read_slices) -> int:
    """Algorithmic HBM bytes of one study's preparation: every stored uint16 value of the slices read
    (each region once), the Rescale table, and every uint8 of the volume written once."""
    from rsna_knee_efficiency_amd import prep
    total = 0
    for row in payload["meta"]:
        K = int(row[prep.M_K])
        if row[prep.M_MODE] != prep.MODE_GPU:
            total += 2 * n_scales * K * img * img          # copied CPU series: read + write
            continue
        rr = prep.read_range(K, int(row[prep.M_FLIP]), read_slices) or (0, K)
        total += 2 * (rr[1] - rr[0]) * int(row[prep.M_HR]) * int(row[prep.M_WR])
        total += 8 * K if row[prep.M_RESC] >= 0 else 0
        total += n_scales * K * img * img
    return total


def prep_cpu_baseline(payload: dict, read_slices) -> dict:
    """The oracle's chain (C resize + numpy percentiles and normalisation) on one study, 1 core."""
    from oracle import prep as oprep
    t = time.perf_counter()
    oprep.payload_to_uint8(payload, IMG, 4, 2, SLICES, read_slices=read_slices)
    dt = time.perf_counter() - t
    return {"value": round(1.0 / dt, 4), "unit": "studies/s", "cores": 1, "kind": "port",
            "sample": f"one synthetic study (4 series, 2 crops, {SLICES} slices, 512 px, slices "
                      f"{read_slices[0]}:{read_slices[1]}) through oracle/prep.py: {dt:.2f} s"}


PREP_TRAFFIC_FILE = ROOT / "profiles" / "prep_study512_hbm_traffic.md"


def prep_studies(dev: torch.device) -> tuple[list, list]:
    """The two synthetic studies of the preparation benchmark: host payloads and their device copies."""
    pays = [synthetic.study_payload(IMG, SLICES, seed=100 + i) for i in range(2)]
    dpays = [{"raw": torch.from_numpy(p["raw"]).to(dev), "u8": torch.from_numpy(p["u8"]).to(dev),
              "resc": torch.from_numpy(p["resc"]).to(dev), "meta": p["meta"]} for p in pays]
    return pays, dpays


def prep_pmc(dev: torch.device, passes: int, copy: bool) -> dict:
    """`passes` studies through the preparation, eagerly (the launches of a counter run)."""
    from rsna_knee_efficiency_amd import prep
    spec = prep.PrepSpec(img=IMG, slices=SLICES, n_seq=4, n_scales=2)
    pays, dpays = prep_studies(dev)
    for k in range(passes):
        prep.payloads_to_uint8([dpays[k % 2]], spec, dev, read_slices=PREP_READ_SLICES)
    torch.cuda.synchronize()
    res = {"passes": passes, "algorithmic_bytes_per_study": sum(prep_bytes(p, IMG, 2, PREP_READ_SLICES)
                                                                for p in pays) / 2}
    if copy:
        res["copy_probe"] = copy_probe(dev, reps=1)
    return res


def prep_traffic_summary(fetch_dir: str, write_dir: str, passes: int, copy_bytes: int = 1 << 30) -> str:
    """HBM bytes per study of the preparation kernels from two `bench.py --path prep --pmc-passes P
    --copy-probe` counter runs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the
    counter reads for k_copy (1 GiB read + 1 GiB written per dispatch)."""
    import csv
    import glob

    def collect(d: str, counter: str) -> dict:
        acc: dict = {}
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                name = r.get("Kernel_Name", "")
                fam = _family(name)
                if fam and r["Counter_Name"] == counter:
                    m = re.search(r"(k_prep_\w+(?:<[^>]*>)?)", name)
                    key = "copy" if fam == "copy" else (m.group(1) if m else name)
                    v = acc.setdefault(key, [0, 0.0])
                    v[0] += 1
                    v[1] += float(r["Counter_Value"]) * 1024
        return acc

    fe, wr = collect(fetch_dir, "FETCH_SIZE"), collect(write_dir, "WRITE_SIZE")
    kf = copy_bytes / (fe["copy"][1] / fe["copy"][0])
    kw = copy_bytes / (wr["copy"][1] / wr["copy"][0])
    pays = [synthetic.study_payload(IMG, SLICES, seed=100 + i) for i in range(2)]
    alg = sum(prep_bytes(p, IMG, 2, PREP_READ_SLICES) for p in pays) / 2
    lines = [f"Calibration: k_copy moves {copy_bytes} B read + {copy_bytes} B written per dispatch; "
             f"FETCH_SIZE scale {kf:.3f}, WRITE_SIZE scale {kw:.3f}.  {passes} studies.", "",
             "| kernel | dispatches per study | HBM read MB/study | HBM write MB/study |",
             "|---|---|---|---|"]
    tot = 0.0
    for k in sorted(set(fe) | set(wr)):
        if k == "copy":
            continue
        n = fe.get(k, [0, 0.0])[0] / passes
        rd = fe.get(k, [0, 0.0])[1] * kf / passes
        wt = wr.get(k, [0, 0.0])[1] * kw / passes
        tot += rd + wt
        lines.append(f"| `{k}` | {n:g} | {rd / 1e6:.2f} | {wt / 1e6:.2f} |")
    lines += ["", f"Traffic per study {tot / 1e6:.1f} MB; algorithmic bytes per study {alg / 1e6:.1f} MB "
                  f"(each stored uint16 value read once, each uint8 written once); ratio "
                  f"{tot / alg:.2f}.", "", "```", f"traffic_per_study = {int(tot)}", "```"]
    return "\n".join(lines)


def committed_prep_traffic() -> int | None:
    try:
        for line in PREP_TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_per_study = "):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


FP32_PEAK_TFLOPS = 157.3     # MI355X fp32, published


def head_flops(w: int, d: int = 1664, cd: int = 256, ff: int = 512, t: int = 12) -> float:
    """Multiply-adds x 2 of the head for one study of w windows (ctx_in, in_proj, attention, out_proj,
    feed-forward, ctx_out, the attention and classifier dots)."""
    mac = w * d * cd + w * cd * 3 * cd + 2 * w * w * cd + w * cd * cd + 2 * w * cd * ff + w * cd * d \
        + 2 * w * d * t
    return 2.0 * mac


def bench_head(dev: torch.device, b: int = 8, w: int = 88, reps: int = 50, with_cpu: bool = False) -> dict:
    """The head after the encoder (`head.KneeHead`, d8s_head) on b studies of w windows, seeded weights
    of the final model's shapes, features resident in HBM."""
    from rsna_knee_efficiency_amd import head as hd
    g = torch.Generator().manual_seed(0)
    keys = hd.KEYS.values()
    shapes = {"slot_emb": (8, 1664), "ctx_in.weight": (256, 1664), "ctx_in.bias": (256,), "ctx_pos": (11, 256),
              "ctx.layers.0.self_attn.in_proj_weight": (768, 256), "ctx.layers.0.self_attn.in_proj_bias": (768,),
              "ctx.layers.0.self_attn.out_proj.weight": (256, 256), "ctx.layers.0.self_attn.out_proj.bias": (256,),
              "ctx.layers.0.norm1.weight": (256,), "ctx.layers.0.norm1.bias": (256,),
              "ctx.layers.0.norm2.weight": (256,), "ctx.layers.0.norm2.bias": (256,),
              "ctx.layers.0.linear1.weight": (512, 256), "ctx.layers.0.linear1.bias": (512,),
              "ctx.layers.0.linear2.weight": (256, 512), "ctx.layers.0.linear2.bias": (256,),
              "ctx_out.weight": (1664, 256), "ctx_out.bias": (1664,), "attn.weight": (12, 1664),
              "attn.bias": (12,), "cls_w": (12, 1664), "cls_b": (12,)}
    sd = {k: torch.randn(shapes[k], generator=g) * 0.02 for k in keys}
    head = hd.KneeHead(sd, dev)
    z = torch.randn((b, w, 1664), generator=g).to(dev)
    slot_of = (torch.arange(w) // 11) % 8
    mask = torch.ones((b, 8), dtype=torch.bool).to(dev)    # every input resident on the device
    for _ in range(5):
        head(z, slot_of, mask)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = time.perf_counter()
    e0.record()
    for _ in range(reps):
        head(z, slot_of, mask)
    e1.record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t) / reps
    ms = e0.elapsed_time(e1) / reps
    tflops = b * head_flops(w) / (ms * 1e-3) / 1e12
    out = {"metric": "head logits (context layer + per-finding attention pooling) studies/s on 1 MI355X",
           "value": round(b / dt, 1), "unit": "studies/s", "studies_per_call": b, "windows": w,
           "gpu_ms_per_call": round(ms, 4), "dtype": "f32",
           "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP32_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / FP32_PEAK_TFLOPS, 4), "traffic": None,
                        "flops_per_study": head_flops(w)}}
    if with_cpu:
        from oracle import head as oh
        torch.set_num_threads(1)
        t = time.perf_counter()
        oh.head_forward(sd, z[:1].cpu(), slot_of, mask[:1].cpu())
        c = time.perf_counter() - t
        out["cpu_baseline"] = {"value": round(1.0 / c, 2), "unit": "studies/s", "cores": 1, "kind": "port",
                               "sample": f"one study of {w} windows through oracle/head.py (torch fp32, 1 thread)"}
    return out


def bench_zoom(dev: torch.device, reps: int = 20) -> dict:
    """The submission's geometric view on one study: the windows of 8 slots x 11 triplets (stride 2,
    depth 3, 24 slices) gathered from the uint8 volume and zoomed 1.10 (`tta.windows_u8`), between HIP
    events.  Bytes: each fp16 output once plus each uint8 slice read once."""
    from rsna_knee_efficiency_amd import tta
    v = torch.randint(0, 256, (1, 8, SLICES, IMG, IMG), dtype=torch.uint8, device=dev)
    starts = list(range(0, SLICES - 2, 2))
    idx = torch.tensor([s * SLICES + t + d for s in range(8) for t in starts for d in range(3)],
                       dtype=torch.int64, device=dev)
    out = torch.empty((idx.numel() // 3, 3, IMG, IMG), dtype=torch.float16, device=dev)
    for _ in range(3):
        tta.windows_u8(v, idx, out, 1.10)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        tta.windows_u8(v, idx, out, 1.10)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nbytes = out.numel() * 2 + 8 * SLICES * IMG * IMG
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"windows": int(out.shape[0]), "gpu_ms": round(ms, 4), "bytes": int(nbytes), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def bench_prep(dev: torch.device, steps: int, warmup: int, with_cpu: bool) -> dict:
    """The preparation path (raw crops -> uint8 volume) on studies resident in HBM."""
    from rsna_knee_efficiency_amd import prep
    spec = prep.PrepSpec(img=IMG, slices=SLICES, n_seq=4, n_scales=2)
    pays, dpays = prep_studies(dev)
    rs = PREP_READ_SLICES
    for k in range(warmup):
        prep.payloads_to_uint8([dpays[k % 2]], spec, dev, read_slices=rs)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = time.perf_counter()
    e0.record()
    for k in range(steps):
        prep.payloads_to_uint8([dpays[k % 2]], spec, dev, read_slices=rs)
    e1.record()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t
    gpu_ms = e0.elapsed_time(e1) / steps
    nbytes = sum(prep_bytes(p, IMG, 2, rs) for p in pays) / 2
    achieved = nbytes / (gpu_ms * 1e-3) / 1e9
    out = {
        "metric": "study preparation (raw uint16 crops -> 8 uint8 stacks of 24 x 512 x 512) studies/s "
                  "on 1 MI355X",
        "value": round(steps / dt, 2), "unit": "studies/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(dt / steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32/f64 (uint16 in, uint8 out)",
        "data": "synthetic study payloads (rsna_knee_efficiency_amd.synthetic.study_payload)",
        "config": {"workload": "one study per step: 4 series x 2 crops (110, 150 mm) x 24 slices at 512 px, "
                               "slices 0:23 read, inputs resident in HBM (payloads_to_uint8)",
                   "parallelism": "none (1 GPU)"},
        "gpu_ms_per_study": round(gpu_ms, 4),
        "roofline": {"bound": "hbm", "kernel": "d8s_prep (its 8 launches per call, between HIP events)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_prep_traffic(),
                     "traffic_unit": "bytes per study (profiles/prep_study512_hbm_traffic.md)",
                     "algorithmic_bytes_per_study": int(nbytes)},
    }
    out["zoom_view"] = bench_zoom(dev)
    if with_cpu:
        log("prep cpu baseline ...")
        out["cpu_baseline"] = prep_cpu_baseline(pays[0], rs)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prof-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--serial", action="store_true",
                    help="run the two seeds' passes of a step back to back on one stream")
    ap.add_argument("--pair", action="store_true",
                    help="run the two seeds' passes of a step as one sequence of paired launches "
                         "(dense8s.EncoderPair) instead of two streams")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time d8s_micro_copy over 1 GiB (HBM floor, counter calibration)")
    ap.add_argument("--rocprof-summary", metavar="DIR",
                    help="print a markdown summary of rocprofv3 CSV output in DIR and exit")
    ap.add_argument("--pmc-passes", type=int, default=0, metavar="P",
                    help="only run P eager configuration-5 passes of one encoder (the launches of "
                         "a counter-collection run), print the per-family times and exit")
    ap.add_argument("--path", choices=("encoder", "prep", "head", "kernels"), default="encoder",
                    help="prep: the upstream preparation (raw crops -> uint8 volume); head: the head "
                         "after the encoder; kernels: configurations 2 and 3 case by case")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the HBM traffic per launch from two --pmc-passes counter runs")
    ap.add_argument("--c4-passes", type=int, default=0, metavar="P",
                    help="only configuration 4: P graph replays of the 24-slice study (latency per "
                         "replay) and its per-family kernel times, one JSON line (a clean kernel trace)")
    ap.add_argument("--mfma-summary", metavar="PMC_DIR",
                    help="print the MFMA use per family from a --pmc-passes counter run")
    ap.add_argument("--c4-summary", metavar="TRACE_CSV",
                    help="print the per-pass kernel times of a --c4-passes kernel trace")
    ap.add_argument("--pmc-nb", type=int, choices=(96, 24), default=96,
                    help="with --pmc-passes: 96 = a configuration-5 flip-TTA pass, 24 = a "
                         "configuration-4 study (plain)")
    ap.add_argument("--c4-counter-summary", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "MFMA_DIR", "WAVE_DIR"),
                    help="print configuration 4's banded-block counters from four --pmc-passes "
                         "--pmc-nb 24 runs")
    ap.add_argument("--wave-summary", metavar="PMC_DIR",
                    help="print where the waves' cycles go per family from a --pmc-passes 1 run of "
                         "the SQ counters WAVE_COUNTERS")
    args = ap.parse_args()
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary))
        return
    if args.mfma_summary:
        print(mfma_summary(args.mfma_summary, passes=args.pmc_passes or 3))
        return
    if args.wave_summary:
        print(wave_summary(args.wave_summary))
        return
    if args.c4_summary:
        print(c4_summary(args.c4_summary))
        return
    if args.c4_counter_summary:
        print(c4_counter_summary(*args.c4_counter_summary, passes=args.pmc_passes or 3))
        return
    if args.traffic_summary:
        if args.path == "prep":
            print(prep_traffic_summary(*args.traffic_summary, passes=args.pmc_passes or 3))
        else:
            print(traffic_summary(*args.traffic_summary, passes=args.pmc_passes or 3))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build runs on one GPU (the encoder is per-GPU, replicas need no "
              f"communication); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(2)
    torch.backends.cudnn.allow_tf32 = False
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    if args.path == "head":
        print(json.dumps(bench_head(dev, with_cpu=not args.no_cpu)), flush=True)
        return
    if args.path == "kernels":
        peak = mfma_probe(dev)
        res = bench_kernels(dev, peak_tops=peak["i8_tops"])
        res["mfma_probe"] = peak
        print(json.dumps(res), flush=True)
        return
    if args.path == "prep":
        if args.pmc_passes:
            print(json.dumps(prep_pmc(dev, args.pmc_passes, args.copy_probe)), flush=True)
        else:
            print(json.dumps(bench_prep(dev, args.steps, args.warmup, not args.no_cpu)), flush=True)
        return
    if args.c4_passes:
        print(json.dumps(bench_c4(dev, args.c4_passes, args.prof_reps)), flush=True)
        return
    t0 = time.perf_counter()
    nb = 4 * SLICES                                     # 2 crops x 24 slices x flip
    if args.pmc_passes:
        nb = args.pmc_nb
        mode = "tta" if nb == 4 * SLICES else False
        enc = build_encoder(0, nb, dev)[0]
        x = torch.from_numpy(synthetic.c5_study(0)).to(dev)
        if nb != 4 * SLICES:
            x = x[:nb].contiguous()
        fam = family_times(enc, x, args.pmc_passes - 1, mode) if args.pmc_passes > 1 else {}
        if args.pmc_passes == 1:
            enc(x, flip=mode)
            torch.cuda.synchronize()
        kb = kernel_bytes(enc.meta, nb, enc.fused)
        res = {"passes": args.pmc_passes, "launches_per_pass": {k: len(v) for k, v in kb.items()},
               "bytes_per_pass": {k: sum(v) for k, v in kb.items()},
            "family_ms": fam}
        if args.copy_probe:
            res["copy_probe"] = copy_probe(dev, reps=1)
        print(json.dumps(res))
        return
    built = [build_encoder(seed, nb, dev) for seed in (0, 1)]
    encs = [e for e, _ in built]
    log(f"encoders built in {time.perf_counter() - t0:.1f} s")
    # the 50 distinct studies of configuration 5 resident in HBM: each 2 crops x 24 slices (uint8)
    studies = [torch.from_numpy(synthetic.c5_study(s)).to(dev) for s in range(C5_STUDIES)]
    log(f"{len(studies)} studies generated and resident ({time.perf_counter() - t0:.1f} s)")
    for e in encs:
        e.capture(2 * SLICES, flip="tta")
    pair = None
    if args.pair:
        pair = dense8s.EncoderPair(encs[0], encs[1])
        pair.capture(2 * SLICES, flip="tta")
    torch.cuda.synchronize()

    # the two seeds' passes are independent: dense8s.encode_concurrent runs each from its own stream,
    # so the small, latency-bound layers of one seed's pass overlap the other's.  --serial runs them
    # back to back, --pair as paired launches.
    def step(k: int) -> None:
        x = studies[k % len(studies)]
        if args.serial:
            for e in encs:
                e(x, flip="tta")
        elif pair is not None:
            pair(x, flip="tta")
        else:
            dense8s.encode_concurrent([(e, x, "tta") for e in encs])

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for k in range(args.steps):
        step(k)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t
    per_step = 2 * nb
    value = per_step * args.steps / dt
    log(f"config 5: {args.steps} studies in {dt:.3f} s: {value:.1f} slices/s")
    # every one of the 50 studies once, back to back (beside the K timed steps)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for k in range(len(studies)):
        step(k)
    torch.cuda.synchronize()
    dt50 = time.perf_counter() - t
    sweep = {"studies": len(studies), "ms_per_study": round(dt50 / len(studies) * 1e3, 3),
             "slices_per_s": round(per_step * len(studies) / dt50, 2)}
    log(f"config 5 over all {len(studies)} studies once: {sweep}")
    # agreement of configuration 5's outputs (study 0, both seeds, 48 plain + 48 mirrored encoded
    # images) with the fp32 DenseNet169 forward of the same weights on the plain and mirrored images
    hw, hb = synthetic.linear_head(1664, 8, seed=99)
    c5_agree = {}
    for seed, e in zip((0, 1), encs):
        got = e(studies[0], flip="tta").double().cpu().numpy()
        m = densenet.seeded_densenet169(seed).to(dev).eval()
        refs = []
        with torch.no_grad():
            for src in (studies[0], torch.flip(studies[0], dims=[-1])):
                for chunk in src.split(16):
                    refs.append(m(synthetic.normalise(chunk.contiguous())).double().cpu())
        del m
        ref = torch.cat(refs).numpy()
        c5_agree[f"seed{seed}"] = {"features": agree(got, ref),
                                   "logits": agree(got @ hw.T + hb, ref @ hw.T + hb)}
    log(f"config 5 fp32 agreement {c5_agree}")

    # configuration 4: one 24-slice study, batch 24, one encoder, then the 1664 -> 8 linear head on the
    # device (d8s_linear): the latency runs from the call to the logits on the device
    enc4, _ = build_encoder(0, SLICES, dev)
    lin4 = head_mod.LinearHead(hw, hb, dev)
    x4 = studies[0][:SLICES].contiguous()
    enc4.capture(SLICES)
    for _ in range(args.warmup):
        lin4(enc4(x4))
    torch.cuda.synchronize()
    lat = []
    for _ in range(max(args.steps, 5)):
        ta = time.perf_counter()
        lin4(enc4(x4))
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - ta)
    study_ms = float(np.median(lat)) * 1e3
    c4_wait_errors = enc4.sync_errors()
    if c4_wait_errors:
        raise RuntimeError(f"config 4: {c4_wait_errors} bounded waits of the banded blocks ran out")
    log(f"config 4: study latency {study_ms:.3f} ms to the logits (median of {len(lat)}), "
        f"banded-block wait errors {c4_wait_errors}")
    roof4 = c4_roofline(enc4, args.prof_reps, None)
    log(f"config 4 dominant launch: {roof4}")

    # agreement of the INT8 features with the fp32 DenseNet169 forward of the same weights on the same
    # study (the GPU, float32 torch), and of the logits of a seeded 1664 -> 8 linear head
    model4 = densenet.seeded_densenet169(0).to(dev).eval()
    with torch.no_grad():
        ref4 = model4(synthetic.normalise(x4)).double().cpu().numpy()
    f4 = enc4(x4)
    got4 = f4.double().cpu().numpy()
    lg4 = lin4(f4).double().cpu().numpy()                  # the device head's logits
    del model4
    fp32_agreement = {"features": agree(got4, ref4), "logits": agree(lg4, ref4 @ hw.T + hb),
                      "slices": SLICES, "gate": "rel_l2 <= 1.05 x 0.067, cos_min >= 0.99",
                      "c5": dict(c5_agree, images="study 0: 48 plain + 48 mirrored, per seed")}
    log(f"fp32 agreement {fp32_agreement}")

    # the reference's own headline shape: one study of 88 images at 288 px through one encoder (graph
    # replay), which the reference quotes at 34 ms on one T4 (kaggle/int8_pack/pack_dense8s.py:29-30)
    ref_model = densenet.seeded_densenet169(0).to(dev)
    with torch.no_grad():
        cal288 = dense8s.calibrate(ref_model, [synthetic.normalise(torch.from_numpy(c).to(dev))
                                               for c in np.split(synthetic.study_u8(32, 288, seed=8), 4)])
    enc288 = dense8s.Dense8SEncoder(dense8s.make_pack(dense8s.make_plan(ref_model.cpu(), cal288, 288), 88,
                                                      input_kind="u8"), dev.index or 0, 88)
    del ref_model
    x288 = torch.from_numpy(synthetic.study_u8(88, 288, seed=4321)).to(dev)
    enc288.capture(88)
    for _ in range(3):
        enc288(x288)
    torch.cuda.synchronize()
    lat288 = []
    for _ in range(max(args.steps, 5)):
        ta = time.perf_counter()
        enc288(x288)
        torch.cuda.synchronize()
        lat288.append(time.perf_counter() - ta)
    ref_study = {"workload": "the reference's study shape: 88 images at 288 px, one encoder, HIP graph replay",
                 "ms_per_study": round(float(np.median(lat288)) * 1e3, 3),
                 "reference_ms_per_study": 34.0, "reference_hardware": "1 x T4 (published, not this metric)"}
    log(f"reference study shape: {ref_study}")
    del enc288

    # per-family kernel times: each family's launches of a pass in a HIP graph, replayed between
    # HIP events on the encoder's stream
    fam = encs[0].time_families(studies[0], reps=args.prof_reps, flip="tta")
    byts = kernel_bytes(encs[0].meta, nb, encs[0].fused)
    ops = kernel_ops(encs[0].meta, nb, encs[0].fused)
    pass_ms = sum(fam.values())
    ranked = sorted(("conv1", "conv2", "chain", "dense", "block", "trans", "stem"), key=lambda k: -fam.get(k, 0.0))
    dom = ranked[0]
    dom_bytes = sum(byts[dom])
    launches = len(byts[dom])
    avg_ms = fam[dom] / launches
    achieved = dom_bytes / launches / (avg_ms * 1e-3) / 1e9
    fam_gbs = {k: round(sum(byts[k]) / (fam[k] * 1e-3) / 1e9, 1) for k in byts if fam.get(k)}
    fam_tops = {k: round(ops[k] / (fam[k] * 1e-3) / 1e12, 1) for k in ops if fam.get(k)}
    log(f"pass of {nb}: {pass_ms:.3f} ms; families ms {json.dumps({k: round(v, 3) for k, v in fam.items()})}")
    log(f"families GB/s {fam_gbs}; int8 TOP/s {fam_tops}")
    # the dominant family's share of a whole pass's graph, alone and beside the other seed's pass (the
    # isolated figure above replays its launches back to back)
    in_pass = family_in_pass(encs, studies[0], args.prof_reps, dom, dom_bytes / launches, False)
    in_sched = family_in_pass(encs, studies[0], args.prof_reps, dom, dom_bytes / launches, True)
    log(f"{dom} launches inside a pass: {in_pass}; beside the other seed's pass: {in_sched}")
    total_bytes = sum(sum(v) for v in byts.values())
    out = {
        "metric": "512px DenseNet169 INT8 slices/sec on 1 MI355X; 24-slice study latency ms",
        "value": round(value, 2), "unit": "slices/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8",
        "data": "synthetic (seeded uint8 slice stacks, seeded DenseNet169 weights)",
        "config": {"workload": "C5 sustained: per step one study = 2 seeds x (2 crops x 24 slices "
                               "+ flip TTA) = 2 passes of 96 encoded 512px slices; step k encodes "
                               "study k mod 50 of 50 distinct resident studies",
                   "global_batch": nb, "seeds": 2, "image": IMG, "studies": len(studies),
                   "parallelism": "none (1 GPU)"},
        "c5_all_studies": sweep,
        "study_latency_ms": round(study_ms, 3),
        "study_wait_errors": c4_wait_errors,
        "study_latency_config": "C4: one 24-slice study, batch 24, one encoder (HIP graph replay), then "
                                "the 1664 -> 8 linear head on the device (d8s_linear), to the logits",
        "fp32_agreement": fp32_agreement,
        "reference_study": ref_study,
        "step_schedule": ("serial (one stream)" if args.serial else
                          "paired launches (one stream)" if args.pair else "the 2 seeds' passes on 2 streams"),
        "pass_ms_kernels": round(pass_ms, 3),
        "pass_hbm_frac": round(total_bytes / (pass_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "family_ms": {k: round(v, 3) for k, v in fam.items()},
        "family_gbs": fam_gbs, "family_int8_tops": fam_tops,
        "roofline": {"bound": "hbm", "kernel": f"d8s_{dom} (all {launches} launches of a pass)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic(dom),
                     "algorithmic_bytes_per_launch": int(dom_bytes / launches),
                     "avg_launch_ms": round(avg_ms, 5),
                     "frac_in_pass": in_pass.get("frac"), "in_pass": in_pass, "in_schedule": in_sched},
        "step_hbm_frac": round(2 * total_bytes / (dt / args.steps) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline_runner_up": family_roofline(ranked[1], fam, byts, ops),
        "roofline_c4": roof4,
    }
    # the upstream preparation (raw crops -> uint8 volume), its own throughput on the same GPU
    pr = bench_prep(dev, max(args.steps, 20), args.warmup, False)
    out["prep"] = {k: pr[k] for k in ("metric", "value", "unit", "gpu_ms_per_study", "roofline", "config",
                                      "zoom_view")}
    log(f"prep: {pr['value']} studies/s, {pr['gpu_ms_per_study']} ms GPU per study")
    out["head"] = bench_head(dev)
    log(f"head: {out['head']['value']} studies/s")
    out["mfma_probe"] = mfma_probe(dev)
    log(f"mfma probe: {out['mfma_probe']}")
    out["family_int8_frac_of_measured_peak"] = {
        k: round(v / out["mfma_probe"]["i8_tops"], 4) for k, v in fam_tops.items()}
    if "achieved" in roof4:
        roof4["frac_of_measured_peak"] = round(roof4["achieved"] / out["mfma_probe"]["i8_tops"], 4)
    out["kernels"] = bench_kernels(dev, peak_tops=out["mfma_probe"]["i8_tops"])
    log(f"kernels: c2 {[(r['S'], r['C_in'], r['gbs']) for r in out['kernels']['c2_cases']]}; "
        f"c3 {[(r['S'], r['gbs']) for r in out['kernels']['c3_cases']]}")
    if args.copy_probe:
        out["copy_probe"] = copy_probe(dev)
        log(f"copy probe: {out['copy_probe']}")
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
