"""bench.py on the CPU: the algorithmic work it divides by (closed forms of DenseNet169 at 512 px), the
counter summaries it reads back from rocprofv3 CSV files, and its one-GPU contract."""
from __future__ import annotations

import csv
import os
import subprocess
import sys
from pathlib import Path

import pytest

import bench
from rsna_knee_efficiency_amd import dense8s

ROOT = Path(__file__).resolve().parents[1]
BLOCKS = [{"c0": 64, "h": 128, "w": 128, "L": 6, "trans": True},
          {"c0": 128, "h": 64, "w": 64, "L": 12, "trans": True},
          {"c0": 256, "h": 32, "w": 32, "L": 32, "trans": True},
          {"c0": 640, "h": 16, "w": 16, "L": 32, "trans": False}]
META = {"img": 512, "blocks": BLOCKS, "n": 96}


def test_ops_per_slice_closed_form():
    """int8 operations per 512 px slice: conv1 16.14 G, conv2 13.89 G, transitions 0.96 G (pooled
    resolution), stem 1.23 G — 32.22 G in all, counted layer by layer from the architecture."""
    ops = bench.kernel_ops(META, 1, {})
    conv1 = sum(2 * b["h"] * b["w"] * (b["c0"] + 32 * l) * 128 for b in BLOCKS for l in range(b["L"]))
    conv2 = sum(2 * b["h"] * b["w"] * 1152 * 32 * b["L"] for b in BLOCKS)
    assert ops["conv1"] == conv1 and ops["conv2"] == conv2
    assert abs(ops["conv1"] / 1e9 - 16.14) < 0.01 and abs(ops["conv2"] / 1e9 - 13.89) < 0.01
    assert abs(ops["trans"] / 1e9 - 0.96) < 0.01 and abs(ops["stem"] / 1e9 - 1.23) < 0.01
    assert abs(sum(ops.values()) / 1e9 - 32.22) < 0.02
    # fused kinds move the same work into their families
    fused = bench.kernel_ops(META, 1, dense8s.fused_blocks(META))
    assert abs(sum(fused.values()) - sum(ops.values())) < 1.0


def test_bytes_scale_with_images_and_match_the_layer_sums():
    one, four = bench.kernel_bytes(META, 1, {}), bench.kernel_bytes(META, 4, {})
    assert len(one["conv1"]) == len(one["conv2"]) == 82 and len(one["trans"]) == 3
    b1 = BLOCKS[1]
    M = b1["h"] * b1["w"]
    # conv1 of block 1, layer 0: activations in, bottleneck out, weights, tables
    assert one["conv1"][6] == M * 128 + M * 128 + 128 * 128 + 128 * 4 + 128 * 12
    # activation bytes scale with the images, weights and tables do not
    assert 4 * one["conv1"][6] - four["conv1"][6] == 3 * (128 * 128 + 128 * 4 + 128 * 12)
    # per slice at batch 24 (weights read once per batch): the 128.7 MB of the layer-by-layer design
    b24 = bench.kernel_bytes(META, 24, {})
    assert abs(sum(sum(v) for v in b24.values()) / 24 / 1e6 - 128.7) < 1.5
    # a chained block (conv2 of a layer with conv1 of the next): L - 1 launches that do not read the new
    # layer's 32 channels back, its first conv1 and last conv2 as before
    base, ch = bench.kernel_bytes(META, 96, {}), bench.kernel_bytes(META, 96, {2: "chain"})
    M2 = 96 * BLOCKS[2]["h"] * BLOCKS[2]["w"]
    assert len(ch["chain"]) == 31 and len(ch["conv1"]) == len(ch["conv2"]) == 82 - 31
    assert sum(map(sum, base.values())) - sum(map(sum, ch.values())) == 31 * M2 * 32
    ops_ch = bench.kernel_ops(META, 96, {2: "chain"})
    assert abs(sum(ops_ch.values()) - sum(bench.kernel_ops(META, 96, {}).values())) < 1.0


def _counter_csv(path: Path, rows: list[tuple[int, str, str, float]]) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for r in rows:
            w.writerow(r)


def test_traffic_summary_scales_by_the_copy_kernel(tmp_path):
    """FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by what they read for the 1 GiB copy."""
    gib = 1 << 30
    conv1 = "void k_conv1p<false, 1, 2, 4>(D8sGemmArgs, int*)"
    fe = [(1, "k_copy(const u32x4*, u32x4*, long)", "FETCH_SIZE", gib / 2 / 1024)]
    wr = [(1, "k_copy(const u32x4*, u32x4*, long)", "WRITE_SIZE", gib / 1024)]
    chain = "void k_c21<32>(D8sConv2Args, D8sGemmArgs)"
    # a pass of the default kinds at 96 images: 13 conv1 launches (block 1, block 2's first layer),
    # 31 chained conv2 + conv1 launches (block 2)
    for d in range(2, 2 + 13):
        fe.append((d, conv1, "FETCH_SIZE", 50e6 / 1024))       # reads 100 MB after the x2 scale
        wr.append((d, conv1, "WRITE_SIZE", 10e6 / 1024))
    for d in range(20, 20 + 31):
        fe.append((d, chain, "FETCH_SIZE", 40e6 / 1024))
        wr.append((d, chain, "WRITE_SIZE", 15e6 / 1024))
    _counter_csv(tmp_path / "f" / "run_counter_collection.csv", fe)
    _counter_csv(tmp_path / "w" / "run_counter_collection.csv", wr)
    out = bench.traffic_summary(str(tmp_path / "f"), str(tmp_path / "w"), passes=1)
    assert "FETCH_SIZE scale 2.000, WRITE_SIZE scale 1.000" in out
    assert "traffic_per_launch[conv1] = 110000000" in out
    assert "| conv1 | 13 | 100.00 | 10.00 | 110.00 |" in out
    assert "traffic_per_launch[chain] = 95000000" in out
    assert "| chain | 31 | 80.00 | 15.00 | 95.00 |" in out


def test_family_run_summary_counts_only_the_timing_replays(tmp_path):
    """The roofline's launch time from a kernel trace: runs of one family on one queue longer than its
    runs in a pass (a pass's 31 chained launches, concurrent with another stream, are left out), the
    first launch of each run not counted."""
    chain = "void k_c21<32>(D8sConv2Args, D8sGemmArgs)"
    conv1 = "void k_conv1p<false, 1, 2, 4>(D8sGemmArgs, int*, D8sGemmArgs, int)"
    rows, t = [], 0

    def add(name, us, q=1):
        nonlocal t
        rows.append({"Kernel_Name": name, "Queue_Id": q, "Start_Timestamp": t,
                     "End_Timestamp": t + int(us * 1000)})
        t += int(us * 1000) + 500

    for _ in range(31):                               # a pass's run: slower, not counted
        add(chain, 50.0)
    add(conv1, 40.0)
    for _ in range(62):                               # the family timing: 2 x 31 launches
        add(chain, 27.0)
    for _ in range(26):                               # conv1's timing: 2 x 13 launches
        add(conv1, 36.0)
    for _ in range(40):                               # another configuration's chain: its own line
        add("void k_c21<64>(D8sConv2Args, D8sGemmArgs)", 20.0)
    for _ in range(8):                                # a family of several kernels: one run
        for r in (2, 3):
            add(f"void k_band<128, {r}>(D8sDenseArgs, int, int, D8sDenseArgs, int)", 100.0 + r)
    path = tmp_path / "run_kernel_trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = "\n".join(bench.family_run_summary(str(path)))
    assert "| chain | `k_c21<32>` | 61 | 27.00 |" in out
    assert "| conv1 | `k_conv1p<false, 1, 2, 4>` | 25 | 36.00 |" in out
    assert "| chain | `k_c21<64>` | 39 | 20.00 |" in out
    assert "| dense | `k_band<128, 2>`, `k_band<128, 3>` | 15 | 102.53 |" in out


def test_wave_summary_percentages_of_wave_cycles(tmp_path):
    chain = "void k_c21<32>(D8sConv2Args, D8sGemmArgs)"
    rows = []
    for d in (1, 2):                                  # two dispatches, summed
        rows += [(d, chain, "SQ_WAVES", 100.0), (d, chain, "SQ_WAVE_CYCLES", 5000.0),
                 (d, chain, "SQ_WAIT_ANY", 2000.0), (d, chain, "SQ_WAIT_INST_ANY", 1000.0),
                 (d, chain, "SQ_ACTIVE_INST_ANY", 2000.0), (d, chain, "SQ_ACTIVE_INST_VALU", 1500.0),
                 (d, chain, "SQ_INSTS_VALU", 30000.0)]
    _counter_csv(tmp_path / "s" / "run_counter_collection.csv", rows)
    out = bench.wave_summary(str(tmp_path / "s"))
    assert "| chain | 2 | 200 | 50 | 40.0 % | 20.0 % | 40.0 % | 30.0 % | 300 |" in out


def test_c4_summary_medians_over_whole_passes(tmp_path):
    """Per-pass kernel times from a configuration-4 trace: passes split at the stem, only whole ones
    (a final-features dispatch and a transition) kept, medians over them."""
    names = {"stem": "void k_stem_rows<true>(D8sStemArgs, int, int, D8sStemArgs, int)",
             "chain": "void k_c21<64>(D8sConv2Args, D8sGemmArgs)",
             "trans": "void k_trans<5, 1, 4, 2>(D8sGemmArgs, D8sGemmArgs, int)",
             "final": "k_final(signed char const*, int, signed char const*, int, int, int, float const*, float*, int)"}
    rows, t = [], 0

    def add(fam, us):
        nonlocal t
        rows.append({"Kernel_Name": names[fam], "Queue_Id": 1, "Start_Timestamp": t,
                     "End_Timestamp": t + int(us * 1000)})
        t += int(us * 1000) + 100

    for p, extra in enumerate((0.0, 1.0, 2.0)):       # three passes: chain 10 + extra us, twice
        add("stem", 60.0)
        add("chain", 10.0 + extra)
        add("chain", 10.0 + extra)
        add("trans", 20.0)
        add("final", 5.0)
    add("stem", 60.0)                                 # a partial pass: not counted
    add("chain", 99.0)
    path = tmp_path / "run_kernel_trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = bench.c4_summary(str(path))
    assert out.startswith("3 whole passes")
    assert "| `k_c21<64>` | chain | 2 | 22.0 |" in out and "| `k_stem_rows<true>` | stem | 1 | 60.0 |" in out


def test_mfma_summary_weights_and_issued_ops(tmp_path):
    conv2 = "void k_conv2<32, 8, 1, 2>(D8sConv2Args, int, int)"
    rows = []
    # two dispatches: 10 % busy over 100 cycles, 40 % busy over 300 cycles -> 32.5 % weighted
    for d, util, gui in ((1, 10.0, 100.0), (2, 40.0, 300.0)):
        rows += [(d, conv2, "MfmaUtil", util), (d, conv2, "GRBM_GUI_ACTIVE", gui),
                 (d, conv2, "SQ_INSTS_VALU_MFMA_MOPS_I8", 1e6), (d, conv2, "SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0)]
    _counter_csv(tmp_path / "m" / "run_counter_collection.csv", rows)
    out = bench.mfma_summary(str(tmp_path / "m"), passes=1)
    line = next(ln for ln in out.splitlines() if ln.startswith("| conv2 |"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[1] == "2" and cells[2] == "32.5"
    assert float(cells[3]) == pytest.approx(2e6 * 512 / 1e9, abs=0.05)


def test_block_work_closed_form():
    """A whole block's algorithmic work: its input read once, 32 new channels per layer written, the
    weights once; operations 2 per MAC of every conv1 and conv2 (block 2 of a 24-image study: 209.4 G)."""
    b = BLOCKS[2]
    byts, ops = bench.block_work(b, 24)
    M = 24 * b["h"] * b["w"]
    w = sum(128 * (b["c0"] + 32 * l) + (b["c0"] + 32 * l) * 4 + 128 * 12 + 36864 + 32 * 8 for l in range(b["L"]))
    assert byts == M * b["c0"] + M * 32 * b["L"] + w
    assert ops == sum(2.0 * M * (b["c0"] + 32 * l) * 128 + 2.0 * M * 1152 * 32 for l in range(b["L"]))
    assert abs(ops / 1e9 - 209.38) < 0.01
    # the same work as the block's launches counted layer by layer
    per = bench.kernel_ops({"img": 512, "blocks": BLOCKS}, 24, {2: "parts:8"})
    assert abs(per["block"] - ops) < 1.0


def test_c4_counter_summary_per_banded_kernel(tmp_path):
    """Configuration 4's banded-block counters: traffic per launch scaled by the copy kernel against
    `block_work`, MfmaUtil weighted by GRBM_GUI_ACTIVE, the wave cycles as percentages."""
    gib = 1 << 30
    copy = "k_copy(const u32x4*, u32x4*, long)"
    k4, k1 = "void k_dparts<4>(D8sPartsArgs)", "void k_dparts<1>(D8sPartsArgs)"
    fe = [(1, copy, "FETCH_SIZE", gib / 2 / 1024)] + [(d, k4, "FETCH_SIZE", 10e6 / 1024) for d in (2, 3)]
    fe += [(d, k1, "FETCH_SIZE", 5e6 / 1024) for d in (4, 5)]
    wr = [(1, copy, "WRITE_SIZE", gib / 1024)] + [(d, k4, "WRITE_SIZE", 30e6 / 1024) for d in (2, 3)]
    wr += [(d, k1, "WRITE_SIZE", 4e6 / 1024) for d in (4, 5)]
    mf = [(2, k4, "MfmaUtil", 10.0), (2, k4, "GRBM_GUI_ACTIVE", 100.0), (2, k4, "SQ_INSTS_VALU_MFMA_MOPS_I8", 1e6),
          (3, k4, "MfmaUtil", 20.0), (3, k4, "GRBM_GUI_ACTIVE", 300.0), (3, k4, "SQ_INSTS_VALU_MFMA_MOPS_I8", 1e6)]
    wv = [(2, k4, "SQ_WAVE_CYCLES", 1000.0), (2, k4, "SQ_WAIT_ANY", 450.0), (2, k4, "SQ_WAIT_INST_ANY", 150.0),
          (2, k4, "SQ_ACTIVE_INST_ANY", 400.0), (2, k4, "SQ_ACTIVE_INST_VALU", 200.0)]
    for name, rows in (("f", fe), ("w", wr), ("m", mf), ("s", wv)):
        _counter_csv(tmp_path / name / "run_counter_collection.csv", rows)
    out = bench.c4_counter_summary(*(str(tmp_path / d) for d in "fwms"), passes=1)
    line = next(ln for ln in out.splitlines() if ln.startswith("| `k_dparts<4>`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    byts, ops = bench.block_work(BLOCKS[2], 24)
    assert cells[1] == "2 (parts:8)" and cells[2] == "2"
    assert float(cells[3]) == pytest.approx(20.0, abs=0.01) and float(cells[4]) == pytest.approx(30.0, abs=0.01)
    assert float(cells[5]) == pytest.approx(50e6 / byts, abs=1e-3)
    assert float(cells[6]) == pytest.approx(17.5, abs=0.05)              # (10 x 100 + 20 x 300) / 400
    assert float(cells[7]) == pytest.approx(1e6 * 512 / 1e9, abs=0.05)  # per launch
    assert float(cells[8]) == pytest.approx(ops / 1e9, abs=0.05)
    assert cells[9:13] == ["45.0", "15.0", "40.0", "20.0"]
    assert any(ln.startswith("| `k_dparts<1>`") for ln in out.splitlines())


def test_family_roofline_divides_per_launch():
    # 31 launches of 100.8 MB in 0.837 ms per pass: 27 us per launch, 3.733 TB/s; 1 POP per pass
    fam, byts, ops = {"chain": 0.837}, {"chain": [100.8e6] * 31}, {"chain": 1e15 * 0.837e-3}
    r = bench.family_roofline("chain", fam, byts, ops)
    assert r["avg_launch_ms"] == pytest.approx(0.027, abs=1e-5)
    assert r["achieved"] == pytest.approx(100.8e6 / 27e-6 / 1e9, abs=0.1)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.HBM_PEAK_GBS, abs=1e-4)
    assert r["int8_tops"] == pytest.approx(1000.0, abs=0.1) and r["frac_mfma_datasheet"] == pytest.approx(0.2)
    assert r["algorithmic_bytes_per_launch"] == int(100.8e6) and "31 launches" in r["kernel"]


def test_more_than_one_gpu_is_refused():
    env = dict(os.environ, PYTHONPATH=str(ROOT))
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, env=env, timeout=300, cwd=ROOT)
    assert r.returncode == 2 and "one GPU" in r.stderr
