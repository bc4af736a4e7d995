"""CPU checks of the benchmark's accounting and its one-GPU contract."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from gmdn_amd import profiling  # noqa: E402
from gmdn_amd.workloads import WORKLOADS  # noqa: E402


def test_algorithmic_bytes_and_flops():
    w = WORKLOADS["gated_delta_b4_h16_t4096_d128"]
    # q, k, v, o bf16 + beta, g fp32 per token-head
    assert bench.fwd_bytes_per_token_head(w) == 1032
    assert bench.fwd_bytes_per_token_head(w) * w.B * w.H * w.T == 270532608
    # 4 C^2 d + 6 C d^2 per chunk-head = 8.39 MFLOP at C=64, d=128
    assert bench.fwd_flops_per_chunk_head(w) == 4 * 64 * 64 * 128 + 6 * 64 * 128 * 128
    wa = WORKLOADS["adam_b2_h8_t4096_d64"]
    assert bench.fwd_bytes_per_token_head(wa) == 8 * 64 + 16


def test_backward_flops():
    w = WORKLOADS["gated_delta_b4_h16_t4096_d128"]
    assert bench.bwd_flops_per_chunk_head(w) == 2 * bench.fwd_flops_per_chunk_head(w)
    wm = WORKLOADS["muon_b2_h16_t8192_d128"]
    gemms = 4 * 64 * 64 * 128 + 6 * 64 * 128 * 128
    assert bench.bwd_flops_per_chunk_head(wm) == 2 * gemms + (2 + 16 * 5) * 128 ** 3


def test_drop_in_accounting():
    # whole-workload totals of the drop-in scan at B=4, H=16, N=64, d=128:
    # 805.4 MB forward and 2.148 GB forward + backward; 17.2 / 51.5 GFLOP (delta)
    chunks = 4 * 16 * 64
    fwd_b, fb_b = bench.drop_in_bytes_per_chunk(128)
    assert fwd_b * chunks == 805371904
    assert fb_b * chunks == 2147680256
    f, b = bench.drop_in_flops_per_chunk("delta", 128, 5)
    assert round(f * chunks / 1e9, 1) == 17.2 and round((f + b) * chunks / 1e9, 1) == 51.5
    f, b = bench.drop_in_flops_per_chunk("muon", 128, 5)
    assert (f, b) == (32 * 128 ** 3, 86 * 128 ** 3)


def test_multi_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_read_traffic(tmp_path):
    f = tmp_path / "t.md"
    f.write_text("# x\n\ntraffic_bytes_per_launch: 12345\nread_bytes_per_launch: 1\n")
    assert profiling.read_traffic(str(f)) == 12345.0
    assert profiling.read_traffic(str(tmp_path / "missing.md")) is None


def test_pmc_csv_parsing(tmp_path):
    hdr = ('"Correlation_Id","Dispatch_Id","Agent_Id","Queue_Id","Process_Id","Thread_Id","Grid_Size",'
           '"Kernel_Id","Kernel_Name","Workgroup_Size","LDS_Block_Size","Scratch_Size","VGPR_Count",'
           '"Accum_VGPR_Count","SGPR_Count","Counter_Name","Counter_Value","Start_Timestamp","End_Timestamp"\n')
    rows = [f'{i},{i},"Agent 1",1,1,1,64,1,"void k<1>(A)",256,0,0,1,0,1,"FETCH_SIZE",{v},0,1\n'
            for i, v in ((1, 100.0), (2, 102.0))]
    (tmp_path / "x_counter_collection.csv").write_text(hdr + "".join(rows))
    assert profiling.counter_per_dispatch(str(tmp_path), "FETCH_SIZE", "k<1>") == [100.0, 102.0]
    with pytest.raises(ValueError):
        profiling.counter_per_dispatch(str(tmp_path), "WRITE_SIZE", "k<1>")


def test_drop_in_cpu_baseline_runs_on_a_small_workload():
    w = WORKLOADS["delta_fp32_small"]
    cb = bench.drop_in_cpu_baseline(w, 0.2)
    assert cb["value"] > 0 and cb["kind"] == "port" and cb["cores"] >= 1
    assert "heads" in cb["sample"]


def test_msign_accounting():
    # per NS step: X X^T (2 m^2 n) + A A (2 m^3) + B X (2 m^2 n), m = min(rows, cols)
    assert bench.msign_flops(3072, 1024, 5) == bench.msign_flops(1024, 3072, 5) == 5 * (4 * 1024 ** 2 * 3072 + 2 * 1024 ** 3)
    shapes = bench.lm_hidden_shapes()
    assert len(shapes) == 60 and shapes[:5] == [(3072, 1024), (24, 1024), (1024, 1024), (4096, 1024), (1024, 4096)]
    # about 3.6 TFLOP per outer optimizer step at the LM shapes
    assert round(sum(bench.msign_flops(*s, 5) for s in shapes) / 1e12, 2) == 3.61


def test_msign_cpu_baseline_runs():
    shapes = [(48, 32), (8, 32), (32, 32), (64, 32), (32, 64)]
    r = bench.msign_cpu_baseline(shapes, 0.1)
    assert r["kind"] == "port" and r["value"] > 0 and r["cores"] >= 1


def test_mfma_counter_summary(tmp_path):
    hdr = ('"Correlation_Id","Dispatch_Id","Agent_Id","Queue_Id","Process_Id","Thread_Id","Grid_Size","Kernel_Id",'
           '"Kernel_Name","Workgroup_Size","LDS_Block_Size","Scratch_Size","VGPR_Count","Accum_VGPR_Count","SGPR_Count",'
           '"Counter_Name","Counter_Value","Start_Timestamp","End_Timestamp"\n')
    rows = []
    for disp, (mops, busy, gui, ns) in enumerate([(1e6, 512, 1, 1000), (3e6, 1024, 1, 3000), (2e6, 768, 1, 2000)]):
        for c, v in (("SQ_INSTS_VALU_MFMA_MOPS_BF16", mops), ("SQ_VALU_MFMA_BUSY_CYCLES", busy),
                     ("GRBM_GUI_ACTIVE", gui)):
            rows.append(f'1,{disp},"Agent 1",1,1,1,1,1,"kA",256,0,0,1,0,1,"{c}",{v},0,{ns}\n')
    (tmp_path / "x_counter_collection.csv").write_text(hdr + "".join(rows))
    m = profiling.mfma_by_kernel(str(tmp_path), "kA", simds=1024, xcds=1)["kA"]
    # medians: 2e6 MOPS x 512 flops over 2000 ns; 768 busy cycles over 1 GUI cycle x 1024 SIMDs
    assert m["dispatches"] == 3 and m["flops"] == 2e6 * 512 and m["us"] == 2.0
    assert abs(m["tflops"] - 512.0) < 1e-9 and abs(m["util"] - 75.0) < 1e-9
