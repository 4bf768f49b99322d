"""The measurement helpers of ``bench.py`` on synthetic rocprofv3 output (no GPU): the block
profile's per-launch means leave the warm-up blocks out and group a split launch's dispatches,
and the denoise-step kernel table divides by every step the run traced (warm-up, then the timed
steps twice)."""

import csv
import json

import bench

FIELDS = ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Workgroup_Size_X", "Workgroup_Size_Y",
          "Start_Timestamp", "End_Timestamp"]


def _trace(path, dispatches):
    """``dispatches``: (kernel name, duration in us) in launch order."""
    path.mkdir(parents=True)
    with open(path / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=FIELDS)
        w.writeheader()
        t = 1_000_000
        for i, (name, us) in enumerate(dispatches):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Grid_Size_X": 256 * 64, "Grid_Size_Y": 1,
                        "Workgroup_Size_X": 256, "Workgroup_Size_Y": 1, "Start_Timestamp": t,
                        "End_Timestamp": t + int(us * 1000)})
            t += int(us * 1000) + 500


GEMM = "void kx::(anonymous namespace)::gemm_lds_kernel<256, 256>(int)"
SPLIT = "void kx::(anonymous namespace)::gemm_lds_kernel<256, 256, 1>(int)"
REDUCE = "void kx::(anonymous namespace)::splitk_reduce_kernel<false>(int)"


def test_profile_summary_leaves_the_warmup_out(tmp_path, capsys):
    launches = [{"label": "gemm a", "entry": "kx_gemm_bf16", "flops": 2e12, "bytes": 0},
                {"label": "gemm b", "entry": "kx_gemm_splitk_bf16", "flops": 1e12, "bytes": 0}]
    (tmp_path / "launches.json").write_text(json.dumps(launches))
    warmup, timed = 3, 4
    dispatches = []
    for block in range(warmup + timed):
        slow = block < warmup
        dispatches += [(GEMM, 2000.0 if slow else 1000.0 + block), (SPLIT, 300.0), (REDUCE, 20.0 if slow else 10.0)]
    _trace(tmp_path / "trace", dispatches)
    assert bench.profile_summary(str(tmp_path), warmup) == 0
    out = capsys.readouterr().out
    rows = {line.split("|")[2].strip(): line.split("|") for line in out.splitlines() if line.startswith("| ")}
    gemm_a = sum(1000.0 + b for b in range(warmup, warmup + timed)) / timed
    assert float(rows["gemm a"][4]) == round(gemm_a, 1)
    assert float(rows["gemm b"][4]) == 310.0  # both dispatches of the split launch, timed blocks only
    assert f"over the {timed} timed blocks, after {warmup} warm-up blocks" in out
    assert f"{(gemm_a + 310.0) / 1e3:.3f} ms" in out


def test_kernel_table_divides_by_every_traced_step(tmp_path, capsys):
    warmup, steps = 1, 2
    total_steps = warmup + 2 * steps
    _trace(tmp_path / "kdn", [(GEMM, 100.0), (GEMM, 100.0), (REDUCE, 10.0)] * total_steps)
    assert bench.kernel_table(str(tmp_path / "kdn"), warmup + 2 * steps) == 0
    out = capsys.readouterr().out
    gemm = next(line.split("|") for line in out.splitlines() if "gemm_lds_kernel" in line)
    assert int(gemm[3]) == 2 * total_steps and int(gemm[4]) == 2  # calls, calls per step
    assert "Sum of this library's kernels: 0.2 ms per step." in out
