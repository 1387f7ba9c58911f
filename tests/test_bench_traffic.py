"""bench.py's HBM-traffic summary (host logic, no GPU): rocprofv3 --pmc
FETCH_SIZE / WRITE_SIZE rows per dispatch and XCD, scaled by the 512 MiB
calibration copy, attributed to the roofline kernels by their template
arguments; the folded-LayerNorm forms (gemm_nt_ln_kernel) are preferred when
the run launched them. Also that the committed summary under profiles/
describes the kernels the default bf16 forward launches."""
import csv
import json
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import bench  # noqa: E402

COPY = "__amd_rocclr_copyBuffer"
RES_FOLD = "_ZN12_GLOBAL__N_117gemm_nt_ln_kernelIDF16bLi256ELi192ELi128ELi2ELi5ELi2ELi4ELi2EEEv8GemmArgs6LnFold"
RES_PLAIN = "_ZN12_GLOBAL__N_114gemm_nt_kernelIDF16bLi256ELi192ELi128ELi2ELi0ELi2ELi4ELi2EEEv8GemmArgs"
QKV_FOLD = "_ZN12_GLOBAL__N_117gemm_nt_ln_kernelIDF16bLi256ELi128ELi64ELi3ELi6ELi2ELi2ELi2EEEv8GemmArgs6LnFold"
WI_PLAIN = "_ZN12_GLOBAL__N_114gemm_nt_kernelIDF16bLi256ELi128ELi64ELi3ELi2ELi2ELi2ELi2EEEv8GemmArgs"
LN = "void (anonymous namespace)::ln_kernel<bool _Accum, int, E, 0, 4>(float const*, int, int)"


def _write(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for disp, name, kib in rows:
            w.writerow([disp, name, counter, kib])


def test_summary_scales_sums_and_prefers_fold_forms(tmp_path):
    mib512 = 512 * 1024  # KiB
    # dispatch id, kernel, KiB (two rows for a dispatch split over XCDs are summed)
    fetch = [(1, COPY, mib512 // 2), (2, COPY, 100),
             (3, RES_FOLD, 1000), (3, RES_FOLD, 500), (4, RES_FOLD, 1500),
             (5, RES_PLAIN, 9999), (6, QKV_FOLD, 2000), (7, WI_PLAIN, 3000), (8, LN, 400), (9, LN, 400)]
    write = [(1, COPY, mib512), (3, RES_FOLD, 700), (4, RES_FOLD, 700), (6, QKV_FOLD, 100), (7, WI_PLAIN, 50),
             (8, LN, 20), (9, LN, 20)]
    _write(str(tmp_path / "f"), "FETCH_SIZE", fetch)
    _write(str(tmp_path / "w"), "WRITE_SIZE", write)
    out = str(tmp_path / "s.json")
    assert bench.summarize_traffic(str(tmp_path / "f"), str(tmp_path / "w"), out) == 0
    d = json.load(open(out))
    assert d["fetch_scale"] == pytest.approx(2.0) and d["write_scale"] == pytest.approx(1.0)
    k = d["kernels"]
    assert k["residual"]["symbol"] == RES_FOLD and k["residual"]["template_args"] == [256, 192, 128, 2, 5, 2, 4, 2]
    assert k["residual"]["dispatches"] == 2
    assert k["residual"]["fetch_bytes_per_launch"] == 1500 * 1024 * 2  # (1000 + 500) and 1500, times 2
    assert k["residual"]["write_bytes_per_launch"] == 700 * 1024
    T, H, I = 32768, bench.H, bench.I
    plain_res = (2 * (T * H + H * H) + 2 * (T * I + H * I) + 16 * T * H) / 2
    assert k["residual"]["algorithmic_bytes_per_launch"] == plain_res + 2 * T * H + 8 * T * (H // 192)
    assert k["qkv"]["symbol"] == QKV_FOLD
    assert k["qkv"]["algorithmic_bytes_per_launch"] == 2 * (T * H + 3 * H * H + 3 * T * H) + 40 * T
    # no folded Wi in this run: the plain form and its algorithmic bytes
    assert k["wi"]["symbol"] == WI_PLAIN and k["wi"]["template_args"][4] == 2
    assert k["wi"]["algorithmic_bytes_per_launch"] == 2 * (T * H + 2 * I * H + T * I)
    # the LayerNorm entry is the LayerNorm kernel, not the folded GEMM whose name contains "ln_kernel"
    assert d["other_kernels"]["layernorm"]["symbol"] == LN


def test_committed_summary_matches_the_default_forward():
    """profiles/gemm_traffic_cfg3.json is read by the bench only for the tiles
    it launches: with the folded LayerNorm (the bf16 default) every roofline
    kernel has its bytes; the plain forms' tiles are not in that summary."""
    fold = bench.read_traffic("cfg3", "bf16", True)
    assert set(fold) == {"residual", "wi", "qkv"} and all(v > 0 for v in fold.values())
    assert bench.read_traffic("cfg3", "bf16", False) == {}
    assert bench.read_traffic("cfg4", "bf16", True) == {}
