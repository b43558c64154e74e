"""The host side of bench.py, on the CPU: the one-GPU rule, the CPU baseline
over workloads 1-5, the algorithmic byte counts the roofline divides by, and
the rocprofv3 summarisers that write profiles/ (fed small synthetic CSVs)."""

import csv
import os
import subprocess
import sys

import pytest

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402
import numpy as np  # noqa: E402

import oracle  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout == ""


def test_algorithmic_bytes_match_the_workload_definitions():
    # add+RMSNorm [8192, 2048] bf16: R x, R delta, W x', W h, R w (fp32)
    assert bench.bytes_add_rms_norm(8192, 2048, 2) == 134_225_920
    # SwiGLU [8192, 2 x 1408] -> [8192, 1408] bf16
    assert bench.bytes_swiglu(8192, 1408, 2) == 69_206_016
    # RoPE Q [8192, 16, 128] + K [8192, 4, 128] bf16 in place + int64 positions
    assert bench.bytes_rope(8192, 20, 128, 2) == 83_951_616
    # fp32 RMSNorm [1024, 2048] and the vision pair LayerNorm + GELU [4096, 1024] bf16
    assert bench.bytes_rms_norm(1024, 2048, 4) == 16_785_408
    assert bench.bytes_layer_norm(4096, 1024, 2) + bench.bytes_gelu(4096 * 1024, 2) == 33_562_624
    assert (bench.bytes_add_rms_norm(8192, 2048, 2) + bench.bytes_swiglu(8192, 1408, 2)
            + bench.bytes_rope(8192, 20, 128, 2)) == 287_383_552


def test_cpu_workloads_report_every_workload():
    cpu = bench.cpu_workloads(0.01, 2)
    assert set(cpu) == {"1", "2", "3", "4", "5"}
    for c in ("1", "3", "4", "5"):
        assert cpu[c]["ms"] > 0 and cpu[c]["gbps"] > 0 and cpu[c]["runs"] >= 3
    assert cpu["2"]["us"] > 0
    for c in ("1", "2", "3", "4", "5"):
        assert cpu[c]["runs"] >= 20  # at least 20 timed runs after 3 warm-ups
    info = bench.host_cpu()
    assert info["nproc"] >= 1 and 1 <= info["affinity"] <= info["nproc"] and info["model"]
    line = bench.cpu_baseline(cpu, 2, info)
    assert line["kind"] == "port" and line["cores"] == 2 and line["unit"] == "GB/s"
    assert line["value"] == cpu["5"]["gbps"] and line["value_1_thread"] > 0
    assert line["cpu_model"] == info["model"] and line["nproc"] == info["nproc"]


def test_decode_chain_in_one_call_is_the_composed_ops():
    """orc_decode_chain (workload 2's CPU figure in one C call) is the
    gather, add + RMSNorm and the two ropes, bit for bit."""
    g = np.random.default_rng(3)
    cols, qh, kh, dim, token, pos = 256, 4, 2, 64, 5, 777
    table = oracle.f32_to_bf16(g.standard_normal((9, cols), dtype=np.float32))
    delta = g.standard_normal(cols, dtype=np.float32)
    w = (1 + 0.02 * g.standard_normal(cols)).astype(np.float32)
    q0 = g.standard_normal(qh * dim, dtype=np.float32)
    k0 = g.standard_normal(kh * dim, dtype=np.float32)
    inv = oracle.rope_inv(dim // 2, 1e4)
    x, h, q, k = np.empty(cols, np.float32), np.empty(cols, np.float32), q0.copy(), k0.copy()
    p = lambda a: a.ctypes.data  # noqa: E731
    oracle.lib().orc_decode_chain(p(table), token, p(delta), p(w), p(x), p(h), cols, 1e-6, p(q), qh, p(k), kh, dim,
                                  pos, p(inv), dim // 2, 1)
    want_x, want_h = oracle.add_rms_norm(oracle.embed(table, np.array([token])).ravel(), delta, w, 1e-6)
    tok = np.array([pos], np.int64)
    assert np.array_equal(x, want_x) and np.array_equal(h, want_h)
    assert np.array_equal(q, oracle.rope(q0.reshape(1, -1), qh, dim, tok=tok, inv_tok=inv).ravel())
    assert np.array_equal(k, oracle.rope(k0.reshape(1, -1), kh, dim, tok=tok, inv_tok=inv).ravel())


def _write_csv(path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def test_trace_summary_takes_durations_per_kernel_and_grid(tmp_path):
    rows = []
    for i, dur in enumerate([4000, 5000, 6000]):
        rows.append({"Kernel_Name": "void uocr_rocm::(anonymous namespace)::rope_rows<unsigned short, 8>(Args)",
                     "Grid_Size": "262144", "Workgroup_Size": "128", "Start_Timestamp": str(1000 * i),
                     "End_Timestamp": str(1000 * i + dur)})
    rows.append({"Kernel_Name": "at::native::vectorized_elementwise_kernel<4>(int)", "Grid_Size": "64",
                 "Workgroup_Size": "64", "Start_Timestamp": "0", "End_Timestamp": "900"})
    _write_csv(tmp_path / "run_kernel_trace.csv", list(rows[0]), rows)
    table = bench.summarize_trace(str(tmp_path))
    lines = table.splitlines()
    assert len(lines) == 3  # header, rule, one kernel: torch's own kernels are left out
    assert "rope_rows<unsigned short, 8>" in lines[2]
    assert "| 262144 | 128 | 3 | 5.00 | 5.00 | 4.00 |" in lines[2]


def test_pmc_summary_counts_each_request_at_its_size(tmp_path):
    """Bytes = 32/64/128 per sized read request and 64/32 per write request;
    a 256 MiB copy issued as 128-byte reads and 64-byte writes comes out at
    256 MiB each way, with no scale factor."""
    copy = bench.COPY_KERNEL
    n128, n64w = bench.COPY_BYTES // 128, bench.COPY_BYTES // 64
    r32, r64, r128 = bench.PMC_PASS_READS
    rall, wall, w64 = bench.PMC_PASS_WRITES

    def rows(kernel, grid, values):
        return [{"Kernel_Name": kernel, "Grid_Size": grid, "Counter_Name": c, "Counter_Value": str(v)}
                for c, v in values.items()]
    reads = rows(copy, "131072", {r32: 0, r64: 0, r128: n128}) + \
        rows("norm_rows<float>(float*)", "256", {r32: 10, r64: 20, r128: 30})
    writes = rows(copy, "131072", {rall: n128, wall: n64w, w64: n64w}) + \
        rows("norm_rows<float>(float*)", "256", {rall: 61, wall: 7, w64: 5})
    (tmp_path / "r").mkdir()
    (tmp_path / "w").mkdir()
    _write_csv(tmp_path / "r" / "run_counter_collection.csv", list(reads[0]), reads)
    _write_csv(tmp_path / "w" / "run_counter_collection.csv", list(writes[0]), writes)
    table = bench.summarize_pmc(str(tmp_path / "r"), str(tmp_path / "w"))
    copy_row = [ln for ln in table.splitlines() if copy in ln][0]
    assert copy_row.endswith(f"| {bench.COPY_BYTES} | {bench.COPY_BYTES} | {2 * bench.COPY_BYTES} |")
    row = [ln for ln in table.splitlines() if "norm_rows" in ln][0]
    read_b, write_b = 32 * 10 + 64 * 20 + 128 * 30, 64 * 5 + 32 * 2
    assert row.endswith(f"| {read_b} | {write_b} | {read_b + write_b} |")
    assert "| 1 |" in row  # one read request of unknown size (61 - 60)


def test_committed_traffic_reads_the_profile():
    got = bench.committed_traffic("norm_rows<unsigned short, 8, 1, 4, (Norm)1", 8192 * 64)
    if not os.path.exists(bench.TRAFFIC_FILE):
        pytest.skip("no committed PMC summary")
    assert got is not None and abs(got - 134_225_920) / 134_225_920 < 0.01
