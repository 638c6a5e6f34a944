"""bench.py's reading of rocprofv3 counter-collection CSVs (roofline.traffic
measured in the run): a counter summed over its dimensions per dispatch,
averaged over the headline GEMV's dispatches, and the calibration copy's
figure; the scale factors applied as live_traffic applies them."""
import csv

import pytest

import bench

FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
          "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
          "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]

GEMV = "void hk::gemv_tiled_kernel<1, 2, 5, 1, false, false>(hk::OrganView const*, unsigned int, float const*)"
COPY = "__amd_rocclr_copyBuffer"


def write_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for did, name, counter, value in rows:
            r = {k: "0" for k in FIELDS}
            r.update(Dispatch_Id=str(did), Kernel_Name=name, Counter_Name=counter, Counter_Value=str(value))
            w.writerow(r)


def test_sums_dimensions_and_averages_headline(tmp_path):
    p = tmp_path / "run_counter_collection.csv"
    # the copy (dispatch 1), a fill that is neither (2), three headline dispatches
    # whose counter comes in two dimensions each, and another counter ignored
    write_csv(p, [(1, COPY, "FETCH_SIZE", 262160.0),
                  (2, "__amd_rocclr_fillBufferAligned", "FETCH_SIZE", 99.0),
                  (3, GEMV, "FETCH_SIZE", 300000.0), (3, GEMV, "FETCH_SIZE", 323000.0),
                  (4, GEMV, "FETCH_SIZE", 310000.0), (4, GEMV, "FETCH_SIZE", 313000.0),
                  (5, GEMV, "FETCH_SIZE", 311000.0), (5, GEMV, "FETCH_SIZE", 312006.0),
                  (5, GEMV, "WRITE_SIZE", 16384.0)])
    mean_kib, copy_kib = bench.pmc_headline_and_copy([str(p)], "FETCH_SIZE")
    assert copy_kib == 262160.0
    assert mean_kib == pytest.approx((623000.0 + 623000.0 + 623006.0) / 3)
    # live_traffic's scaling: KiB per dispatch x (512 MiB in KiB / copy KiB)
    factor = bench.PMC_CALIB_MB * 1024.0 / copy_kib
    assert factor == pytest.approx(1.99988, rel=1e-5)


def test_rejects_a_pass_without_headline_or_copy(tmp_path):
    p = tmp_path / "run_counter_collection.csv"
    write_csv(p, [(1, COPY, "WRITE_SIZE", 524288.0), (2, GEMV, "WRITE_SIZE", 16384.0)])
    with pytest.raises(RuntimeError):
        bench.pmc_headline_and_copy([str(p)], "WRITE_SIZE")  # one headline dispatch only
    q = tmp_path / "b_counter_collection.csv"
    write_csv(q, [(d, GEMV, "WRITE_SIZE", 16384.0) for d in range(3)])
    with pytest.raises(RuntimeError):
        bench.pmc_headline_and_copy([str(q)], "WRITE_SIZE")  # no copy
