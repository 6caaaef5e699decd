"""bench.py's traffic table (`--traffic-table`) on synthetic rocprofv3 counter
files: the regions cut at the marker launches (`pk_traffic_mark`, the
runtime's own fill kernels left out), each launch's three calls averaged,
every KiB scaled by what the copy probe's region reads against the probe's
known 256 MiB, `__`-keys left out of the table, and a region count that does
not match the keys refused."""
import csv
import json

import pytest

import bench

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def write_csv(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (kname, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": kname, "Counter_Name": counter, "Counter_Value": value})


def regions(probe, a, b):
    """marker, 3 probe dispatches, marker, setup, marker, 3 of A (a fill
    kernel among them), marker, 3 of B, marker (the end)."""
    m = ("pk_traffic_mark_p0", 1.0)
    return ([m] + [("pk_neg_p0", probe)] * 3 + [m, ("pk_setup", 9999.0), m]
            + [("pk_a_p0", a), ("__amd_rocclr_fillBufferAligned", 5000.0), ("pk_a_p0", a), ("pk_a_p0", a)]
            + [m] + [("pk_b_p0", b)] * 3 + [m])


def test_traffic_table_scales_by_the_copy_probe(tmp_path):
    keys = {"keys": ["__copy_probe__", "__setup__", "kernel a | generic sequential", "kernel b | gemm mfma-k16", "__end__"],
            "src_sha": "0123456789abcdef"}
    kp = tmp_path / "keys.json"
    kp.write_text(json.dumps(keys))
    probe = 4 << 26                              # bytes the probe reads (and writes)
    # FETCH counts half the probe's bytes (factor 2), WRITE all of them (factor 1)
    write_csv(tmp_path / "f.csv", "FETCH_SIZE", regions(probe / 1024 / 2, 100.0, 7.0))
    write_csv(tmp_path / "w.csv", "WRITE_SIZE", regions(probe / 1024, 10.0, 3.0))
    out = tmp_path / "traffic.json"
    bench.traffic_table(str(kp), str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(out))
    d = json.loads(out.read_text())
    assert d["src_sha"] == "0123456789abcdef"
    assert "FETCH x 2.000" in d["method"] and "WRITE x 1.000" in d["method"]
    got = {x["key"]: x for x in d["launches"]}
    assert list(got) == ["kernel a | generic sequential", "kernel b | gemm mfma-k16"]
    a, b = got["kernel a | generic sequential"], got["kernel b | gemm mfma-k16"]
    assert a["fetch_bytes"] == 100 * 1024 * 2 and a["write_bytes"] == 10 * 1024 and a["dispatches"] == 1
    assert b["fetch_bytes"] == 7 * 1024 * 2 and b["write_bytes"] == 3 * 1024
    assert a["bytes_per_launch"] == a["fetch_bytes"] + a["write_bytes"]


def test_traffic_table_refuses_a_missing_region(tmp_path):
    keys = {"keys": ["__copy_probe__", "__setup__", "kernel a", "kernel b", "kernel c", "__end__"], "src_sha": "x"}
    kp = tmp_path / "keys.json"
    kp.write_text(json.dumps(keys))
    write_csv(tmp_path / "f.csv", "FETCH_SIZE", regions(1.0, 1.0, 1.0))
    write_csv(tmp_path / "w.csv", "WRITE_SIZE", regions(1.0, 1.0, 1.0))
    with pytest.raises(SystemExit, match="6 regions expected, 5 / 5 found"):
        bench.traffic_table(str(kp), str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "t.json"))
