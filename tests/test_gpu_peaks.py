"""The measured peaks bench.py reports beside the vendor's nominal ones:
presk_hip_mfma_probe's MFMA rates (independent MFMA loops on every CU) and
the HBM rate of a plain copy nest.  A rate above the nominal peak would mean
the loops were not run as counted; far below it, that they stalled."""
import ctypes

import pytest

import bench
from presk_amd import hip

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ty,vendor", [("bf16", 2500.0), ("f32", 157.3)])
def test_mfma_probe_rate(ty, vendor):
    hip.init(0)
    ms, fl = ctypes.c_double(), ctypes.c_double()
    hip.check(hip.lib().presk_hip_mfma_probe(ty.encode(), 4000, None, ctypes.byref(ms), ctypes.byref(fl)))
    rate = fl.value / (ms.value * 1e-3) / 1e12
    print(f"[peaks] {ty}: {rate:.1f} TFLOP/s ({ms.value:.3f} ms)", flush=True)
    assert 0.3 * vendor < rate <= 1.02 * vendor


def test_measured_peaks_record():
    p = bench.measured_peaks()
    print(f"[peaks] {p}", flush=True)
    assert 0.3 * 2500 < p["mfma_bf16_tflops"] <= 1.02 * 2500
    assert 0.3 * 157.3 < p["mfma_f32_tflops"] <= 1.02 * 157.3
    assert 1000 < p["hbm_copy_gbs"] <= 8000
    roof = bench.with_measured({"bound": "mfma", "achieved": 100.0}, "f32", p)
    assert roof["frac_of_measured"] == round(100.0 / p["mfma_f32_tflops"], 4)
