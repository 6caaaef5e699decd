"""The executor's environment switches, without a GPU: PRESK_HIP_MODE (the
parity switch), PRESK_HIP_GEMM_TILE (contraction tiles and k splits in place
of the planner's) and PRESK_HIP_DEVICE, each malformed value refused by
presk_hip_init before any device is touched."""
import ctypes

import pytest

from presk_amd import hip, lower as L

A, O = L.ax, L.Operand


def dot(m, k, n, dt):
    return L.dot([O(A(("seq", m), ("model", k))), O(A(k, n))], dt)


def compiled(low, mode=hip.FAST):
    return hip.Compiled(low.text, low.dtype, low.lanes, mode)


def test_mode_switch_forces_exact(monkeypatch):
    low = dot(256, 512, 256, "f32")
    assert compiled(low).kind == "gemm"
    exact = compiled(low, hip.EXACT)
    monkeypatch.setenv("PRESK_HIP_MODE", "exact")
    forced = compiled(low, hip.FAST)
    assert (forced.kind, forced.order) == (exact.kind, exact.order) and forced.kind != "gemm"
    monkeypatch.setenv("PRESK_HIP_MODE", "fast")
    assert compiled(low, hip.EXACT).kind == "gemm"


def test_tile_override(monkeypatch):
    bf = dot(2048, 1024, 2048, "bf16")
    f32 = dot(256, 8192, 256, "f32")
    assert compiled(bf).order == "mfma-k16"          # the planner: 128 x 128 tiles of 32x32x16 MFMAs
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x96")
    assert compiled(bf).order == "mfma-k32"          # 128 x 96 tiles of 16x16x32 MFMAs
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "256x256")
    assert compiled(bf).order == "mfma-k16"
    assert compiled(f32).order.startswith("mfma-f32-k4")  # no 256 x 256 f32 tiles: the planner's
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "256x96")
    assert compiled(f32).order == "mfma-f32-k4"      # f32 256-row tiles: never split
    assert compiled(bf).order == "mfma-k16"          # no 256 x 96 16-bit tiles: the planner's
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x64/4")
    assert compiled(f32).order == "mfma-f32-k4-split4"
    assert compiled(bf).order == "mfma-k16-split4"
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x96/4")
    assert compiled(bf).order == "mfma-k32-split4"
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x128/1")
    assert compiled(f32).order == "mfma-f32-k4"


def test_eight_wave_tile_override(monkeypatch):
    # `w8` after 128x128: the eight-wave 128 x 128 tiles, split or not, in
    # both storage families; the order names the same MFMAs and split
    f32, bf = dot(256, 8192, 256, "f32"), dot(256, 8192, 256, "bf16")
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x128w8/7")
    assert compiled(f32).order == "mfma-f32-k4-split7"
    assert compiled(bf).order == "mfma-k16-split7"
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x128w8/1")
    assert compiled(f32).order == "mfma-f32-k4"
    monkeypatch.setenv("PRESK_HIP_GEMM_TILE", "128x128w8")      # no split named: the planner's
    assert compiled(f32).order.startswith("mfma-f32-k4-split")
    # (without a GPU init fails for the missing device, never for the switch)
    if hip.lib().presk_hip_init(-1) != 0:
        assert "PRESK_HIP_GEMM_TILE" not in hip.lib().presk_hip_last_error().decode()


@pytest.mark.parametrize("var,value", [("PRESK_HIP_GEMM_TILE", "256x64"), ("PRESK_HIP_GEMM_TILE", "128x128/0"),
                                       ("PRESK_HIP_GEMM_TILE", "128x64w8"), ("PRESK_HIP_GEMM_TILE", "256x128w8"),
                                       ("PRESK_HIP_GEMM_TILE", "128x128w4"),
                                       ("PRESK_HIP_GEMM_TILE", "128x128x"), ("PRESK_HIP_MODE", "fastest"),
                                       ("PRESK_HIP_DEVICE", "one")])
def test_malformed_switch_fails_init(monkeypatch, var, value):
    monkeypatch.setenv(var, value)
    assert hip.lib().presk_hip_init(-1) != 0
    msg = hip.lib().presk_hip_last_error().decode()
    assert msg.startswith("E10001") and var in msg
