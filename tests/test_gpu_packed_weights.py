"""GPU: CpuPackedWeights through the C++ drop-in (tests/cpp/packed_weights_check.cpp,
built by `make -C quixicore-cpu_amd`), as the reference's
tests/correctness/test_packed_weights.cpp exercises it, plus canonical int8
tensors.  The program checks the reference test's assertions itself (info
fields, the panel index formula with its zero-padded tail, qgemm_prepacked
against qgemm for M in {1, 3, 17, 65}, workspace reuse, the invalid layout
99); here every prepared panel (panel bytes plus side tables) and info
record is compared byte for byte with what the reference's own
CpuPackedWeights (oracle/_ref, built from the reference sources) makes of
the same inputs -- including kAuto, which both resolve from this host's CPU.
"""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "quixicore-cpu_amd", "lib", "packed_weights_check")
LAYOUTS = {"auto": 0, "portable_rows1": 1, "neon_rows4": 2, "avx2_rows8": 3, "avx512_rows16": 4}
N, K = 19, 64


@pytest.fixture(scope="module")
def run(qc, tmp_path_factory):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built (make -C quixicore-cpu_amd)")
    out = tmp_path_factory.mktemp("packed")
    print("running packed_weights_check", flush=True)
    r = subprocess.run([BINARY, str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    cases = [line.split()[0] for line in open(out / "manifest.txt")]
    return out, cases


def _load(out, name):
    info = np.fromfile(out / f"{name}.info", dtype=np.int64)
    panel = np.fromfile(out / f"{name}.panel", dtype=np.uint8)
    inp = np.fromfile(out / f"{name}.in", dtype=np.uint8)
    return info, panel, inp


def test_program_ran_every_case(run):
    out, cases = run
    for fmt in ("q4_0", "q8_0"):
        for lay in LAYOUTS:
            assert f"{fmt}_{lay}" in cases
    for lay in list(LAYOUTS)[1:]:
        assert f"smoothquant_{lay}" in cases and f"affine_group32_{lay}" in cases


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("lay", list(LAYOUTS))
def test_gguf_panel_and_info_match_reference(run, ref, fmt, lay):
    out, _ = run
    info, panel, packed = _load(out, f"{fmt}_{lay}")
    st, want_panel, want_info = ref.prepare_gguf(0 if fmt == "q8_0" else 1, packed, N, K,
                                                 LAYOUTS[lay])
    assert st == 0
    assert np.array_equal(info, want_info), (info, want_info)
    assert np.array_equal(panel, want_panel)


@pytest.mark.parametrize("lay", list(LAYOUTS)[1:])
def test_canonical_panels_match_reference(run, ref, lay):
    out, _ = run
    w = np.fromfile(out / "canon_w.in", dtype=np.int8).reshape(N, K)
    ws = np.fromfile(out / "canon_ws.in", dtype=np.float32)
    as_ = np.fromfile(out / "canon_as.in", dtype=np.float32)
    azp = np.fromfile(out / "canon_azp.in", dtype=np.int32)
    info, panel, _ = _load(out, f"smoothquant_{lay}")
    st, want_panel, want_info = ref.prepare_smoothquant(w, ws, as_, azp, LAYOUTS[lay])
    assert st == 0
    assert np.array_equal(info, want_info), (info, want_info)
    assert np.array_equal(panel, want_panel)
    scales = np.fromfile(out / "canon_af_scales.in", dtype=np.float32)
    zps = np.fromfile(out / "canon_af_zps.in", dtype=np.float32)
    info, panel, _ = _load(out, f"affine_group32_{lay}")
    st, want_panel, want_info = ref.prepare_canonical_int8(1, w, N, K, 32, 4, scales, zps,
                                                           layout=LAYOUTS[lay])
    assert st == 0
    assert np.array_equal(info, want_info), (info, want_info)
    assert np.array_equal(panel, want_panel)
