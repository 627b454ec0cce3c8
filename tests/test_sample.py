"""The GPU sampler's expf (agent-serve_amd/csrc/expf_libm.hpp) against the host libm's expf,
which the reference's sample_logits calls (sampler.cpp:29): every float argument in
[-128, -0] must give the same bits. Host code only (hipcc compiles the header for the host)."""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("hipcc") is None and not pathlib.Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_expf_restatement_matches_libm_exhaustively(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    exe = tmp_path / "expf_check"
    subprocess.run([hipcc, "-O2", "-std=c++17", f"-I{ROOT / 'agent-serve_amd' / 'csrc'}", "-o", str(exe),
                    str(ROOT / "tests" / "expf_check.cpp"), "-pthread"], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600)
    assert out.stdout.strip() == "0", f"{out.stdout.strip()} arguments differ from libm's expf"
