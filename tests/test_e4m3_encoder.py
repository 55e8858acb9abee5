"""The product's FP8 store arithmetic (csrc/fa_device.h; the functions the
store kernels run), checked on the CPU by tests/native/e4m3_check.hip
(compiled for the host by hipcc):

* e4m3_code against the oracle's C codec (oracle/fp8_e4m3.c, itself pinned to
  torch's cast and the reference's rounding table) on every one of the 2^32
  fp32 bit patterns;
* div_by_scale (reciprocal + one FMA residual step) against IEEE division on
  every finite bf16 and fp16 input, over 4000 scales.
Each sweep takes a few seconds on 8 cores."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
NATIVE = ROOT / "tests" / "native"
BUILD = NATIVE / "_build"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _checker():
    exe = BUILD / "e4m3_check"
    sources = [NATIVE / "e4m3_check.hip", ROOT / "flash-attn-mps_amd" / "csrc" / "fa_device.h",
               ROOT / "oracle" / "fp8_e4m3.c"]
    if exe.exists() and all(exe.stat().st_mtime > s.stat().st_mtime for s in sources):
        return exe
    BUILD.mkdir(exist_ok=True)
    subprocess.run(["gcc", "-O2", "-std=c11", "-fno-fast-math", "-c", str(ROOT / "oracle" / "fp8_e4m3.c"),
                    "-o", str(BUILD / "fp8_oracle.o")], check=True)
    subprocess.run([HIPCC, "-O2", "-std=c++17", "--offload-arch=gfx950", "-c", str(NATIVE / "e4m3_check.hip"),
                    "-o", str(BUILD / "e4m3_check.o")], check=True, capture_output=True)
    subprocess.run([HIPCC, "--offload-arch=gfx950", str(BUILD / "e4m3_check.o"), str(BUILD / "fp8_oracle.o"),
                    "-o", str(exe), "-lpthread"], check=True, capture_output=True)
    return exe


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc is needed to build the host checker")
def test_encoder_matches_the_c_codec_on_every_fp32_pattern():
    run = subprocess.run([str(_checker()), "enc", "1"], capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "all 4294967296 patterns agree" in run.stdout


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc is needed to build the host checker")
def test_reciprocal_division_is_correctly_rounded():
    run = subprocess.run([str(_checker()), "div", "4000"], capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "division agrees on 4000 scales" in run.stdout
