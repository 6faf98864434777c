"""CPU check of the constant-divisor division the int32 LINQ interpreter uses
(dotcompute_amd/csrc/dc_intdiv.hpp): host build of tests/cpp/intdiv_check.hip, every quotient
compared with int64 truncating division (C#'s int `/`)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_magic_division_matches_truncating_division(tmp_path):
    exe = tmp_path / "intdiv_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "--offload-arch=gfx950",
                    os.path.join(ROOT, "tests", "cpp", "intdiv_check.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
