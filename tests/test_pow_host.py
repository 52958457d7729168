"""The device pow of whitematter_amd/csrc/wm_pow.hpp, compiled for the host
(the header is plain C++ with explicit fma), checked against long double
powl.  Runs on the CPU: no GPU needed."""
import os
import subprocess


def test_pow_tables_host_build_against_powl(tmp_path):
    """The device pow (whitematter_amd/csrc/wm_pow.hpp) compiled for the host,
    against long double powl on a million random and special operand pairs:
    pow within 1 ulp with the C library's NaN / infinity / zero pattern, and
    the backward's three parts within their documented bounds."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = str(tmp_path / "pow_table_check")
    subprocess.run(["g++", "-std=c++17", "-O2", os.path.join(root, "tests", "cpp", "pow_table_check.cpp"), "-o", exe],
                   check=True)
    r = subprocess.run([exe, "1000000"], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and "POW CHECK PASSED" in r.stdout, r.stdout + r.stderr
