"""Host-compiled checks of device helpers that also build for the CPU.

- q8_bounds_check: the Q8_0 half-block read geometry of the gather kernels
  (synthesize.cpp_amd/csrc/shp_q8.hpp) reads only inside a row, for every lane
  of every row width the kernels take, and decodes each lane's scale and quants.
- trig_check: the rope's double-precision cos/sin (shp_trig.hpp) rounds to the
  same f32 as libm's double sin/cos.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "synthesize.cpp_amd", "csrc")


def _build_and_run(tmp_path, name):
    exe = tmp_path / name
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-I" + CSRC, "-o", str(exe),
                    os.path.join(HERE, "host", name + ".cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    return r.returncode, r.stdout


def test_q8_half_block_reads_stay_inside_the_row(tmp_path):
    rc, out = _build_and_run(tmp_path, "q8_bounds_check")
    checked, failures = map(int, out.split()[-2:])
    assert rc == 0 and failures == 0 and checked > 2000, out


def test_rope_sincos_is_correctly_rounded(tmp_path):
    rc, out = _build_and_run(tmp_path, "trig_check")
    assert rc == 0, out
