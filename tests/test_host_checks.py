"""Host-compiled checks of device helpers that also build for the CPU.

- q8_bounds_check: the Q8_0 half-block read geometry of the gather kernels
  (synthesize.cpp_amd/csrc/shp_q8.hpp) reads only inside a row, for every lane
  of every row width the kernels take, and decodes each lane's scale and quants.
- q5k_window_check: the Q5_K gather->sum windows (shp_q5k.hpp) read only inside
  each lane's super-block, tile the slab, and decode the scale, min and quants
  of ggml's byte layout.
- trig_check: the rope's double-precision cos/sin (shp_trig.hpp) rounds to the
  same f32 as libm's double sin/cos.
- div_check: Snake's division by a per-channel double reciprocal (shp_div.hpp)
  gives the IEEE f32 quotient, also with a reciprocal one ulp off, and the
  device's Newton steps give that reciprocal.
- sinf_check: Snake's branch-free sine (shp_sinf.hpp) is within 1 ulp of the
  correctly rounded sine over its whole range.
- expf_check: the table-driven exp of the softmax, SnakeBeta and ggml_exp
  (shp_expf.hpp) against the double exp rounded once, over all 2^32 f32 inputs
  (multi-threaded, ~30 s on 8 cores).
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "synthesize.cpp_amd", "csrc")


def _build_and_run(tmp_path, name):
    exe = tmp_path / name
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-ffp-contract=off", "-I" + CSRC, "-o", str(exe),
                    os.path.join(HERE, "host", name + ".cpp"), "-lm", "-pthread"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    return r.returncode, r.stdout


def test_q8_half_block_reads_stay_inside_the_row(tmp_path):
    rc, out = _build_and_run(tmp_path, "q8_bounds_check")
    checked, failures = map(int, out.split()[-2:])
    assert rc == 0 and failures == 0 and checked > 2000, out


def test_q5k_window_reads_and_decoding(tmp_path):
    rc, out = _build_and_run(tmp_path, "q5k_window_check")
    checked, failures = map(int, out.split()[-2:])
    assert rc == 0 and failures == 0 and checked == 2000 * 64, out


def test_rope_sincos_is_correctly_rounded(tmp_path):
    rc, out = _build_and_run(tmp_path, "trig_check")
    assert rc == 0, out


def test_snake_division_by_reciprocal_is_the_ieee_quotient(tmp_path):
    rc, out = _build_and_run(tmp_path, "div_check")
    pairs, bad, rcps, rcp_bad = map(int, out.split()[-4:])
    assert rc == 0 and bad == 0 and rcp_bad == 0 and pairs > 10 ** 7 and rcps > 10 ** 6, out


def test_snake_fast_sine_within_one_ulp(tmp_path):
    rc, out = _build_and_run(tmp_path, "sinf_check")
    tested, worst, _exact, _glibc = out.split()[-4:]
    assert rc == 0 and int(tested) > 8 * 10 ** 6 and float(worst) <= 1.0, out


def test_table_exp_matches_the_rounded_double_exp_on_every_input(tmp_path):
    """At most 1 ulp anywhere, NaN kept, and mismatches on at most 1 input in
    10^6 (measured: 19 of 4,294,967,296; glibc's expf: 170,648)."""
    rc, out = _build_and_run(tmp_path, "expf_check")
    inputs, mismatches, max_ulp, _glibc = map(int, out.split()[-4:])
    assert rc == 0 and inputs == 2 ** 32 and max_ulp <= 1 and mismatches <= 100, out
