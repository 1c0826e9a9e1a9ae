"""The device restatement of the C library's expf (questwend_amd/csrc/
qwm_expf.h) equals this image's libm expf on every one of the 2^32 float
inputs.  ggml-CPU calls libm expf in the sigmoid (shared-expert gate, sigmoid
routing) and in the scalar tails of soft_max and silu, so these bits are the
CPU's.  The header is compiled for the host here (g++ with OpenMP); the GPU
tests then see the device copy reproduce the oracle's results bit for bit."""
import os
import subprocess

import numpy as np

from tests.helpers import ROOT, oracle


def test_libm_expf_restatement_every_float(tmp_path):
    exe = str(tmp_path / "expf_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fopenmp", "-ffp-contract=off", "-o", exe,
                    os.path.join(ROOT, "tests", "expf_check.cpp")], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    assert out[0] == "0", f"{out[0]} mismatches, first at input bits 0x{out[1]}"


def test_oracle_sigmoid_is_libm():
    """The oracle's sigmoid is 1 / (1 + expf(-x)) with the C library's expf
    (ggml-cpu unary-ops.cpp:31-33); known values and the fp64 closed form."""
    xs = np.array([0.0, 1.0, -1.0, 10.0, -10.0, 88.0, -88.0, 0.5], np.float32)
    got = np.array([oracle().qwo_sigmoid(float(v)) for v in xs], np.float32)
    assert got[0] == 0.5
    ref = (1.0 / (1.0 + np.exp(-xs.astype(np.float64)))).astype(np.float32)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 2 * np.spacing(ref))
    assert np.float32(oracle().qwo_expf(0.0)) == 1.0
