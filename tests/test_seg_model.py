"""The CPU model of the draft verify's exact sequential-sum engine (tests/cpp/seg_model.cpp):
the segment records with their crossing data, the walk and its crossing shortcut, the one-wave
exact segments and the residual draw's search,
transliterated from turbo-winfare-dense_amd/csrc/verify.hip over a simulated 64-lane wave.
1,600 rows of six kinds (softmax terms, residual terms, exact half-way ties, powers of two,
terms near 0.5, zeros with tiny and sparse big terms), 1,000 to 300,000 terms, each summed
without a stop, with a stop threshold inside the sum, and through the residual draw's search,
bit for bit against the in-order fp32 loop, with asserts on every LDS index, on the values the
device code keeps uniform across the wave, and on the progress of every loop."""
import os
import subprocess

from helpers import ROOT


def test_segmented_sum_model(tmp_path):
    exe = tmp_path / "seg_model"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-Wall", "-Werror",
                    os.path.join(ROOT, "tests", "cpp", "seg_model.cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    res = subprocess.run([str(exe), "1600"], capture_output=True, text=True, timeout=900)
    print(res.stdout)
    assert res.returncode == 0 and "MODEL OK" in res.stdout, res.stdout + res.stderr
