"""The integer emulation of sequential f32 folds (hi_amd/csrc/exact_fold.h),
built for the host, against a literal left-to-right f32 fold: term by term,
runs of equal terms, and threshold searches (tests/native/fold_check.cpp)."""
import os
import subprocess


def test_exact_fold_matches_sequential_fold(tmp_path):
    here = os.path.dirname(__file__)
    src = os.path.join(here, "native", "fold_check.cpp")
    inc = os.path.join(os.path.dirname(here), "hi_amd", "csrc")
    exe = tmp_path / "fold_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I", inc, src, "-o", str(exe),
                    "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and "mismatches 0" in out.stdout, out.stdout
    cases = int(out.stdout.split("cases ")[1].split()[0])
    assert cases > 200000
