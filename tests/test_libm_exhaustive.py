"""q38_expf and q38_logf (qwen3.8-27b-in-c_amd/csrc/q38_libm.h) against the
host C library's expf and logf on all 2^32 float inputs, bit for bit (CPU
only, about 20 s on 8 cores).  The reference engine evaluates its
exponentials and logarithms with the host C library
(src/qwen38/qwen38_model.c:439, 444, 554, 771, 867)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_logf_match_host_libm_on_every_float(tmp_path):
    exe = str(tmp_path / "libm_check")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "qwen3.8-27b-in-c_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "libm_check.c"), "-o", exe, "-lm"], check=True)
    lines = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.splitlines()
    seen = {}
    for line in lines:
        name, _, checked, _, mismatches, _, first = line.split()
        seen[name] = (int(checked), int(mismatches), first)
    assert set(seen) == {"expf", "logf"}
    for name, (checked, mismatches, first) in seen.items():
        assert checked == 1 << 32, name
        assert mismatches == 0, "%s: %d mismatches (first input bits %s)" % (name, mismatches, first)
