"""Drop-in link test of the model and kernel ABIs, CPU only: the reference's
own CLI and model probes (src/cli/qwen38_main.c, qwen38_spec_bench.c,
qwen38_spec_probe.c, qwen38_mtp_probe.c, qwen38_batch_probe.c,
qwen38_forward_probe.c, qwen38_logits_probe.c) and its kernel unit test
(tests/unit/test_qwen38_quant.c), compiled from its sources by
oracle/Makefile and linked against libq38hip.so in place of its model and
kernel objects, link with no unresolved symbol, and the reference's model
header and include/q38model.h declare the same functions.  Needs the reference sources
(this container); the GPU run of the linked probes is in
tests/test_gpu_reference_probes.py."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
LINKED = ["qwen38-hip"] + ["qwen38-%s-hip" % p for p in
                           ("spec-bench", "spec-probe", "mtp-probe", "batch-probe", "forward-probe", "logits-probe")] + \
    ["test-qwen38-quant-hip"]

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src", "cli")),
                                reason="reference sources not present")


@pytest.fixture(scope="module")
def linked():
    if not os.path.exists(os.path.join(ROOT, "qwen3.8-27b-in-c_amd", "libq38hip.so")):
        pytest.skip("libq38hip.so not built")
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
    return REF_DIR


def test_reference_programs_link_against_libq38hip(linked):
    lib = os.path.realpath(os.path.join(ROOT, "qwen3.8-27b-in-c_amd", "libq38hip.so"))
    for name in LINKED:
        path = os.path.join(linked, name)
        assert os.path.exists(path), name
        ldd = subprocess.run(["ldd", path], capture_output=True, text=True, check=True).stdout
        line = [l for l in ldd.splitlines() if "libq38hip.so" in l]
        assert line and "not found" not in line[0], ldd
        assert os.path.realpath(line[0].split("=>")[1].split("(")[0].strip()) == lib


def test_reference_cli_runs(linked):
    out = subprocess.run([os.path.join(linked, "qwen38-hip"), "--help"], capture_output=True, text=True,
                         timeout=60)
    assert out.returncode == 0
    assert "--mtp-depth" in out.stdout + out.stderr


def test_model_header_matches_reference(tmp_path):
    """One C translation unit includes the reference's qwen38_model.h and
    include/q38model.h: every shared prototype must be identical, or the C
    compiler rejects the redeclaration."""
    src = tmp_path / "both.c"
    src.write_text('#include "qwen38_model.h"\n#include "q38model.h"\nint main(void) { return 0; }\n')
    subprocess.run(["gcc", "-std=c11", "-Werror", "-Wall", "-I", os.path.join(REF, "include", "qwen38"),
                    "-I", os.path.join(ROOT, "include"), str(src), "-o", str(tmp_path / "both")],
                   check=True, capture_output=True)
