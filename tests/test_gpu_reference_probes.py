"""The reference's own speculative-decoding programs run on the GPU through
libq38hip: src/cli/qwen38_spec_bench.c and qwen38_spec_probe.c, compiled from
the reference's sources and linked against libq38hip.so (oracle/Makefile,
built in the container that holds the reference; skipped where they were not
built).  Each program checks, itself, that speculative greedy decoding
reproduces plain greedy decoding (qwen38_spec_bench.c:100-119,
qwen38_spec_probe.c:87-96) and exits non-zero otherwise.  They run on the
Q4_K_M synthetic model (random weights: every draft rejected) and on the
"accept" checkpoint pair with its separate MTP file (drafts accepted)."""
import os
import subprocess

import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")


def program(name):
    path = os.path.join(REF_DIR, name)
    if not os.path.exists(path):
        pytest.skip("%s not built (needs the reference sources)" % name)
    return path


def run(args):
    print(" ".join(os.path.basename(a) for a in args), flush=True)
    out = subprocess.run(args, capture_output=True, text=True, timeout=540)
    print(out.stdout, out.stderr, flush=True)
    return out


@pytest.mark.parametrize("variant", ["q4km", "accept"])
def test_reference_spec_bench_on_gpu(device, variant):
    from conftest import synthetic_model
    bench = program("qwen38-spec-bench-hip")
    args = [bench, synthetic_model(variant)]
    if variant == "accept":
        args.append(synthetic_model("accept_mtp"))
    out = run(args)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    assert lines[0].startswith("mode=baseline")
    assert [l.split()[1] for l in lines[1:5]] == ["depth=1", "depth=2", "depth=3", "depth=4"]
    if variant == "accept":
        # accepted drafts: fewer transactions than tokens at depth 4
        assert int(lines[4].split()[2].split("=")[1]) < 15


def test_reference_spec_probe_on_gpu(device):
    from conftest import synthetic_model
    probe = program("qwen38-spec-probe-hip")
    out = run([probe, synthetic_model("accept"), synthetic_model("accept_mtp")])
    assert out.returncode == 0, out.stderr


def test_reference_kernel_unit_test_on_gpu(device):
    """tests/unit/test_qwen38_quant.c of the reference, linked against
    libq38hip.so: its known answers for every format, its portable
    restatements of the IQ kernels on random blocks, GEMM-equals-GEMV over
    batch sizes 1..7, the IQ1_S repack identity and the F32 path, all through
    this library's GPU kernels."""
    out = run([program("test-qwen38-quant-hip")])
    assert out.returncode == 0, out.stderr
    assert "qwen38 quant: ok" in out.stdout
