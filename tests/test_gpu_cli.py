"""The reference CLI on the GPU: src/cli/qwen38_main.c compiled from the
reference's sources and linked against libq38hip.so (oracle/_ref/qwen38-hip,
oracle/Makefile), run on the synthetic 27B Q4_K_M model with the arguments
of each case in tests/golden/cli_q4km_s1.json, whose stdout the same CLI
built whole from the reference's sources (model and kernels on the CPU)
wrote (tests/golden/make_cli_golden.py).

Each run tokenizes the prompt through the chat template, prefills it,
generates (greedy, greedy with MTP verification at depth 3 and 5, and
sampled with top-k / top-p / presence penalty on the host logits) and
detokenizes, as the CLI does on a real checkpoint (src/cli/qwen38_main.c:
349-433, 481-592).  Bar: stdout identical byte for byte.

The same CLI's OpenAI-compatible server (--server PORT, qwen38_main.c:
1145-1396) runs on the loopback port with the fixture's server arguments
and answers the fixture's chat-completion requests (plain JSON and
server-sent events, greedy with and without MTP, sampled): every reply's
content, finish reason and token counts equal the reference server's."""
import json
import os
import subprocess

import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "cli_q4km_s1.json")
CLI = os.path.join(ROOT, "oracle", "_ref", "qwen38-hip")


def _golden(key):
    if not os.path.exists(GOLDEN):
        return []
    with open(GOLDEN) as f:
        return json.load(f).get(key, [])


@pytest.fixture(scope="module")
def model_path(device):
    from conftest import synthetic_model
    if not os.path.exists(CLI):
        pytest.skip("reference CLI not linked (oracle/_ref/qwen38-hip)")
    return synthetic_model("q4km")


@pytest.mark.parametrize("case", _golden("cases"), ids=lambda c: c["name"])
def test_cli_output_matches_reference(model_path, case):
    print("case %s: %s" % (case["name"], " ".join(case["args"])), flush=True)
    out = subprocess.run([CLI, "--model", model_path] + case["args"], capture_output=True, timeout=500)
    assert out.returncode == 0, out.stderr.decode(errors="replace")[-2000:]
    assert out.stdout.decode("utf-8") == case["stdout"], (out.stdout[:200], case["stdout"][:200])


@pytest.mark.parametrize("run", _golden("servers"), ids=lambda r: r["name"])
def test_server_replies_match_reference(model_path, run):
    from golden.make_cli_golden import run_server
    print("server %s: %s" % (run["name"], " ".join(run["args"])), flush=True)
    replies = run_server(CLI, model_path, run["args"], run["requests"], timeout=300)
    assert replies == run["replies"]
