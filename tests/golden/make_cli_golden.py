#!/usr/bin/env python3
"""Golden output of the reference CLI (src/cli/qwen38_main.c) on the
synthetic 27B Q4_K_M model: the CLI built whole from the reference's own
sources, model and kernels included (oracle/_ref/qwen38-ref, oracle/Makefile),
run on the CPU in this container.

The synthetic GGUF carries a byte-level BPE tokenizer
(qwen3.8-27b-in-c_amd/synth/q38_synth_gguf.c), so the CLI tokenizes the
prompt through its chat template, prefills it, generates and detokenizes as
it would on a real checkpoint (src/cli/qwen38_main.c:481-592, the MTP loop
:349-433).  Each case stores the CLI's arguments and its stdout bytes; the
GPU test runs the same CLI sources linked against libq38hip.so
(oracle/_ref/qwen38-hip) with the same arguments and compares stdout byte for
byte (tests/test_gpu_cli.py).

The OpenAI-compatible server of the same CLI (--server PORT,
src/cli/qwen38_main.c:1145-1396) is run the same way: SERVER_RUNS start it
with their arguments, send their chat-completion requests (plain JSON and
server-sent events) to the loopback port, and store each reply's
content, finish reason and token counts.

Run from the repository root (about 20 min on 8 cores):
  python tests/golden/make_cli_golden.py [GGUF_PATH]
"""
import json
import os
import socket
import subprocess
import sys
import time
import urllib.request

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "qwen3.8-27b-in-c_amd"))

SEED = 1
# (name, arguments after --model PATH)
CASES = [
    ("greedy", ["--context", "512", "--prompt", "hello there", "--temperature", "0", "--max-tokens", "32",
                "--no-thinking"]),
    ("greedy_mtp", ["--context", "512", "--prompt", "hello there", "--temperature", "0", "--max-tokens", "32",
                    "--no-thinking", "--mtp"]),
    ("mtp_depth5_system", ["--context", "512", "--system", "Answer in one line.", "--prompt", "the cat sat",
                           "--temperature", "0", "--max-tokens", "20", "--mtp", "--mtp-depth", "5"]),
    ("sampled", ["--context", "512", "--prompt", "write a haiku", "--temperature", "0.8", "--top-k", "20",
                 "--top-p", "0.95", "--seed", "7", "--max-tokens", "24"]),
    ("sampled_presence", ["--context", "512", "--prompt", "tell me", "--no-thinking", "--seed", "11",
                          "--max-tokens", "24"]),
]

# (name, server arguments after --model PATH, requests: chat-completion bodies)
SERVER_RUNS = [
    ("server", ["--context", "512", "--no-thinking"], [
        {"model": "qwen3.8-27b-in-c", "messages": [{"role": "user", "content": "hello there"}],
         "temperature": 0, "max_tokens": 16},
        {"model": "qwen3.8-27b-in-c", "messages": [{"role": "system", "content": "Be brief."},
                                                  {"role": "user", "content": "the cat sat"}],
         "temperature": 0.7, "top_p": 0.9, "seed": 5, "max_tokens": 12, "stream": True},
        {"model": "qwen3.8-27b-in-c", "messages": [{"role": "user", "content": "hello there"}],
         "temperature": 0, "max_tokens": 16},
    ]),
    ("server_mtp", ["--context", "512", "--no-thinking", "--mtp", "--temperature", "0"], [
        {"model": "qwen3.8-27b-in-c", "messages": [{"role": "user", "content": "hello there"}],
         "temperature": 0, "max_tokens": 16},
        {"model": "qwen3.8-27b-in-c", "messages": [{"role": "user", "content": "and again"}],
         "temperature": 0, "max_tokens": 10, "stream": True},
    ]),
]


def free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def post(port, body, timeout):
    """One chat-completion request; for a streamed reply the content of the
    server-sent deltas joined and the last finish reason"""
    req = urllib.request.Request("http://127.0.0.1:%d/v1/chat/completions" % port, data=json.dumps(body).encode(),
                                 headers={"Content-Type": "application/json"})
    with urllib.request.urlopen(req, timeout=timeout) as r:
        raw = r.read().decode("utf-8")
    if not body.get("stream"):
        reply = json.loads(raw)
        choice = reply["choices"][0]
        return {"content": choice["message"]["content"], "finish_reason": choice["finish_reason"],
                "usage": reply["usage"]}
    content, finish = [], None
    for line in raw.splitlines():
        if not line.startswith("data: ") or line == "data: [DONE]":
            continue
        event = json.loads(line[6:])
        for choice in event.get("choices", []):
            content.append(choice.get("delta", {}).get("content") or "")
            finish = choice.get("finish_reason") or finish
    return {"content": "".join(content), "finish_reason": finish}


def run_server(cli, model, args, requests, timeout=600):
    """Start `cli --model MODEL --server PORT args`, wait for /health, send
    `requests` in order, stop the server; the replies"""
    port = free_port()
    proc = subprocess.Popen([cli, "--model", model, "--server", str(port)] + args, stdout=subprocess.PIPE,
                            stderr=subprocess.PIPE, env=dict(os.environ, QWEN38_THREADS=str(os.cpu_count() or 8)))
    try:
        deadline = time.time() + timeout
        while True:
            if proc.poll() is not None:
                raise RuntimeError("server exited: %s" % proc.stderr.read().decode(errors="replace")[-2000:])
            try:
                with urllib.request.urlopen("http://127.0.0.1:%d/health" % port, timeout=5) as r:
                    if r.status == 200:
                        break
            except OSError:
                pass
            if time.time() > deadline:
                raise RuntimeError("server did not come up")
            time.sleep(0.5)
        return [post(port, body, timeout) for body in requests]
    finally:
        proc.terminate()
        try:
            proc.wait(timeout=30)
        except subprocess.TimeoutExpired:
            proc.kill()
            proc.wait()


def main():
    from q38hip import synth
    path = sys.argv[1] if len(sys.argv) > 1 else synth.model_path(SEED, "q4km")
    synth.write_model_gguf(path, SEED, "q4km")
    cli = os.path.join(ROOT, "oracle", "_ref", "qwen38-ref")
    if not os.path.exists(cli):
        raise SystemExit("build the reference CLI first: make -C oracle")
    cases = []
    for name, args in CASES:
        t0 = time.time()
        out = subprocess.run([cli, "--model", path] + args, capture_output=True, check=True,
                             env=dict(os.environ, QWEN38_THREADS=str(os.cpu_count() or 8)))
        stdout = out.stdout.decode("utf-8")
        print("[%6.1f s] %s: %r" % (time.time() - t0, name, stdout[:80]), flush=True)
        cases.append({"name": name, "args": args, "stdout": stdout})
    greedy = {c["name"]: c["stdout"] for c in cases}
    if greedy["greedy"] != greedy["greedy_mtp"]:
        raise AssertionError("reference CLI: MTP output differs from greedy output")
    servers = []
    for name, args, requests in SERVER_RUNS:
        t0 = time.time()
        replies = run_server(cli, path, args, requests)
        print("[%6.1f s] %s: %s" % (time.time() - t0, name, [r["content"][:40] for r in replies]), flush=True)
        servers.append({"name": name, "args": args, "requests": requests, "replies": replies})
    dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cli_q4km_s%d.json" % SEED)
    with open(dest, "w") as f:
        json.dump({"seed": SEED, "variant": "q4km", "cases": cases, "servers": servers}, f, indent=1)
    print("wrote " + dest)


if __name__ == "__main__":
    main()
