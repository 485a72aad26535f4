"""The drop-in under its real caller: the reference's own server
(sml/sml-server.c, compiled from its sources into oracle/_ref/sml-server with
this repository's library linked in place of its GPU object, as
sml/Makefile:111-116 links sml-gpu-lib.o) serves a chat turn on the card, and
the same binary on the reference's CPU path (--device cpu) gives the same
reply, token for token, when the library runs in exact mode (SML_EXACT=1: the
CPU path's float order) and the CPU server reads prompts per 32 values
(SML_PROMPT_SB=0, equal to stepping).

The synthetic model gets a byte-fallback vocabulary in the reference's binary
vocabulary format (sml/sml-vocab.c:64-78: counts, bos, eos, offsets, bytes,
no merges): 256 "<0xNN>" byte tokens, the ChatML markers the server looks for
(sml/sml-server.c:1615-1621) and filler words, so that the server's template,
prompt probe (sml/sml-server.c:1622-1681) and greedy generation all run.
"""
import json
import os
import socket
import struct
import subprocess
import time
import urllib.request

import pytest

import sheep_amd as sa
from sheep_amd import ssf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SERVER = os.path.join(ROOT, "oracle", "_ref", "sml-server")
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(SERVER), reason="oracle/_ref/sml-server not built "
                                 "(the reference's sources were absent at build time)")]


def add_vocab(path, n_vocab):
    """Append a byte-fallback vocabulary of n_vocab tokens to an SSF file and
    point the header's tok_off / tok_n at it."""
    toks = [f"<0x{b:02X}>".encode() for b in range(256)] + [s.encode() for s in SPECIALS]
    toks += [f"▁w{i}".encode() for i in range(len(toks), n_vocab)]
    assert len(toks) == n_vocab
    offs = [0]
    for t in toks:
        offs.append(offs[-1] + len(t))
    bos, eos = 256, 258
    blob = struct.pack("<4I", n_vocab, 0, bos, eos) + struct.pack(f"<{n_vocab + 1}I", *offs) + b"".join(toks)
    names = ssf.HEADER_FIELDS
    fmt = ssf.HEADER_FMT
    # byte offset of a header field: the packed format's size up to it
    codes = []
    i = 1
    while i < len(fmt):
        j = i
        while fmt[j].isdigit():
            j += 1
        n = int(fmt[i:j]) if j > i else 1
        c = fmt[j]
        codes += [c] if c == "s" else [c] * n
        if c == "s":
            codes[-1] = fmt[i:j + 1]
        i = j + 1
    assert len(codes) == len(names)
    at = {nm: struct.calcsize("<" + "".join(codes[:k])) for k, nm in enumerate(names)}
    with open(path, "r+b") as f:
        f.seek(0, 2)
        end = f.tell()
        off = (end + 255) // 256 * 256
        f.write(b"\0" * (off - end) + blob)
        f.seek(at["tok_off"])
        f.write(struct.pack("<Q", off))
        f.seek(at["tok_n"])
        f.write(struct.pack("<Q", len(blob)))


def free_port():
    with socket.socket(socket.AF_INET, socket.SOCK_STREAM) as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def http(port, path, body=None, timeout=60):
    req = urllib.request.Request(f"http://127.0.0.1:{port}{path}",
                                 data=None if body is None else json.dumps(body).encode(),
                                 headers={"Content-Type": "application/json"})
    with urllib.request.urlopen(req, timeout=timeout) as r:
        return r.read()


def serve_turn(model, device, workdir, messages, env=None, args=()):
    """Start the server on the model, wait for /health, run one greedy chat
    turn, read /stats, stop the server. Returns (reply text, stats, log)."""
    port = free_port()
    log_path = os.path.join(workdir, f"server_{device}.log")
    with open(log_path, "w") as log:
        print(f"starting sml-server --device {device} {' '.join(args)} on port {port}", flush=True)
        p = subprocess.Popen([SERVER, "-m", model, "--port", str(port), "-c", "256", "--threads", "4",
                              "--device", device, *args], stdout=log, stderr=subprocess.STDOUT, cwd=workdir,
                             env=dict(os.environ, **(env or {})))
        try:
            deadline = time.time() + 90
            while True:
                if p.poll() is not None:
                    raise AssertionError(f"server exited {p.returncode}: {open(log_path).read()[-2000:]}")
                try:
                    http(port, "/health", timeout=5)
                    break
                except OSError:
                    if time.time() > deadline:
                        raise AssertionError(f"server not up after 90 s: {open(log_path).read()[-2000:]}")
                    time.sleep(0.5)
            raw = http(port, "/v1/chat/completions",
                       {"messages": messages, "max_tokens": 24, "temperature": 0, "cache": False})
            reply = json.loads(raw.decode("utf-8", errors="replace"))
            stats = json.loads(http(port, "/stats").decode("utf-8", errors="replace"))
        finally:
            p.terminate()
            try:
                p.wait(timeout=20)
            except subprocess.TimeoutExpired:
                p.kill()
                p.wait(timeout=20)
    return reply["choices"][0]["message"]["content"], stats, open(log_path).read()


@pytest.mark.parametrize("mode", ["exact", "fast"])
def test_reference_server_on_this_library(tmp_path, mode):
    """exact: the library in exact mode serves the same reply as the CPU path,
    token for token, on a zero-mean synthetic model whose reply takes several
    distinct words. fast: the default kernels; the reference's own soundness
    rule for a GPU prompt path applies (the first 4 words equal,
    sml/sml-server.c:1668-1673)."""
    model = str(tmp_path / "chat.ssf")
    sa.synth_model(model, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, random_perm=True, seed=7)
    add_vocab(model, 2000)
    msgs = [{"role": "user", "content": "Name three rivers in Africa, one per line."}]
    gpu_env = {"SML_EXACT": "1" if mode == "exact" else "0"}
    gpu_text, gpu_stats, gpu_log = serve_turn(model, "gpu", str(tmp_path), msgs, gpu_env)
    assert gpu_stats["device"] == "gpu", gpu_log[-2000:]
    assert gpu_stats["gpu_layers"] == gpu_stats["gpu_of"] == 2, gpu_stats
    assert gpu_stats["last_gen"] > 0 and gpu_stats["template"] == "chatml", gpu_stats
    cpu_text, cpu_stats, cpu_log = serve_turn(model, "cpu", str(tmp_path), msgs, {"SML_PROMPT_SB": "0"})
    assert cpu_stats["device"] == "cpu", cpu_log[-2000:]
    assert gpu_stats["last_prompt"] == cpu_stats["last_prompt"] == 61
    assert len(gpu_text) > 0
    if mode == "exact":
        assert len(set(cpu_text.split())) >= 4, cpu_text
        assert gpu_stats["last_gen"] == cpu_stats["last_gen"]
        assert gpu_text == cpu_text, (gpu_text, cpu_text)
    else:
        assert gpu_text.split()[:4] == cpu_text.split()[:4], (gpu_text, cpu_text)


def test_reference_server_hybrid_split(tmp_path):
    """--device hybrid --gpu-layers 1 on a two-layer model: the library keeps
    one layer's matrices on the card and streams the other's, the server
    reports the split as hybrid (sml/sml-server.c:1596-1604), and in exact
    mode the reply equals the CPU path's token for token."""
    model = str(tmp_path / "chat.ssf")
    sa.synth_model(model, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, random_perm=True, seed=7)
    add_vocab(model, 2000)
    msgs = [{"role": "user", "content": "Name three rivers in Africa, one per line."}]
    gpu_text, gpu_stats, gpu_log = serve_turn(model, "hybrid", str(tmp_path), msgs, {"SML_EXACT": "1"},
                                              ("--gpu-layers", "1"))
    assert gpu_stats["device"] == "hybrid", gpu_log[-2000:]
    assert (gpu_stats["gpu_layers"], gpu_stats["gpu_of"]) == (1, 2), gpu_stats
    cpu_text, cpu_stats, cpu_log = serve_turn(model, "cpu", str(tmp_path), msgs, {"SML_PROMPT_SB": "0"})
    assert len(set(cpu_text.split())) >= 4, cpu_text
    assert gpu_stats["last_gen"] == cpu_stats["last_gen"]
    assert gpu_text == cpu_text, (gpu_text, cpu_text)


@pytest.mark.parametrize("fail", ["open:40", "prefill:2", "step:90"])
def test_reference_server_falls_back_to_cpu(tmp_path, fail):
    """The library fails one entry point (SML_GPU_FAIL): the 40th HIP call of
    the open; the second prompt the server reads (its load-time probe,
    sml/sml-server.c:1622-1681, reads the first); or the 90th step, the fifth
    token of the reply (the probe steps 61 prompt ids and 2 x 12 tokens
    first). The server keeps serving: it retires the GPU and finishes on its
    CPU path (sml/sml-server.c:204-265), and, the library running exact, the
    reply equals the CPU server's."""
    model = str(tmp_path / "chat.ssf")
    sa.synth_model(model, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, random_perm=True, seed=7)
    add_vocab(model, 2000)
    msgs = [{"role": "user", "content": "Name three rivers in Africa, one per line."}]
    env = {"SML_EXACT": "1", "SML_GPU_FAIL": fail, "SML_PROMPT_SB": "0"}
    text, stats, log = serve_turn(model, "gpu", str(tmp_path), msgs, env)
    cpu_text, cpu_stats, _ = serve_turn(model, "cpu", str(tmp_path), msgs, {"SML_PROMPT_SB": "0"})
    assert stats["device"] == "cpu", (stats, log[-2000:])
    assert "serving on the CPU" in log or fail.startswith("open"), log[-2000:]
    assert text == cpu_text, (text, cpu_text, log[-2000:])
