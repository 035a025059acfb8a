"""The reference's epoll server relinked against this repository's
libtinyinfer_llm.so: socket greedy == direct greedy.

oracle/Makefile builds oracle/_ref/tinyinfer_server from the reference's own
server/src/main.cpp with TI_SERVER_NATIVE=1 (reference server/CMakeLists.txt:22-29),
linked to tinyinfer_amd/libtinyinfer_llm.so.  As the reference's native socket
gate (reference server/tests/native_correctness.py:335-447): each case's tokens
are first generated directly through the library (one slot, the context closed
before the server starts), then the same prompts go over one TCP connection;
every request must get a FIRST response with the first token and a FINAL
response with exactly the direct tokens, status ok, 1 <= batch size <= max batch.

Wire format (reference server/include/protocol.hpp): a request frame is a
4-byte big-endian body length, then version u16 = 1, kind u16 (1 generate),
id u64, max_new u32, count u32 and count u32 token ids; a response frame is a
4-byte length (60 + 4 n), version, kind u16 (0x8001 final, 0x8002 first), id
u64, status u32, n u32, batch size u32, a reserved u32, four u64 timings and n
u32 tokens.
"""
import queue
import signal
import socket
import struct
import subprocess
import threading
import time
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SERVER = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "tinyinfer_server"
MAX_BATCH, CAPACITY, MAX_NEW = 8, 256, 32
FINAL, FIRST = 0x8001, 0x8002
# (offset, prompt length, new tokens): the reference gate's three cases and one
# longer generation that overlaps them in the server's batches.
CASES = [(0, 8, 1), (19, 17, 3), (53, 33, 5), (90, 20, 16)]


def say(*args):
    print("[case]", *args, flush=True)


def request_frame(ident, tokens, max_new):
    body = struct.pack(">HHQII", 1, 1, ident, max_new, len(tokens)) + struct.pack(f">{len(tokens)}I", *tokens)
    return struct.pack(">I", len(body)) + body


def read_exact(sock, n):
    out = b""
    while len(out) < n:
        chunk = sock.recv(n - len(out))
        if not chunk:
            raise ConnectionError("server closed the connection")
        out += chunk
    return out


def read_response(sock):
    (length,) = struct.unpack(">I", read_exact(sock, 4))
    body = read_exact(sock, length)
    version, kind, ident, status, n, batch, _ = struct.unpack(">HHQIIII", body[:28])
    assert version == 1 and length == 60 + 4 * n
    tokens = list(struct.unpack(f">{n}I", body[60:60 + 4 * n]))
    return {"kind": kind, "id": ident, "status": status, "batch_size": batch, "tokens": tokens}


def free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


@pytest.fixture(scope="module")
def artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import GPT2_SMALL, write_synthetic
    say("writing GPT-2 small synthetic artifact for the server")
    return write_synthetic(tmp_path_factory.mktemp("gpt2srv"), GPT2_SMALL, seed=42)


def test_socket_greedy_equals_direct(artifact):
    if not SERVER.exists():
        pytest.skip("oracle/_ref/tinyinfer_server not built (needs the reference checkout at build time)")
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    frozen = np.random.default_rng(2026).integers(0, 50257, 128).tolist()
    prompts = [frozen[o:o + n] for o, n, _ in CASES]
    expected = []
    say("direct greedy through the library")
    with NativeModel(LLM_LIB, artifact, max_batch=MAX_BATCH, cache_slots=MAX_BATCH, capacity=CAPACITY) as model:
        for prompt, (_, _, count) in zip(prompts, CASES):
            model.reset_all()
            result = model.greedy([prompt], count, slots=[0])
            assert result["output_lengths"] == [count]
            expected.append(result["tokens"][0])
    port = free_port()
    argv = [str(SERVER), "--model", "native", "--manifest", str(artifact), "--host", "127.0.0.1",
            "--port", str(port), "--max-batch", str(MAX_BATCH), "--capacity", str(CAPACITY),
            "--max-new-tokens", str(MAX_NEW), "--device", "0"]
    say("starting relinked server on port", port)
    proc = subprocess.Popen(argv, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = queue.Queue()
    threading.Thread(target=lambda: [lines.put(l) for l in proc.stdout], daemon=True).start()
    try:
        deadline, ready = time.monotonic() + 120, None
        while ready is None and time.monotonic() < deadline:
            try:
                line = lines.get(timeout=0.5)
            except queue.Empty:
                assert proc.poll() is None, "server exited before readiness"
                continue
            if '"ready":true' in line:
                ready = line
        assert ready and '"model":"native"' in ready, "server did not report native readiness"
        say("server ready; sending", len(CASES), "requests on one connection")
        with socket.create_connection(("127.0.0.1", port), timeout=120) as sock:
            sock.sendall(b"".join(request_frame(i + 1, p, c[2]) for i, (p, c) in enumerate(zip(prompts, CASES))))
            first, final = {}, {}
            while len(final) < len(CASES):
                r = read_response(sock)
                i = r["id"] - 1
                assert 0 <= i < len(CASES) and i not in final, r
                assert r["status"] == 0 and 1 <= r["batch_size"] <= MAX_BATCH, r
                if r["kind"] == FIRST:
                    assert i not in first and r["tokens"] == expected[i][:1], (i, r, expected[i])
                    first[i] = r
                else:
                    assert r["kind"] == FINAL and i in first, r
                    assert r["tokens"] == expected[i], (i, r["tokens"], expected[i])
                    final[i] = r
        say("socket tokens equal direct tokens for", len(final), "requests; batch sizes",
            [final[i]["batch_size"] for i in sorted(final)])
    finally:
        proc.send_signal(signal.SIGTERM)
        try:
            proc.wait(timeout=30)
        except subprocess.TimeoutExpired:
            proc.kill()
            proc.wait(timeout=30)
