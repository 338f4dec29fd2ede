"""The client side of the serve-directory protocol (the reference's ml-eval/fhe_client.py:1394-1492,
serve_roundtrip and stop_server): hand a request to a running server and wait for its answer.

Request N inside the directory: the ciphertext files req.N.0 .. req.N.<count-1>, the one-line JSON meta req.N.meta,
optionally req.N.reset (written before the ready marker, so the server sees it with the same request), and
req.N.ready last.  The answer is complete when resp.N.done exists and req.N.ready no longer does (the server removes
the ready marker after writing done); resp.N.error means the server refused or failed the request.
"""
from __future__ import annotations

import json
import os
import time

META_KEYS = ("count", "packTokens", "tokensReal", "dpad", "interleave", "lanes", "ringDim", "level")


def request_meta(count: int, lanes: int, level: int, tokens_real: int | None = None, pack_tokens: int = 1,
                 dpad: int = 1024, interleave: int = 0, ring_dim: int = 1 << 16) -> str:
    """the meta sidecar's one line, keys in the reference's order (gpu_real_model.cu:2332-2339)"""
    vals = {"count": count, "packTokens": pack_tokens, "tokensReal": count if tokens_real is None else tokens_real,
            "dpad": dpad, "interleave": interleave, "lanes": lanes, "ringDim": ring_dim, "level": level}
    return json.dumps({k: int(vals[k]) for k in META_KEYS}, separators=(",", ":")) + "\n"


def submit(directory: str, n: int, write_file, count: int, meta: str, reset: bool = False) -> None:
    """request n: write_file(t, path) writes ciphertext t; then the meta; the reset marker; the ready marker last"""
    req = os.path.join(directory, f"req.{n}")
    if reset:
        with open(f"{req}.reset", "w") as f:
            f.write("reset\n")
    for t in range(count):
        write_file(t, f"{req}.{t}")
    with open(f"{req}.meta", "w") as f:
        f.write(meta)
    with open(f"{req}.ready", "w") as f:
        f.write("ready\n")


class ServeError(RuntimeError):
    pass


def wait(directory: str, n: int, timeout: float = 600.0, poll: float = 0.05, alive=None) -> str:
    """wait for request n's answer; returns the response prefix.  Raises ServeError on resp.n.error, on a server
    that `alive()` reports dead, or on timeout."""
    req = os.path.join(directory, f"req.{n}")
    resp = os.path.join(directory, f"resp.{n}")
    t0 = time.time()
    while True:
        if os.path.exists(f"{resp}.done") and not os.path.exists(f"{req}.ready"):
            return resp
        if os.path.exists(f"{resp}.error"):
            raise ServeError(f"server reported an error for request {n}")
        if alive is not None and not alive():
            raise ServeError(f"server exited while serving request {n}")
        if time.time() - t0 > timeout:
            raise ServeError(f"no answer to request {n} within {timeout} s")
        time.sleep(poll)


def response_meta(directory: str, n: int) -> dict:
    with open(os.path.join(directory, f"resp.{n}.meta")) as f:
        return json.loads(f.read())


def status(directory: str) -> dict | None:
    """serve.status ({"nextReq","served","pid","stateful","storeFile"}), None before the server wrote it"""
    p = os.path.join(directory, "serve.status")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.loads(f.read())


def stop(directory: str) -> None:
    with open(os.path.join(directory, "stop"), "w") as f:
        f.write("stop\n")
