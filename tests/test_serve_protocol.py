"""The serve-directory protocol (host/serve.cpp, fhe_ssm_serve_dir) on the CPU, with a mock request handler in the
manner of the reference's ml-eval/mock_fhe_server.py: each request file holds float64 rows, the mock model is
hidden = 0.5 x + 0.5 carry with the carry kept per server (or dropped per request when stateless).  The real
handler (the decode step) is exercised on the GPU in test_gpu_decode.py.

What is checked is the protocol of gpu_real_model.cu:4363-4483 and :5525-5576 as its client
(ml-eval/fhe_client.py:1394-1492) relies on it: request numbering, the reset marker, stateless requests, the meta
sidecar, resp.N.done / resp.N.error, removal of the request files after the answer (ready last), serve.status,
the `stop` file and the idle timeout.
"""
import json
import os
import threading

import numpy as np
import pytest

from engine_loader import load_module

ND = load_module("native_decode")
SC = load_module("serve_client")


class Mock:
    def __init__(self, fail_on=()):
        self.carry = None
        self.calls = []
        self.fail_on = set(fail_on)

    def __call__(self, req, req_prefix, resp_prefix, meta, reset):
        self.calls.append((req, meta, reset))
        if req in self.fail_on:
            raise ValueError(f"mock failure on {req}")
        count, lanes = meta["count"], meta["lanes"]
        if reset or self.carry is None:
            self.carry = np.zeros((lanes, 4))
        for t in range(count):
            x = np.fromfile(f"{req_prefix}.{t}", dtype="<f8").reshape(lanes, 4)
            self.carry = 0.5 * x + 0.5 * self.carry
            self.carry.astype("<f8").tofile(f"{resp_prefix}.{t}")
        with open(f"{resp_prefix}.meta", "w") as f:
            f.write(SC.request_meta(count, lanes, meta["level"]))


def start(d, handler, **kw):
    box = {}
    log = open(os.path.join(d, "server.jsonl"), "w")

    def run():
        box["report"] = ND.serve_dir(str(d), handler, poll_ms=10, log_fd=log.fileno(), **kw)
    th = threading.Thread(target=run, daemon=True)
    th.start()
    return th, box, log


def finish(d, th, box, log):
    SC.stop(str(d))
    th.join(timeout=30)
    assert not th.is_alive()
    log.close()
    with open(os.path.join(d, "server.jsonl")) as f:
        events = [json.loads(l) for l in f if l.strip()]
    return box["report"], events


def send(d, n, rows, reset=False, lanes=2):
    def write(t, path):
        np.asarray(rows[t], dtype="<f8").tofile(path)
    SC.submit(str(d), n, write, len(rows), SC.request_meta(len(rows), lanes, 17), reset=reset)


def read(prefix, t, lanes=2):
    return np.fromfile(f"{prefix}.{t}", dtype="<f8").reshape(lanes, 4)


def test_stateful_requests_carry_and_reset(tmp_path):
    d = tmp_path
    mock = Mock()
    th, box, log = start(d, mock, stateful=True, timeout_sec=60)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 2, 4))
    send(d, 0, x[:2], reset=True)
    r0 = SC.wait(str(d), 0, timeout=30)
    # the request's files are gone once it is answered; the ready marker with them
    assert not any(os.path.exists(os.path.join(d, f"req.0.{s}")) for s in ("0", "1", "meta", "ready", "reset"))
    assert SC.response_meta(str(d), 0)["count"] == 2
    send(d, 1, x[2:3])
    r1 = SC.wait(str(d), 1, timeout=30)
    send(d, 2, x[3:4], reset=True)
    r2 = SC.wait(str(d), 2, timeout=30)
    rep, events = finish(d, th, box, log)
    # the carry runs through tokens of one request and across requests; the reset marker restarts it
    c = np.zeros((2, 4))
    want = []
    for t in range(3):
        c = 0.5 * x[t] + 0.5 * c
        want.append(c)
    np.testing.assert_array_equal(read(r0, 0), want[0])
    np.testing.assert_array_equal(read(r0, 1), want[1])
    np.testing.assert_array_equal(read(r1, 0), want[2])
    np.testing.assert_array_equal(read(r2, 0), 0.5 * x[3])
    assert [c[2] for c in mock.calls] == [True, False, True]
    assert rep == {"served": 3, "failed": 0, "next_req": 3, "exit_reason": "stop"}
    kinds = [e["serve"] for e in events]
    assert kinds.count("stateReset") == 2 and kinds.count("served") == 3 and kinds[-1] == "exit"
    assert events[-1]["reason"] == "stop"
    st = SC.status(str(d))
    assert st["nextReq"] == 3 and st["served"] == 3 and st["stateful"] is True and st["pid"] == os.getpid()


def test_stateless_server_starts_every_request_cold(tmp_path):
    d = tmp_path
    mock = Mock()
    th, box, log = start(d, mock, stateful=False, timeout_sec=60)
    x = np.ones((2, 2, 4))
    for n in range(2):
        send(d, n, x[n:n + 1])
        r = SC.wait(str(d), n, timeout=30)
        np.testing.assert_array_equal(read(r, 0), 0.5 * x[n])
    rep, _ = finish(d, th, box, log)
    assert [c[2] for c in mock.calls] == [True, True]
    assert rep["served"] == 2 and SC.status(str(d))["stateful"] is False


def test_bad_meta_and_handler_failure_answer_error(tmp_path):
    d = tmp_path
    mock = Mock(fail_on={2})
    th, box, log = start(d, mock, stateful=True, timeout_sec=60)
    # request 0: meta without tokensReal -> badRequest, only the ready marker is removed
    with open(os.path.join(d, "req.0.meta"), "w") as f:
        f.write('{"count":1,"lanes":2}\n')
    with open(os.path.join(d, "req.0.ready"), "w") as f:
        f.write("ready\n")
    with pytest.raises(SC.ServeError):
        SC.wait(str(d), 0, timeout=30)
    # request 1: no meta at all
    with open(os.path.join(d, "req.1.ready"), "w") as f:
        f.write("ready\n")
    with pytest.raises(SC.ServeError):
        SC.wait(str(d), 1, timeout=30)
    # request 2: the handler raises -> resp.2.error, the request's files still removed
    send(d, 2, np.zeros((1, 2, 4)))
    with pytest.raises(SC.ServeError):
        SC.wait(str(d), 2, timeout=30)
    # request 3 is served normally after the failures
    send(d, 3, np.ones((1, 2, 4)))
    SC.wait(str(d), 3, timeout=30)
    rep, events = finish(d, th, box, log)
    assert rep == {"served": 2, "failed": 3, "next_req": 4, "exit_reason": "stop"}
    assert [c[0] for c in mock.calls] == [2, 3]      # bad requests never reach the handler
    bad = [e for e in events if e["serve"] == "badRequest"]
    assert [e["req"] for e in bad] == [0, 1]
    failed = [e for e in events if e["serve"] == "served" and e["failed"]]
    assert len(failed) == 1 and "mock failure on 2" in failed[0]["error"]
    for n in (0, 1, 2):
        assert os.path.exists(os.path.join(d, f"resp.{n}.error")) and not os.path.exists(os.path.join(d, f"req.{n}.ready"))
    assert not os.path.exists(os.path.join(d, "req.2.0")) and not os.path.exists(os.path.join(d, "req.2.meta"))
    assert os.path.exists(os.path.join(d, "req.0.meta"))  # a bad request's other files stay for inspection


def test_idle_timeout_and_first_request_index(tmp_path):
    d = tmp_path
    rep = ND.serve_dir(str(d), Mock(), timeout_sec=1, poll_ms=20, first_req=5)
    assert rep == {"served": 0, "failed": 0, "next_req": 5, "exit_reason": "idleTimeout"}
    assert SC.status(str(d))["nextReq"] == 5


def test_stop_file_present_at_start(tmp_path):
    SC.stop(str(tmp_path))
    rep = ND.serve_dir(str(tmp_path), Mock(), timeout_sec=60, poll_ms=20)
    assert rep["exit_reason"] == "stop" and rep["served"] == 0


def test_refuses_a_missing_directory(tmp_path):
    with pytest.raises(RuntimeError, match="is not a directory"):
        ND.serve_dir(str(tmp_path / "absent"), Mock(), timeout_sec=1)


def test_meta_int_matches_whole_keys():
    """the sidecar reader finds a key by its quoted name and colon (gpu_real_model.cu:2327-2331)"""
    text = '{"count":3,"packTokens":1,"tokensReal":3,"dpad":1024,"interleave":0,"lanes":32,"ringDim":65536,"level":17}'
    assert ND.meta_int(text, "count") == 3 and ND.meta_int(text, "lanes") == 32 and ND.meta_int(text, "level") == 17
    assert ND.meta_int(text, "ringDim") == 65536
    assert ND.meta_int(text, "tokens", -7) == -7          # a prefix of tokensReal is not a key
    assert ND.meta_int('{"count":-2}', "count") == -2
    assert json.loads(SC.request_meta(3, 32, 17)) == json.loads(text)
    assert SC.request_meta(3, 32, 17).strip() == text     # the reference's key order, no spaces


def test_decoder_entry_points_refuse_null_arguments(tmp_path):
    """the decoder's serve and reset entry points check their arguments before any device work"""
    import ctypes
    lib = ND.load()
    opts = ND.ServeOpts(1, 10, 1, -1, 0)
    rep = ND.ServeReport()
    assert lib.fhe_ssm_decoder_serve(None, str(tmp_path).encode(), ctypes.byref(opts), ctypes.byref(rep)) != 0
    assert b"null" in lib.fhe_ssm_last_error()
    assert lib.fhe_ssm_decoder_reset(None) != 0
    seed = (ctypes.c_uint8 * 32)()
    assert lib.fhe_ssm_client_encrypt_rows(None, None, str(tmp_path / "r").encode(), 1, 1, 4, 4, 2, 2.0**40, seed) != 0
    assert b"null" in lib.fhe_ssm_last_error()
    assert lib.fhe_ssm_client_decrypt_logits(None, None, str(tmp_path / "r").encode(), None, 1, 4, 4) != 0
    assert b"null" in lib.fhe_ssm_last_error()


def test_log_matches_a_reference_session(tmp_path):
    """the log against a reference server session's (tests/golden/serve_log_reference.jsonl, extracted by
    tests/golden/extract_serve_log.py: its first two one-token requests, the first with the reset marker, then the
    end of the session): the same events in the same order, each carrying the reference line's keys and the same
    request numbers, token counts, served counts and failure flags.  The reference's per-stage timing keys of the
    served line (eval, bootstrap, layer-loop milliseconds, peak VRAM) are not produced here."""
    from conftest import GOLDEN
    ref = [json.loads(l) for l in open(os.path.join(GOLDEN, "serve_log_reference.jsonl"))]
    d = tmp_path
    th, box, log = start(d, Mock(), stateful=True, timeout_sec=60)
    send(d, 0, np.ones((1, 2, 4)), reset=True)
    SC.wait(str(d), 0, timeout=30)
    send(d, 1, np.ones((1, 2, 4)))
    SC.wait(str(d), 1, timeout=30)
    _, events = finish(d, th, box, log)
    want = ref[:7] + ref[-2:]  # two requests, then the waiting line that ends in `stop`, and the exit line
    assert [e["serve"] for e in events] == [e["serve"] for e in want]
    timing = {"reqEvalMs", "reqBootMs", "reqEncPtMs", "reqBoots", "reqNormBootMs", "reqMsPerTokenExBoot",
              "reqLayerLoopMs", "reqLayerLoopUntimedMs", "reqStageMs", "reqHostPtEncodeMs", "reqHostPtEncodeCount",
              "peakVramGB"}
    for i, (ours, theirs) in enumerate(zip(events, want)):
        keys = set(theirs) - (timing if theirs["serve"] == "served" else set())
        assert keys <= set(ours), (ours, theirs)
        if i < 7:
            for k in ("req", "tokens", "failed", "served"):
                if k in theirs:
                    assert ours[k] == theirs[k], (k, ours, theirs)
    assert events[-1] == {"serve": "exit", "reason": "stop", "served": 2}


def test_log_lines_stay_json_for_any_directory_name(tmp_path):
    d = tmp_path / 'odd "name"\nwith\tcontrol'
    d.mkdir()
    with open(tmp_path / "log.jsonl", "w") as log:
        ND.serve_dir(str(d), Mock(), timeout_sec=0, poll_ms=10, log_fd=log.fileno())
    events = [json.loads(l) for l in open(tmp_path / "log.jsonl")]
    assert events[0]["dir"] == str(d) and events[-1]["reason"] == "idleTimeout"
