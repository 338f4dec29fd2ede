"""Writes tests/golden/serve_log_reference.jsonl: the serve-protocol log lines of a reference server session
(results/dense-demo-s31/pod_2xbw_20260917/pod_pull/s37/serve_A11/logs/server.jsonl in the reference tree, written by
gpu_real_model.cu's --serve loop): its first two requests and the end of the session.  Run in the build container,
where the reference tree is present; the fixture is committed, the reference is not needed to test against it."""
import json
import os
import sys

SRC = os.path.join(sys.argv[1] if len(sys.argv) > 1 else "/root/reference",
                   "results/dense-demo-s31/pod_2xbw_20260917/pod_pull/s37/serve_A11/logs/server.jsonl")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "serve_log_reference.jsonl")

lines = []
for raw in open(SRC):
    raw = raw.strip()
    if raw.startswith('{"serve"'):
        lines.append(json.loads(raw))
head = []
for e in lines:
    if e["serve"] == "waiting" and e["req"] == 2:
        break
    head.append(e)
tail = lines[-2:]  # the last waiting line and the exit line
with open(OUT, "w") as f:
    for e in head + tail:
        f.write(json.dumps(e, separators=(",", ":")) + "\n")
print(f"{len(head) + len(tail)} lines -> {OUT}")
