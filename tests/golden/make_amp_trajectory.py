"""Extract the AMP loss-scale trajectory that the reference ships as data.

Source: the training dashboard of the reference, index.html:374 (the `raw`
array, format `[step, loss*1000, ppl, scale, skip]`, index.html:369), logged
every 100 applied steps by Trainer::run (training.rs:444-452).  Only the
step, scale and cumulative-skip columns are kept; they pin the loss-scale
growth cadence (training.rs:316-326), the cap and the restart behaviour
(training.rs:120) that tests/test_oracle_amp.py replays.

Usage: python tests/golden/make_amp_trajectory.py [/root/reference]
"""
import json
import os
import re
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
line = open(os.path.join(ref, "index.html"), encoding="utf-8").read().splitlines()[373]
rows = json.loads(re.search(r"const raw = (\[.*\]);", line).group(1))
out = {
    "source": "reference index.html:374 (raw = [step, loss*1000, ppl, scale, skip])",
    "columns": ["step", "scale", "skips"],
    "rows": [[int(r[0]), float(r[3]), int(r[4])] for r in rows],
}
dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "amp_trajectory_index_html.json")
with open(dst, "w") as f:
    json.dump(out, f, separators=(",", ":"))
print(f"{len(rows)} rows -> {dst}")
