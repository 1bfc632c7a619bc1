"""Writes input_digests.json: SHA-256 digests of the generated inputs of the
decode configurations C1-C5 (full, and of each sequence's first 256 tokens).
The GPU tests of those configurations and a CPU test assert them, so a drift
of the counter-based generator (libm's log/cos/sqrt in Box-Muller, rounding to
the storage dtype) between machines fails loudly.

    python tests/golden/make_input_digests.py      # ~1-2 min, ~5 GB of RAM
"""
from __future__ import annotations

import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))

from common import CONFIGS, DIGEST_PREFIX, config_args, make_workload, workload_digest  # noqa: E402


def main():
    out = {}
    for name in CONFIGS:
        t0 = time.time()
        args = config_args(name)
        w = make_workload(**args)
        out[name] = {"args": args, "prefix_tokens": DIGEST_PREFIX,
                     "sha256": workload_digest(w), "prefix_sha256": workload_digest(w, DIGEST_PREFIX)}
        del w
        print(f"{name}: {out[name]['sha256'][:16]} ({time.time() - t0:.1f}s)", flush=True)
    with open(os.path.join(HERE, "input_digests.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
