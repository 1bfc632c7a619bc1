"""The configurations' generated inputs hash to the committed digests
(tests/golden/input_digests.json, written by make_input_digests.py beside
it): the first 256 tokens of every sequence for each configuration, and the
whole of the small one.  The GPU tests of each configuration check the full
digest of what they upload."""
from __future__ import annotations

import pytest

from common import CONFIGS, DIGEST_PREFIX, config_args, input_digests, make_workload, workload_digest


@pytest.mark.parametrize("name", CONFIGS)
def test_prefix_digest(name):
    want = input_digests()[name]
    args = config_args(name)
    assert want["args"] == args
    assert want["prefix_tokens"] == DIGEST_PREFIX
    w = make_workload(**args, prefix=DIGEST_PREFIX)
    assert workload_digest(w, DIGEST_PREFIX) == want["prefix_sha256"]


@pytest.mark.parametrize("name", ["C1_f16", "C1_bf16"])
def test_full_digest_small_config(name):
    w = make_workload(**config_args(name))
    assert workload_digest(w) == input_digests()[name]["sha256"]
