"""Host-side API of the Python mirror that needs no GPU: the newCache
parameters that stay on the reference's path."""
from __future__ import annotations

import pytest


def test_new_cache_rejects_rotating_window():
    """newCache with maxKVSize asks for the reference's RotatingKVCache
    (LanguageModel.swift:219-223), which the block-sparse cache does not
    replace: the call fails before any device work."""
    import bsattn
    with pytest.raises(ValueError, match="RotatingKVCache"):
        bsattn.newCache([8, 8], bsattn.GenerateParameters(maxKVSize=4096), num_q_heads=32,
                        max_seqs=1, max_tokens=1024)


def test_generate_parameters_defaults():
    """Defaults of GenerateParameters' cache fields (Evaluate.swift:64-73)."""
    import bsattn
    p = bsattn.GenerateParameters()
    assert (p.maxKVSize, p.kvBits, p.kvGroupSize, p.quantizedKVStart) == (None, None, 64, 0)
