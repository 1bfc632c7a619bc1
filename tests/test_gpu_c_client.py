"""The C ABI from a plain C program (tests/c_client/decode_client.c, linked
against libbsattn.so and the HIP runtime; no Python or torch in the
process): create -> append -> decode -> select, checked against the oracle
and against the Python binding on the same inputs."""
from __future__ import annotations

import os
import struct
import subprocess

import numpy as np
import pytest

from common import from_dev, log, make_workload, new_cache, oracle_decode, output_error, to_dev
import oracle as O

pytestmark = pytest.mark.gpu

CLIENT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_client", "decode_client")


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,T,K", [
    ("bf16", 32, 8, 64, 3000, 8),
    ("f16", 64, 4, 32, 2100, 16),
])
def test_c_client_decode(gpu, tmp_path, dtype, Hq, Hkv, Tb, T, K):
    import torch
    if not os.path.exists(CLIENT):
        pytest.fail(f"{CLIENT} is missing: build it with `make -C tests/c_client`")
    B = 2
    w = make_workload(9100 + Hq + T, B=B, Hq=Hq, Hkv=Hkv, T=T, Tb=Tb, dtype=dtype, top_k=K)
    prob = tmp_path / "problem.bin"
    res = tmp_path / "result.bin"
    with open(prob, "wb") as f:
        f.write(struct.pack("<9if", B, Hq, Hkv, T, Tb, 0 if dtype == "f16" else 1, K, w.ns, w.nr,
                            w.scale))
        f.write(np.stack(w.keys).astype(np.uint16).tobytes())
        f.write(np.stack(w.values).astype(np.uint16).tobytes())
        f.write(w.q.astype(np.uint16).tobytes())
    log(f"[c-client] {dtype} Hq={Hq} Hkv={Hkv} Tb={Tb} T={T}")
    r = subprocess.run([CLIENT, str(prob), str(res)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"client failed: {r.stdout}{r.stderr}"
    raw = res.read_bytes()
    nq = B * Hq * 128 * 2
    out = np.frombuffer(raw[:nq], np.uint16).reshape(B, Hq, 128)
    rest = np.frombuffer(raw[nq:], np.int32)
    idx_dec, idx_sel = rest[:rest.size // 2].reshape(B, Hkv, -1), rest[rest.size // 2:].reshape(B, Hkv, -1)
    # against the oracle
    idx_ref, out_ref = oracle_decode(w)
    assert np.array_equal(idx_dec, idx_ref) and np.array_equal(idx_sel, idx_ref)
    err = output_error(O.to_f32(out, dtype).astype(np.float64), out_ref, dtype)
    assert err <= 2e-3, f"output error {err:.3g}"
    # against the Python binding (same library, same inputs: identical bits)
    cache = new_cache(w)
    for b in range(B):
        cache.append(to_dev(w.keys[b][None], dtype, gpu), to_dev(w.values[b][None], dtype, gpu), seq_ids=[b])
    got = cache.decode(to_dev(w.q[:, :, None, :], dtype, gpu), w.scale)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(got).reshape(B, Hq, 128), out)
    log(f"[c-client] err={err:.3g}")
