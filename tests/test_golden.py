"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle reproduces them bit for bit and sits within 2e-6 of their fp64
brute-force values; on a GPU the HIP path matches them within the
north-star tolerance."""
import glob
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests.refimpl import assert_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FILES = sorted(glob.glob(os.path.join(HERE, "*.npz")))


def load(path):
    z = np.load(path)  # plain arrays, no pickles
    n_seq, T, H, n_kv, hd, window, ring, prefill = (int(x) for x in z["meta"])
    return z, dict(n_kv=n_kv, window=window, ring_cap=ring), bool(prefill)


def test_fixtures_exist():
    assert len(FILES) >= 7


@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_fixture(path):
    z, kw, prefill = load(path)
    sinks = z["sinks"] if "sinks" in z.files else None
    out = orc.attention(z["q"], z["k"], z["v"], seq_kv_len=z["lens"], seq_kv_offset=z["offs"], sinks=sinks, **kw)
    assert np.array_equal(out.view(np.uint16 if prefill else np.uint32),
                          z["out"].view(np.uint16 if prefill else np.uint32))
    got = out.view(np.float16).astype(np.float64) if prefill else out.astype(np.float64)
    tol = 1e-3 if prefill else 2e-6
    assert_close(got, z["ref64"], atol=tol, rtol=tol, what=os.path.basename(path))


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p)[:-4])
def test_gpu_matches_fixture(path):
    import torch

    from pelica_amd import attn

    z, kw, prefill = load(path)
    dev = "cuda"
    q = torch.from_numpy(z["q"]).to(dev)
    if prefill:
        q = q.view(torch.float16)
    k = torch.from_numpy(z["k"]).to(dev).view(torch.float16)
    v = torch.from_numpy(z["v"]).to(dev).view(torch.float16)
    lens = torch.from_numpy(z["lens"]).to(dev)
    offs = torch.from_numpy(z["offs"]).to(dev)
    sinks = torch.from_numpy(z["sinks"]).to(dev) if "sinks" in z.files else None
    fn = attn.prefill if prefill else attn.decode
    out = fn(q, k, v, kv_len=int(z["lens"].max()), seq_kv_len=lens, seq_kv_offset=offs, sinks=sinks, **kw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().astype(np.float64)
    want = z["out"].view(np.float16).astype(np.float64) if prefill else z["out"].astype(np.float64)
    assert_close(got, want, what=os.path.basename(path))
