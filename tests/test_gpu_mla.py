"""GPU parity of pelica_attn_mla (latent attention, K = V = the latent rows,
one kv head of 512 dims: mla, src/gpu.rs:262-307) against the CPU oracle's
attention with the latent as both cache tensors, on the same seeded inputs.

Tolerance (north star): max |gpu - oracle| <= 2e-3, rel-L2 <= 1e-3, f32 out.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pelica_amd import attn
from tests.gpu_util import as_f64, to_np_f16
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def _inputs(n_seq, T, n_head, L, seed, rows=None):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(n_seq, T, n_head, 512, generator=g, device="cuda") * 0.25
    lat = (torch.randn(rows or n_seq * L, 512, generator=g, device="cuda") * 0.5).half()
    return q, lat


def _oracle(q, lat, L, scale, **kw):
    qn = q.cpu().numpy()
    ln = to_np_f16(lat)
    return orc.attention(qn, ln, ln, n_kv=1, kv_len=L, scale=scale, **kw)


@pytest.mark.parametrize("n_head,T,L", [(32, 1, 4096), (16, 1, 37), (64, 1, 20000), (20, 8, 3000), (8, 64, 700),
                                         (32, 4, 33000)])
def test_mla_matches_oracle(n_head, T, L):
    scale = 1.0 / np.sqrt(192)  # the engine's 1/sqrt(qk_nope)
    print(f"[case] mla h{n_head} T{T} L{L}", flush=True)
    q, lat = _inputs(1, T, n_head, L, seed=L + T)
    out = attn.mla(q, lat, kv_len=L, scale=scale)
    torch.cuda.synchronize()
    assert_close(as_f64(out), _oracle(q, lat, L, scale).astype(np.float64), what=f"mla h{n_head} T{T} L{L}")


def test_mla_ragged_batch_and_row_stride():
    n_seq, T, n_head = 3, 2, 16
    lens = [900, 2, 2500]
    offs = [0, 1000, 1010]
    q, _ = _inputs(n_seq, T, n_head, 0, seed=5, rows=1)
    g = torch.Generator(device="cuda").manual_seed(6)
    stride = 512 + 64
    lat = torch.zeros(offs[-1] + lens[-1], stride, dtype=torch.float16, device="cuda")
    lat[:, :512] = (torch.randn(lat.shape[0], 512, generator=g, device="cuda") * 0.5).half()
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    so = torch.tensor(offs, dtype=torch.int64, device="cuda")
    print("[case] mla ragged", flush=True)
    out = attn.mla(q, lat, kv_len=max(lens), seq_kv_len=sl, seq_kv_offset=so, kv_row_stride=stride)
    torch.cuda.synchronize()
    ln = np.ascontiguousarray(to_np_f16(lat)[:, :512])
    ref = orc.attention(q.cpu().numpy(), ln, ln, n_kv=1, seq_kv_len=np.array(lens, np.int32),
                        seq_kv_offset=np.array(offs, np.int64))
    assert_close(as_f64(out), ref.astype(np.float64), what="mla ragged")


def test_mla_equal_rows_give_the_row():
    # K = V: with every latent row the same, the output is that row
    q, lat = _inputs(1, 1, 32, 5000, seed=9)
    lat.copy_(lat[0].expand_as(lat))
    out = attn.mla(q, lat, kv_len=5000)
    torch.cuda.synchronize()
    want = lat[0].float().cpu().numpy().astype(np.float64)
    assert np.abs(as_f64(out)[0, 0] - want[None, :]).max() < 1e-5


def test_mla_rejects_other_layouts():
    q, lat = _inputs(1, 1, 8, 100, seed=10)
    desc = attn.make_desc(8, 2, 512, kv_len=100)
    lib = attn.load_library()
    import ctypes
    assert lib.pelica_attn_mla(ctypes.byref(desc), q.data_ptr(), lat.data_ptr(), q.data_ptr(), None, 0,
                               None) == attn.EUNSUPPORTED
