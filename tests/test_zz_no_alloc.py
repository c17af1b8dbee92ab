"""pelica_attn_decode_noalloc (the decode entry point that allocates nothing:
split partials in the library's per-device static scratch) against
pelica_attn_decode with a caller workspace, through the C ABI: two calls in
a row on one GPU, the second with a smaller input, each bit-identical to the
workspace path (same plan, same kernels) and within the north-star
tolerance of the oracle."""
import pytest
import torch

from pelica_amd import attn
from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, oracle_run
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def _both(inp):
    cfg = inp.cfg
    kw = dict(n_kv=cfg.n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=cfg.window)
    if inp.ragged:
        kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    ref = attn.decode(inp.q, inp.k, inp.v, **kw)
    got = torch.full_like(inp.q, float("nan"))
    attn.decode_noalloc(inp.q, inp.k, inp.v, out=got, **kw)
    torch.cuda.synchronize()
    return got, ref


@pytest.mark.parametrize("first,second", [
    (wl.C3_FULL, wl.C3_FULL.scaled(kv_len=5000, seed=31)),   # split grid, then fewer splits
    (wl.C5, wl.C5.scaled(n_seq=5, kv_len=3000, ragged=(4, 3000), seed=32)),  # stream-K, then a smaller batch
    (wl.C2, wl.C1),                                          # Qwen3 GQA, then OLMoE MHA
], ids=["c3", "c5", "c2-c1"])
def test_noalloc_matches_workspace_decode(first, second):
    for i, cfg in enumerate((first, second)):
        print(f"[case] noalloc call {i}: {cfg.name} kv_len {cfg.kv_len} n_seq {cfg.n_seq}", flush=True)
        inp = wl.make_inputs(cfg, "cuda")
        got, ref = _both(inp)
        assert torch.equal(got, ref), f"call {i} ({cfg.name}) differs from pelica_attn_decode"
        if i == 1:
            assert_close(as_f64(got), as_f64(oracle_run(inp)), what=f"noalloc {cfg.name}")
