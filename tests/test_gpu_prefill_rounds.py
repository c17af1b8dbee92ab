"""GPU parity of pelica_attn_prefill_round: a prompt's attention over keys
that arrive in rounds (VRAM rows and staged copies of rows past HBM), folded
into a running state in key order (attn_pre + attn_fold,
src/moe_kernels.rs:810-990, rounds at src/moe.rs:1609-1627), against the CPU
oracle's single-pass prompt attention on the same inputs.

Tolerance (north star): max |gpu - oracle| <= 2e-3, rel-L2 <= 1e-3, f16 out.
"""
import numpy as np
import pytest
import torch

from pelica_amd import attn
from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, gpu_run, oracle_run
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def run_rounds(inp, bounds, *, window=0, staged=True, out_each=False):
    cfg = inp.cfg
    T = cfg.q_tokens
    state = torch.empty(1, T, cfg.n_head, cfg.hd + 2, dtype=torch.float32, device="cuda")
    state.fill_(float("nan"))  # first=1 must not read it
    out = torch.empty_like(inp.q)
    for i, (a, b) in enumerate(zip(bounds[:-1], bounds[1:])):
        # a round's rows: a staging copy (rows past HBM) or a view of the cache
        k = inp.k[a:b].clone() if staged else inp.k[a:b]
        v = inp.v[a:b].clone() if staged else inp.v[a:b]
        last = i == len(bounds) - 2
        attn.prefill_round(inp.q, k, v, state, n_kv=cfg.n_kv, kv_len=inp.kv_len, key_begin=a, key_end=b,
                           first=i == 0, sinks=inp.sinks, window=window, out=out if (last or out_each) else None)
    torch.cuda.synchronize()
    return out, state


@pytest.mark.parametrize("hd,n_head,n_kv,T,L,bounds", [
    (64, 64, 8, 1000, 2500, [0, 700, 1900, 2500]),      # gpt-oss heads, prompt after a 1500-key prefix
    (128, 32, 4, 64, 20000, [0, 16384, 20000]),        # Qwen3 heads, 16K-key rounds (RK)
    (128, 16, 16, 300, 300, [0, 1, 65, 200, 300]),     # OLMoE heads, ragged round edges, prompt = cache
])
def test_rounds_match_single_pass(hd, n_head, n_kv, T, L, bounds):
    print(f"[case] rounds hd{hd} h{n_head}/{n_kv} T{T} L{L} {bounds}", flush=True)
    cfg = wl.AttnConfig("rounds", "prefill", n_head, n_kv, hd, L, q_tokens=T, sinks=hd == 64, seed=L + T)
    inp = wl.make_inputs(cfg, "cuda")
    out, state = run_rounds(inp, bounds)
    ref = oracle_run(inp)
    assert_close(as_f64(out), as_f64(ref), what="rounds vs oracle")
    one = gpu_run(inp)
    assert np.abs(as_f64(out) - as_f64(one)).max() < 2e-3
    s = state.cpu().numpy()
    assert np.isfinite(s).all() and (s[..., 1] >= 1.0 - 1e-6).all()  # every row saw its own key


def test_rounds_with_window_and_views():
    cfg = wl.AttnConfig("rwin", "prefill", 64, 8, 64, 3000, q_tokens=900, window=128, sinks=True, seed=77)
    inp = wl.make_inputs(cfg, "cuda")
    print("[case] rounds window 128", flush=True)
    out, _ = run_rounds(inp, [0, 1000, 2100, 2200, 3000], window=128, staged=False)
    assert_close(as_f64(out), as_f64(oracle_run(inp)), what="rounds + window")


def test_round_boundaries_do_not_change_the_result():
    cfg = wl.AttnConfig("rb", "prefill", 32, 4, 128, 5000, q_tokens=256, seed=78)
    inp = wl.make_inputs(cfg, "cuda")
    a, _ = run_rounds(inp, [0, 5000])
    b, _ = run_rounds(inp, [0, 1234, 2345, 4999, 5000])
    assert np.abs(as_f64(a) - as_f64(b)).max() <= 2 ** -10


def test_rows_before_any_key_output_zero():
    # tokens at positions < the first round's end see no key of a round that
    # starts after them: after a first round of keys [4000, 5000) only tokens
    # at positions >= 4000 have output
    cfg = wl.AttnConfig("rz", "prefill", 16, 16, 128, 5000, q_tokens=2000, seed=79)
    inp = wl.make_inputs(cfg, "cuda")
    state = torch.empty(1, 2000, 16, 130, dtype=torch.float32, device="cuda")
    out = torch.full_like(inp.q, 7.0)
    attn.prefill_round(inp.q, inp.k[4000:].clone(), inp.v[4000:].clone(), state, n_kv=16, kv_len=5000,
                       key_begin=4000, key_end=5000, first=True, out=out)
    torch.cuda.synchronize()
    o = as_f64(out)[0]
    first_pos = 5000 - 2000
    assert not np.any(o[: 4000 - first_pos])
    assert np.all(np.abs(o[4000 - first_pos:]).sum(-1) > 0)


def test_round_errors():
    cfg = wl.AttnConfig("re", "prefill", 16, 16, 128, 500, q_tokens=100, seed=80)
    inp = wl.make_inputs(cfg, "cuda")
    state = torch.empty(1, 100, 16, 130, dtype=torch.float32, device="cuda")
    with pytest.raises(attn.AttnError) as e:
        attn.prefill_round(inp.q, inp.k, inp.v, state, n_kv=16, kv_len=500, key_begin=400, key_end=600,
                           first=True)
    assert e.value.code == attn.EINVAL
