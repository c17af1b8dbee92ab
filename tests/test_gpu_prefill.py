"""GPU parity of pelica_attn_prefill against the CPU oracle (f16 in/out, f32
softmax and accumulation) on identical seeded inputs, through the C ABI.

Both sides round the output to f16, so besides the 2e-3 / 1e-3 contract the
residual is about one f16 ulp of the output.
"""
import numpy as np
import pytest
import torch

from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, gpu_run, oracle_run
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def test_c4_full_causal_all_rows():
    # every one of the 4096 prompt rows x 64 heads against the oracle
    inp = wl.make_inputs(wl.C4_FULL, "cuda")
    print("[case] c4 full", flush=True)
    got = as_f64(gpu_run(inp))
    ref = as_f64(oracle_run(inp))
    assert_close(got, ref, what="c4 full causal, all rows")


def test_c4_window_all_rows():
    inp = wl.make_inputs(wl.C4_SWA, "cuda")
    print("[case] c4 swa", flush=True)
    got = as_f64(gpu_run(inp))
    ref = as_f64(oracle_run(inp))
    assert_close(got, ref, what="c4 window 128")


@pytest.mark.parametrize("T", [1, 7, 33, 64, 100, 257])
@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 64, 8), (128, 32, 4), (64, 8, 8), (128, 16, 1)])
def test_small_prompts(T, hd, n_head, n_kv):
    cfg = wl.AttnConfig("p", "prefill", n_head, n_kv, hd, T, q_tokens=T, sinks=(T % 2 == 1), seed=T + hd)
    inp = wl.make_inputs(cfg, "cuda")
    print(f"[case] prefill T{T} hd{hd} h{n_head}/{n_kv}", flush=True)
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what=f"T{T} hd{hd}")


@pytest.mark.parametrize("window", [1, 17, 64, 128, 1000])
@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 64, 8), (128, 32, 4), (64, 16, 4)])
def test_windows(window, hd, n_head, n_kv):
    cfg = wl.AttnConfig("pw", "prefill", n_head, n_kv, hd, 700, q_tokens=700, window=window, sinks=True,
                        seed=window + hd)
    inp = wl.make_inputs(cfg, "cuda")
    print(f"[case] prefill window {window} hd{hd}", flush=True)
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what=f"window {window} hd{hd}")


def test_prompt_after_cached_prefix():
    # a second prompt chunk: 300 new tokens after 900 cached positions
    cfg = wl.AttnConfig("chunk", "prefill", 64, 8, 64, 1200, q_tokens=300, sinks=True, seed=71)
    inp = wl.make_inputs(cfg, "cuda")
    print("[case] prefill after prefix", flush=True)
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what="prefix")


def test_ragged_sequences():
    cfg = wl.AttnConfig("pr", "prefill", 32, 4, 128, 600, q_tokens=64, n_seq=3, ragged=(64, 600), seed=72)
    inp = wl.make_inputs(cfg, "cuda")
    print("[case] prefill ragged", flush=True)
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what="ragged")


@pytest.mark.parametrize("hd,n_head,n_kv,T", [(64, 64, 8, 512), (128, 32, 4, 512), (64, 64, 8, 4096)])
def test_ring_window_prefill(hd, n_head, n_kv, T):
    # (4096 tokens at head dim 64: two token blocks per workgroup over
    # resident tiles; 512: one)
    cap, L, W = 128 + T, T + 2488, 128
    cfg = wl.AttnConfig("pring", "prefill", n_head, n_kv, hd, L, q_tokens=T, window=W, sinks=True, seed=73 + hd)
    inp = wl.make_inputs(cfg, "cuda")
    kr = torch.zeros(cap, n_kv, hd, dtype=torch.float16, device="cuda")
    vr = torch.zeros_like(kr)
    idx = torch.arange(L - cap, L, device="cuda")
    kr[idx % cap] = inp.k[idx]
    vr[idx % cap] = inp.v[idx]
    print(f"[case] prefill ring hd{hd} T{T}", flush=True)
    got = gpu_run(inp, ring_cap=cap, k=kr, v=vr)
    assert_close(as_f64(got), as_f64(oracle_run(inp)), what=f"prefill ring hd{hd}")


def test_prefill_matches_decode_rows():
    # the prompt's last row equals a one-token decode at that position
    # (f32 queries rounded the same way), within the f16 output rounding
    cfg = wl.AttnConfig("pd", "prefill", 64, 8, 64, 500, q_tokens=500, sinks=True, seed=74)
    inp = wl.make_inputs(cfg, "cuda")
    from pelica_amd import attn

    pre = gpu_run(inp)
    dec = attn.decode(inp.q[:, -1:].float().contiguous(), inp.k, inp.v, n_kv=8, kv_len=500, sinks=inp.sinks)
    torch.cuda.synchronize()
    assert_close(as_f64(pre[:, -1:]), as_f64(dec), atol=2e-3, rtol=1e-3, what="prefill vs decode")


@pytest.mark.parametrize("logit", [-40.0, -120.0])
def test_all_logits_far_below_zero(logit):
    # every key has the same score, far below 0 (no sinks): the softmax is
    # uniform, the output the causal mean of V — the kernel must not lose
    # the keys to f16 underflow before it has a running max
    T, L, hd = 300, 700, 64
    cfg = wl.AttnConfig("neg", "prefill", 8, 8, hd, L, q_tokens=T, seed=31)
    inp = wl.make_inputs(cfg, "cuda")
    k0 = torch.randn(hd, device="cuda")
    k0 = k0 / k0.norm() * 4.0
    inp.k.copy_(k0.half().expand_as(inp.k))
    kf = inp.k[0, 0].float()
    qv = kf * (logit * np.sqrt(hd) / float(kf @ kf))
    inp.q.copy_(qv.half().expand_as(inp.q))
    print(f"[case] logit {logit}", flush=True)
    got = gpu_run(inp)
    ref = oracle_run(inp)
    assert_close(as_f64(got), as_f64(ref), what=f"logit {logit}")


# Sliding-window shapes the persistent ring kernel takes (head dim 64, 8
# heads per kv head, window <= 130, linear cache): prompts after a cached
# prefix, no sinks, prompts that end inside a 64-token block, several
# sequences, and blocks per workgroup from 1 to 4.
@pytest.mark.parametrize("T,L,window,sinks,n_seq", [
    (300, 1200, 128, False, 1),    # after a prefix, no sinks (exact path first)
    (65, 65, 128, True, 1),        # one full block and one token
    (4096, 4096, 100, True, 1),    # two blocks per workgroup
    (8192, 8192, 130, True, 1),    # four blocks per workgroup, widest ring span
    (200, 900, 33, True, 3),       # several sequences with ragged prefixes
    (1, 500, 128, True, 1),        # one token: seven waves without rows
    (63, 63, 1, False, 1),         # a window of one key, no sinks
])
def test_slide_window(T, L, window, sinks, n_seq):
    ragged = (T, L) if n_seq > 1 else None
    cfg = wl.AttnConfig("pslide", "prefill", 64, 8, 64, L, q_tokens=T, window=window, sinks=sinks, n_seq=n_seq,
                        ragged=ragged, seed=90 + window + T)
    inp = wl.make_inputs(cfg, "cuda")
    print(f"[case] slide window T{T} L{L} W{window} sinks{sinks} seqs{n_seq}", flush=True)
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what=f"slide T{T} W{window}")


def test_slide_window_logits_far_below_zero():
    # uniform scores far below 0, no sinks, under a window: each row's output
    # is the mean of V over its window
    T, L, hd, W = 300, 700, 64, 128
    cfg = wl.AttnConfig("negw", "prefill", 64, 8, hd, L, q_tokens=T, window=W, seed=32)
    inp = wl.make_inputs(cfg, "cuda")
    k0 = torch.randn(hd, device="cuda")
    k0 = k0 / k0.norm() * 4.0
    inp.k.copy_(k0.half().expand_as(inp.k))
    kf = inp.k[0, 0].float()
    qv = kf * (-120.0 * np.sqrt(hd) / float(kf @ kf))
    inp.q.copy_(qv.half().expand_as(inp.q))
    print("[case] slide window logit -120", flush=True)
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what="slide window logit -120")


def test_slide_window_ring_ragged_sequences():
    # two sequences, each with its own ring of `cap` rows (key j of sequence
    # s in row s*cap + j % cap), ragged lengths, window 128
    from oracle import oracle as orc
    from pelica_amd import attn
    from tests.gpu_util import to_np_f16

    T, W = 300, 128
    cfg = wl.AttnConfig("pringr", "prefill", 64, 8, 64, 1300, q_tokens=T, window=W, sinks=True, n_seq=2,
                        ragged=(700, 1300), seed=91)
    inp = wl.make_inputs(cfg, "cuda")
    cap = W + T
    lens = inp.seq_len.cpu().tolist()
    offs = inp.seq_off.cpu().tolist()
    kr = torch.zeros(2 * cap, 8, 64, dtype=torch.float16, device="cuda")
    vr = torch.zeros_like(kr)
    for s_i, (n, off) in enumerate(zip(lens, offs)):
        j = torch.arange(n - cap, n, device="cuda")
        kr[s_i * cap + j % cap] = inp.k[off + j]
        vr[s_i * cap + j % cap] = inp.v[off + j]
    ring_off = torch.tensor([0, cap], dtype=torch.int64, device="cuda")
    print("[case] slide window ring ragged", flush=True)
    got = attn.prefill(inp.q, kr, vr, n_kv=8, kv_len=inp.kv_len, sinks=inp.sinks, window=W, ring_cap=cap,
                       seq_kv_len=inp.seq_len, seq_kv_offset=ring_off)
    torch.cuda.synchronize()
    ref = orc.attention(inp.q.cpu().numpy().view(np.uint16), to_np_f16(kr), to_np_f16(vr), n_kv=8,
                        kv_len=inp.kv_len, seq_kv_len=inp.seq_len.cpu().numpy(),
                        seq_kv_offset=np.array([0, cap], dtype=np.int64), sinks=inp.sinks.cpu().numpy(), window=W,
                        ring_cap=cap)
    assert_close(as_f64(got), as_f64(ref), what="slide ring ragged")
