"""GPU parity of pelica_attn_decode (and the partials merge) against the CPU
oracle on identical seeded inputs, through the C ABI.

Tolerance (north star): max |gpu - oracle| <= 2e-3 and
||gpu - oracle||_2 / ||oracle||_2 <= 1e-3, fp32 output.
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pelica_amd import attn
from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, gpu_run, oracle_run, to_np_f16
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def check(inp, what, **kw):
    print(f"[case] {what}", flush=True)
    got = gpu_run(inp, **kw)
    ref = oracle_run(inp, **kw)
    return assert_close(as_f64(got), as_f64(ref), what=what)


@pytest.mark.parametrize("cfg", [wl.C1, wl.C2, wl.C3_FULL, wl.C3_SWA, wl.C5], ids=lambda c: c.name)
def test_baseline_configs_full_size(cfg):
    inp = wl.make_inputs(cfg, "cuda")
    max_abs, rel = check(inp, cfg.name)
    print(f"{cfg.name}: max_abs {max_abs:.2e} rel {rel:.2e}")


@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 64, 8), (128, 32, 4), (64, 16, 16), (128, 16, 16)])
@pytest.mark.parametrize("kv_len", [1, 63, 65, 257, 1000, 4099])
def test_lengths(hd, n_head, n_kv, kv_len):
    cfg = wl.AttnConfig("len", "decode", n_head, n_kv, hd, kv_len, sinks=hd == 64, seed=kv_len)
    check(wl.make_inputs(cfg, "cuda"), f"hd{hd} h{n_head}/{n_kv} len{kv_len}")


@pytest.mark.parametrize("T", [2, 3, 4, 8])
@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 64, 8), (128, 32, 4), (128, 16, 16)])
def test_draft_tokens(T, hd, n_head, n_kv):
    cfg = wl.AttnConfig("drafts", "decode", n_head, n_kv, hd, 777, q_tokens=T, sinks=True, seed=T)
    check(wl.make_inputs(cfg, "cuda"), f"T{T} hd{hd} h{n_head}/{n_kv}")


@pytest.mark.parametrize("window", [1, 5, 128, 2000])
@pytest.mark.parametrize("T", [1, 4])
@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 64, 8), (128, 32, 4), (128, 16, 16)])
def test_windows(window, T, hd, n_head, n_kv):
    cfg = wl.AttnConfig("win", "decode", n_head, n_kv, hd, 1500, q_tokens=T, window=window, sinks=True,
                        seed=window + hd)
    check(wl.make_inputs(cfg, "cuda"), f"window {window} T{T} hd{hd} h{n_head}/{n_kv}")


def test_ragged_batch_with_minimum_lengths():
    cfg = wl.AttnConfig("ragged", "decode", 32, 4, 128, 3000, q_tokens=4, n_seq=6, ragged=(4, 3000), seed=9)
    inp = wl.make_inputs(cfg, "cuda")
    lens = inp.seq_len.clone()
    lens[0] = 4          # only the drafts themselves
    lens[1] = 5
    inp.seq_len.copy_(lens)
    check(inp, "ragged minimum lengths")


@pytest.mark.parametrize("hd,n_head,n_kv,T,n_seq,kv_len", [
    (64, 64, 8, 1, 9, 5000),     # gpt-oss batch, one row tile
    (64, 64, 8, 4, 5, 3000),     # two row tiles
    (128, 32, 4, 2, 150, 700),   # more sequences than one wave scans at once
    (128, 16, 16, 1, 40, 2500),  # MHA
])
def test_ragged_stream_k(hd, n_head, n_kv, T, n_seq, kv_len):
    # ragged batches without window or ring share their blocks over a fixed
    # grid: pieces of a sequence end on arbitrary block boundaries
    cfg = wl.AttnConfig("sk", "decode", n_head, n_kv, hd, kv_len, q_tokens=T, n_seq=n_seq, ragged=(T, kv_len),
                        sinks=hd == 64, seed=n_seq)
    check(wl.make_inputs(cfg, "cuda"), f"stream-K hd{hd} T{T} n_seq{n_seq}")


@pytest.mark.parametrize("window,T", [(128, 1), (300, 4)])
def test_ragged_batch_with_window(window, T):
    # ragged batches of a window layer stay on the split grid (stream-K
    # takes no window); some sequences are shorter than the window
    cfg = wl.AttnConfig("ragged-win", "decode", 64, 8, 64, 4000, q_tokens=T, n_seq=7, ragged=(T, 4000), window=window,
                        sinks=True, seed=window + T)
    check(wl.make_inputs(cfg, "cuda"), f"ragged window {window} T{T}")


def test_stream_k_matches_grid_splits(monkeypatch):
    inp = wl.make_inputs(wl.C5.scaled(n_seq=12), "cuda")
    outs = []
    try:
        for sk in ("0", "1"):
            monkeypatch.setenv("PELICA_ATTN_STREAMK", sk)
            attn.reload_tuning()
            check(inp, f"C5 x12, stream-K {sk}")
            outs.append(as_f64(gpu_run(inp)))
    finally:
        monkeypatch.delenv("PELICA_ATTN_STREAMK")
        attn.reload_tuning()
    assert np.abs(outs[0] - outs[1]).max() < 1e-5


def test_batch_without_offsets():
    cfg = wl.AttnConfig("batch", "decode", 16, 4, 64, 700, n_seq=3, seed=21)
    check(wl.make_inputs(cfg, "cuda"), "n_seq 3, default offsets")


@pytest.mark.parametrize("hd,n_head,n_kv,T", [(64, 64, 8, 3), (128, 32, 4, 1), (128, 32, 4, 4), (128, 16, 16, 2)])
def test_ring_buffer_window_layer(hd, n_head, n_kv, T):
    # the window layer's ring (src/oss.rs:570-572): position j in row j % cap
    cap, L, W = 160, 5000, 128
    cfg = wl.AttnConfig("ring", "decode", n_head, n_kv, hd, L, q_tokens=T, window=W, sinks=True, seed=33 + hd + T)
    inp = wl.make_inputs(cfg, "cuda")
    kr = torch.zeros(cap, n_kv, hd, dtype=torch.float16, device="cuda")
    vr = torch.zeros_like(kr)
    idx = torch.arange(L - cap, L, device="cuda")
    kr[idx % cap] = inp.k[idx]
    vr[idx % cap] = inp.v[idx]
    print(f"[case] ring hd{hd} h{n_head}/{n_kv} T{T}", flush=True)
    got = gpu_run(inp, ring_cap=cap, k=kr, v=vr)
    ref = oracle_run(inp)  # linear cache, same keys
    assert_close(as_f64(got), as_f64(ref), what=f"ring hd{hd} T{T}")


@pytest.mark.parametrize("hd,n_head,n_kv,T,n_seq,window", [(64, 64, 8, 1, 5, 0), (128, 32, 4, 4, 6, 0),
                                                            (64, 64, 8, 2, 4, 500), (128, 16, 16, 1, 3, 2000)])
def test_device_lengths_above_kv_len_are_clipped(hd, n_head, n_kv, T, n_seq, window):
    # seq_kv_len entries above the kv_len bound (e.g. a graph replayed after
    # the lengths grew) are clipped to kv_len: the result is that of kv_len
    # keys, no workspace slot or cache row past the bound is touched
    # every sequence owns L cache rows, so the clipped lengths stay inside them
    L = 3000
    cfg = wl.AttnConfig("clip", "decode", n_head, n_kv, hd, L, q_tokens=T, n_seq=n_seq, window=window, sinks=True,
                        seed=91 + hd)
    inp = wl.make_inputs(cfg, "cuda")
    lens = torch.tensor([L + 5000] + [700 + 300 * i for i in range(n_seq - 2)] + [L + 64], dtype=torch.int32,
                        device="cuda")
    print(f"[case] clipped lengths hd{hd} T{T} window {window}", flush=True)
    got = attn.decode(inp.q, inp.k, inp.v, n_kv=n_kv, kv_len=L, sinks=inp.sinks, window=window, seq_kv_len=lens,
                      seq_kv_offset=inp.seq_off)
    torch.cuda.synchronize()
    inp.seq_len.copy_(lens.clamp(max=L))
    ref = oracle_run(inp)
    assert_close(as_f64(got), as_f64(ref), what="clipped lengths")


def test_padded_row_stride():
    cfg = wl.AttnConfig("stride", "decode", 32, 4, 128, 900, sinks=True, seed=44)
    inp = wl.make_inputs(cfg, "cuda")
    stride = 4 * 128 + 64
    kp = torch.zeros(900, stride, dtype=torch.float16, device="cuda")
    vp = torch.zeros_like(kp)
    kp[:, :512] = inp.k.reshape(900, 512)
    vp[:, :512] = inp.v.reshape(900, 512)
    got = gpu_run(inp, k=kp, v=vp, kv_row_stride=stride)
    ref = oracle_run(inp)
    assert_close(as_f64(got), as_f64(ref), what="row stride")


def test_split_count_invariance(monkeypatch):
    # the result does not depend on how the keys are split (fixed-order merge)
    inp = wl.make_inputs(wl.C3_FULL.scaled(kv_len=9000), "cuda")
    outs = []
    try:
        for sb in ("1", "3", "16", "200"):
            monkeypatch.setenv("PELICA_ATTN_SPLIT_BLOCKS", sb)
            attn.reload_tuning()
            outs.append(as_f64(gpu_run(inp)))
    finally:
        monkeypatch.delenv("PELICA_ATTN_SPLIT_BLOCKS")
        attn.reload_tuning()
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 2e-6


def test_split_only_leaves_output_alone():
    # the measurement flag runs the split kernel only: out keeps its contents
    inp = wl.make_inputs(wl.C3_FULL.scaled(kv_len=8192), "cuda")
    out = torch.full_like(inp.q, float("nan"))
    kw = dict(n_kv=8, kv_len=8192, sinks=inp.sinks, out=out)
    attn.decode(inp.q, inp.k, inp.v, split_only=True, **kw)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    attn.decode(inp.q, inp.k, inp.v, **kw)
    assert_close(as_f64(out), as_f64(oracle_run(inp)), what="after a split-only call")


def test_output_is_deterministic():
    inp = wl.make_inputs(wl.C5, "cuda")
    a = gpu_run(inp)
    b = gpu_run(inp)
    assert torch.equal(a, b)


def test_partials_merge_joins_cpu_tier():
    # the CPU tier's chunk partials (cpu_attn format) merged on the GPU with
    # the sinks give the full attention (src/moe.rs:1713-1729)
    cfg = wl.AttnConfig("merge", "decode", 32, 4, 128, 2000, sinks=True, seed=55)
    inp = wl.make_inputs(cfg, "cuda")
    q = inp.q.cpu().numpy()
    parts = orc.partials(q, to_np_f16(inp.k), to_np_f16(inp.v), n_kv=4, kv_len=2000)
    # pad with empty slots the way cpu_layer does (max -3e38)
    empty = np.zeros((3, 32, 130), np.float32)
    empty[:, :, 0] = -3e38
    parts = np.concatenate([parts[:2], empty, parts[2:]])
    out = attn.partials_merge(torch.from_numpy(parts).cuda(), n_head=32, hd=128, sinks=inp.sinks)
    torch.cuda.synchronize()
    ref = oracle_run(inp)
    assert_close(as_f64(out), as_f64(ref)[0, 0], what="partials merge")


def test_errors_surface_as_exceptions():
    inp = wl.make_inputs(wl.C3_FULL.scaled(kv_len=128), "cuda")
    with pytest.raises(attn.AttnError) as e:
        attn.decode(inp.q, inp.k, inp.v, n_kv=8, kv_len=128, window=-3)
    assert e.value.code == attn.EINVAL


def test_workspace_reuse():
    # one workspace (uninitialised contents) serves repeated calls
    from pelica_amd.attn import make_desc, new_workspace

    inp = wl.make_inputs(wl.C3_FULL.scaled(kv_len=20000), "cuda")
    desc = make_desc(64, 8, 64, kv_len=20000)
    ws = new_workspace(desc)
    outs = [attn.decode(inp.q, inp.k, inp.v, n_kv=8, kv_len=20000, sinks=inp.sinks, workspace=ws)
            for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    ref = oracle_run(inp)
    assert_close(as_f64(outs[2]), as_f64(ref), what="reused workspace")


def test_graph_replays_match_eager():
    # a decode recorded into a HIP graph gives the eager result on every replay
    from pelica_amd.attn import make_desc, new_workspace

    inp = wl.make_inputs(wl.C2, "cuda")
    desc = make_desc(32, 4, 128, kv_len=inp.kv_len)
    ws = new_workspace(desc)
    eager = attn.decode(inp.q, inp.k, inp.v, n_kv=4, kv_len=inp.kv_len, workspace=ws).clone()
    out = torch.empty_like(eager)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attn.decode(inp.q, inp.k, inp.v, n_kv=4, kv_len=inp.kv_len, workspace=ws, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = (inp.q * 2).sum().item()  # unrelated eager work between replays


def test_stream_k_graph_follows_device_lengths():
    # stream-K computes its layout on the device from seq_kv_len: a graph
    # recorded once stays right when the lengths change between replays
    cfg = wl.C5.scaled(n_seq=8, kv_len=6000, ragged=(4, 6000))
    inp = wl.make_inputs(cfg, "cuda")
    kw = dict(n_kv=4, kv_len=inp.kv_len, seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    desc = attn.make_desc(32, 4, 128, n_seq=8, q_tokens=4, kv_len=inp.kv_len, seq_kv_len=inp.seq_len,
                          seq_kv_offset=inp.seq_off)
    ws = attn.new_workspace(desc)
    out = torch.empty_like(inp.q)
    attn.decode(inp.q, inp.k, inp.v, workspace=ws, out=out, **kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attn.decode(inp.q, inp.k, inp.v, workspace=ws, out=out, **kw)
    gen = torch.Generator().manual_seed(3)
    orig = inp.seq_len.cpu()
    for _ in range(3):
        # new lengths within each sequence's rows (the offsets stay)
        lens = (4 + (torch.rand(8, generator=gen) * (orig - 3).float()).to(torch.int32)).clamp(max=orig)
        inp.seq_len.copy_(lens)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = attn.decode(inp.q, inp.k, inp.v, workspace=attn.new_workspace(desc), **kw)
        torch.cuda.synchronize()
        assert torch.equal(got, eager)
    assert_close(as_f64(got), as_f64(oracle_run(inp)), what="stream-K graph, last lengths")


def test_reused_workspace_with_changing_inputs():
    # consecutive calls on one workspace with different queries and caches:
    # the combine must read this call's partials, never an earlier call's
    from pelica_amd.attn import make_desc, new_workspace

    desc = make_desc(64, 8, 64, kv_len=30000)
    ws = new_workspace(desc)
    ws.fill_(0xFF)  # garbage contents are fine
    for seed in (101, 102, 103):
        inp = wl.make_inputs(wl.C3_FULL.scaled(kv_len=30000, seed=seed), "cuda")
        got = attn.decode(inp.q, inp.k, inp.v, n_kv=8, kv_len=30000, sinks=inp.sinks, workspace=ws)
        torch.cuda.synchronize()
        assert_close(as_f64(got), as_f64(oracle_run(inp)), what=f"seed {seed}")


def test_workspace_init_zero_fills():
    ws = torch.full((4096,), 0xAB, dtype=torch.uint8, device="cuda")
    assert attn.load_library().pelica_attn_workspace_init(ws.data_ptr(), ws.numel(), None) == 0
    torch.cuda.synchronize()
    assert int(ws.sum()) == 0


def test_per_kernel_timing():
    inp = wl.make_inputs(wl.C3_FULL, "cuda")
    attn.prof_enable(True)
    for _ in range(3):
        attn.decode(inp.q, inp.k, inp.v, n_kv=8, kv_len=inp.kv_len, sinks=inp.sinks)
    torch.cuda.synchronize()
    recs = attn.prof_read()
    attn.prof_enable(False)
    names = [n for n, _ in recs]
    assert names.count("decode_split") == 3 and names.count("decode_combine") == 3
    assert all(ms > 0 for _, ms in recs)
    assert attn.prof_read() == []
