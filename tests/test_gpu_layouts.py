"""GPU parity of the layouts the reference's call sites pass, through the C ABI.

The reference's attention kernels read the queries in place in the fused
[q | k | v] activation rows (q stride arg 9 = qkv_rows) and write the output
into a wider activation row (out stride arg 10 = attw): ATTN_T and attn_s
(src/oss_batch.rs:172-176,267-270), attn_p (src/oss_prefill.rs:400-402),
dispatched at src/oss.rs:675-693,734-741 with f32 queries and f32 output.
attn_s and attn_p take keys below `res` from VRAM and the rest from the far
buffers.  Each test runs the step before (pelica_attn_qkv_rope_cache on the
fused rows) and the attention call on the same buffers, and compares with
the oracle chain (qkv oracle, then attention oracle) at the north-star
tolerance (max-abs 2e-3, rel 1e-3).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pelica_amd import attn
from tests.gpu_util import as_f64, to_np_f16
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu

N_HEAD, N_KV, HD = 64, 8, 64            # gpt-oss
QD, KD = N_HEAD * HD, N_KV * HD
QKV_ROWS = QD + 2 * KD                   # the fused row of one token
ATTW = QD + 64                           # a wider output row (the rest must stay intact)


def _chain_inputs(T, L, seed):
    """Fused activation rows of the pass's T tokens, a cache holding the L - T
    positions before them (random f16 rows), sinks and a rope table."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    act = torch.randn(T, QKV_ROWS, generator=g, device="cuda")
    kc = (torch.randn(L, KD, generator=g, device="cuda") * 0.5).half()
    vc = (torch.randn(L, KD, generator=g, device="cuda") * 0.5).half()
    sinks = torch.randn(N_HEAD, generator=g, device="cuda")
    table = torch.from_numpy(orc.rope_table(L, HD)).cuda()
    return act, kc, vc, sinks, table


def _step_before(act, kc, vc, table, T, L):
    """The qkv step on the fused rows (q rotated in place), and its oracle."""
    a0 = act.cpu().numpy()
    kc0, vc0 = to_np_f16(kc).copy(), to_np_f16(vc).copy()
    attn.qkv_rope_cache(act[:, :QD], act[:, QD:QD + KD], act[:, QD + KD:], kc, vc, n_kv=N_KV, kv_len=L, table=table,
                        token_stride=QKV_ROWS, n_seq=1, q_tokens=T, n_head=N_HEAD, hd=HD)
    qo, kco, vco = orc.qk_norm_rope_cache(a0[:, :QD].reshape(1, T, N_HEAD, HD),
                                          a0[:, QD:QD + KD].reshape(1, T, N_KV, HD),
                                          a0[:, QD + KD:].reshape(1, T, N_KV, HD), n_kv=N_KV, kv_len=L,
                                          table=table.cpu().numpy(), k_cache=kc0, v_cache=vc0)
    return qo, kco, vco


def _q_view(act, T):
    # the queries where the step before left them: token stride QKV_ROWS
    q = act[:, :QD].view(1, T, N_HEAD, HD)
    assert attn.token_stride(q) == (QKV_ROWS if T > 1 else 0)  # (one token's rows are contiguous)
    return q


def _out_rows(T, dtype):
    xo = torch.full((T, ATTW), 7.0, dtype=dtype, device="cuda")
    return xo, xo[:, :QD].view(1, T, N_HEAD, HD)


def _check_rest(xo):
    assert torch.all(xo[:, QD:] == 7.0), "values past the output heads were overwritten"


@pytest.mark.parametrize("T,L,window", [(4, 3000, 0), (4, 3000, 128), (1, 9000, 0)])
def test_qkv_step_then_decode_on_fused_rows(T, L, window):
    # drafts (T = 4) and a single token, full and window layers (ATTN_T / attn_s + ATTN_M)
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=100 + T + window)
    qo, kco, vco = _step_before(act, kc, vc, table, T, L)
    xo, out = _out_rows(T, torch.float32)
    print(f"[case] chain decode T{T} L{L} window{window}", flush=True)
    attn.decode(_q_view(act, T), kc, vc, n_kv=N_KV, kv_len=L, sinks=sinks, window=window, out=out)
    torch.cuda.synchronize()
    ref = orc.attention(qo, kco, vco, n_kv=N_KV, kv_len=L, sinks=sinks.cpu().numpy(), window=window)
    assert_close(as_f64(out), ref.astype(np.float64), what=f"decode T{T} window{window}")
    _check_rest(xo)


@pytest.mark.parametrize("T,L,window", [(300, 300, 0), (300, 300, 128), (300, 700, 0), (200, 900, 128)])
def test_qkv_step_then_f32_prefill_on_fused_rows(T, L, window):
    # attn_p's layout: f32 queries in the fused rows, f32 output rows of attw
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=200 + T + L + window)
    qo, kco, vco = _step_before(act, kc, vc, table, T, L)
    xo, out = _out_rows(T, torch.float32)
    print(f"[case] chain prefill f32 T{T} L{L} window{window}", flush=True)
    attn.prefill(_q_view(act, T), kc, vc, n_kv=N_KV, kv_len=L, sinks=sinks, window=window, out=out)
    torch.cuda.synchronize()
    ref = orc.attention(qo, kco, vco, n_kv=N_KV, kv_len=L, sinks=sinks.cpu().numpy(), window=window)
    assert_close(as_f64(out), ref.astype(np.float64), what=f"prefill f32 T{T} L{L} window{window}")
    _check_rest(xo)


def test_f16_prefill_with_token_strides():
    # the f16 form with strided queries and output equals the dense call bitwise
    T, L = 260, 260
    g = torch.Generator(device="cuda").manual_seed(5)
    rows = (torch.randn(1, T, QKV_ROWS, generator=g, device="cuda") * 0.5).half()
    kc = (torch.randn(L, KD, generator=g, device="cuda") * 0.5).half()
    vc = (torch.randn(L, KD, generator=g, device="cuda") * 0.5).half()
    sinks = torch.randn(N_HEAD, generator=g, device="cuda")
    q = rows[..., :QD].view(1, T, N_HEAD, HD)
    for window in (0, 128):
        dense = attn.prefill(q.contiguous(), kc, vc, n_kv=N_KV, sinks=sinks, window=window)
        xo = torch.zeros(1, T, ATTW, dtype=torch.float16, device="cuda")
        attn.prefill(q, kc, vc, n_kv=N_KV, sinks=sinks, window=window, out=xo[..., :QD].view(1, T, N_HEAD, HD))
        torch.cuda.synchronize()
        assert torch.equal(xo[..., :QD].reshape(dense.shape), dense), window
        assert torch.all(xo[..., QD:] == 0)


@pytest.mark.parametrize("res_from_end,window", [(700, 0), (2, 0), (4, 0), (300, 128), (3000, 0)])
def test_far_rows_as_two_ranges_and_a_merge(res_from_end, window):
    # attn_s over VRAM rows [0, res) and far rows [res, L): two key-range
    # partial passes and the batched merge with the sinks (ATTN_M)
    T, L = 4, 3000
    res = L - res_from_end
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=300 + res_from_end)
    qo, kco, vco = _step_before(act, kc, vc, table, T, L)
    q = _q_view(act, T)
    print(f"[case] far rows res {res} window {window}", flush=True)
    slots = []
    if res > 0:
        slots.append(attn.decode_partials_range(q, kc[:res].clone(), vc[:res].clone(), n_kv=N_KV, kv_len=L,
                                                key_begin=0, key_end=res, window=window))
    slots.append(attn.decode_partials_range(q, kc[res:].clone(), vc[res:].clone(), n_kv=N_KV, kv_len=L,
                                            key_begin=res, key_end=L, window=window))
    parts = torch.stack([s.reshape(T, N_HEAD, HD + 2) for s in slots]).contiguous()
    out = attn.partials_merge_batch(parts, sinks=sinks)
    torch.cuda.synchronize()
    ref = orc.attention(qo, kco, vco, n_kv=N_KV, kv_len=L, sinks=sinks.cpu().numpy(), window=window)
    assert_close(as_f64(out).reshape(ref.shape), ref.astype(np.float64), what=f"far rows res {res}")


def test_key_range_slots_of_rows_that_see_none_of_it():
    # window rows that see no key of the range get empty slots (M = -3e38, L = 0, O = 0)
    T, L, window = 4, 3000, 128
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=7)
    q = _q_view(act, T)
    parts = attn.decode_partials_range(q, kc[:1000].clone(), vc[:1000].clone(), n_kv=N_KV, kv_len=L, key_begin=0,
                                       key_end=1000, window=window)
    torch.cuda.synchronize()
    p = parts.cpu().numpy()
    assert np.all(p[..., 0] <= -1e38) and np.all(p[..., 1:] == 0)


def test_f32_prefill_rounds_over_staged_rows():
    # attn_p's far rows come from a staging copy: rounds [0, res) and [res, L)
    T, L, res = 300, 700, 450
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=9)
    qo, kco, vco = _step_before(act, kc, vc, table, T, L)
    q = _q_view(act, T)
    state = torch.empty(1, T, N_HEAD, HD + 2, device="cuda")
    xo, out = _out_rows(T, torch.float32)
    attn.prefill_round(q, kc[:res].clone(), vc[:res].clone(), state, n_kv=N_KV, kv_len=L, key_begin=0, key_end=res,
                       first=True, sinks=sinks)
    attn.prefill_round(q, kc[res:].clone(), vc[res:].clone(), state, n_kv=N_KV, kv_len=L, key_begin=res, key_end=L,
                       first=False, sinks=sinks, out=out)
    torch.cuda.synchronize()
    ref = orc.attention(qo, kco, vco, n_kv=N_KV, kv_len=L, sinks=sinks.cpu().numpy())
    assert_close(as_f64(out), ref.astype(np.float64), what="f32 prefill rounds")
    _check_rest(xo)


def test_decode_workspace_contents_do_not_matter():
    # a fresh workspace full of NaN patterns, then reused with the last call's contents
    T, L = 4, 20000
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=11)
    q = act[:, :QD].contiguous().view(1, T, N_HEAD, HD)
    desc = attn.make_desc(N_HEAD, N_KV, HD, q_tokens=T, kv_len=L)
    ws = torch.full((attn.workspace_bytes(desc),), 0xFF, dtype=torch.uint8, device="cuda")
    a = attn.decode(q, kc, vc, n_kv=N_KV, kv_len=L, sinks=sinks, workspace=ws)
    b = attn.decode(q, kc, vc, n_kv=N_KV, kv_len=L, sinks=sinks, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ref = orc.attention(q.cpu().numpy(), to_np_f16(kc), to_np_f16(vc), n_kv=N_KV, kv_len=L, sinks=sinks.cpu().numpy())
    assert_close(as_f64(a), ref.astype(np.float64), what="0xFF workspace")


def test_mla_with_token_strides():
    # MLA queries and output as token rows of wider buffers: bitwise the dense result
    T, H, L = 3, 16, 2000
    g = torch.Generator(device="cuda").manual_seed(13)
    qrows = torch.randn(1, T, H * 512 + 64, generator=g, device="cuda")
    lat = (torch.randn(L, 512, generator=g, device="cuda") * 0.5).half()
    q = qrows[..., :H * 512].view(1, T, H, 512)
    dense = attn.mla(q.contiguous(), lat, kv_len=L, scale=0.1)
    xo = torch.zeros(1, T, H * 512 + 128, device="cuda")
    attn.mla(q, lat, kv_len=L, scale=0.1, out=xo[..., :H * 512].view(1, T, H, 512))
    torch.cuda.synchronize()
    assert torch.equal(xo[..., :H * 512].reshape(dense.shape), dense)
    assert torch.all(xo[..., H * 512:] == 0)


def _widen(t, extra):
    """t [n_seq, T, H, hd] copied into token rows of H*hd + extra values; the view."""
    n_seq, T, H, hd = t.shape
    rows = torch.full((n_seq, T, H * hd + extra), 5.0, dtype=t.dtype, device=t.device)
    rows[..., :H * hd] = t.reshape(n_seq, T, H * hd)
    return rows, rows[..., :H * hd].view(n_seq, T, H, hd)


@pytest.mark.parametrize("hd,n_head,n_kv,T,n_seq,kv_len", [(128, 32, 4, 4, 12, 6000), (64, 64, 8, 1, 9, 5000)])
def test_strided_ragged_stream_k(hd, n_head, n_kv, T, n_seq, kv_len):
    # ragged batches (stream-K) reading strided queries and writing strided rows
    from pelica_amd import workloads as wl
    from tests.gpu_util import oracle_run

    cfg = wl.AttnConfig("sk-strided", "decode", n_head, n_kv, hd, kv_len, q_tokens=T, n_seq=n_seq,
                        ragged=(T, kv_len), sinks=hd == 64, seed=31 + n_seq)
    inp = wl.make_inputs(cfg, "cuda")
    kw = dict(n_kv=n_kv, kv_len=inp.kv_len, sinks=inp.sinks, seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    dense = attn.decode(inp.q, inp.k, inp.v, **kw)
    _, q = _widen(inp.q, 96)
    xo, out = _widen(torch.zeros_like(inp.q), 32)
    print(f"[case] strided stream-K hd{hd} T{T} n_seq{n_seq}", flush=True)
    attn.decode(q, inp.k, inp.v, out=out, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, dense)
    assert torch.all(xo[..., n_head * hd:] == 5.0)
    assert_close(as_f64(out), as_f64(oracle_run(inp)), what="strided stream-K")


@pytest.mark.parametrize("hd,n_head,n_kv,T,L,window,ring,n_seq", [
    (128, 32, 4, 150, 150, 0, 0, 1),       # head dim 128
    (128, 32, 4, 96, 400, 64, 0, 1),       # window, prefix
    (64, 64, 8, 200, 900, 128, 384, 1),    # ring cache of a window layer
    (64, 16, 4, 70, 300, 0, 0, 3),         # ragged sequences
])
def test_f32_prefill_shapes(hd, n_head, n_kv, T, L, window, ring, n_seq):
    # the f32 form against the f32 oracle, on the layouts of the f16 tests
    from pelica_amd import workloads as wl

    cfg = wl.AttnConfig("pf32", "decode", n_head, n_kv, hd, L, q_tokens=T, n_seq=n_seq, window=window,
                        ragged=(T, L) if n_seq > 1 else None, sinks=True, seed=41 + hd + T)
    inp = wl.make_inputs(cfg, "cuda")
    k, v = inp.k, inp.v
    kw = dict(n_kv=n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=window)
    if n_seq > 1:
        kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    if ring:
        kr = torch.zeros(ring, n_kv, hd, dtype=torch.float16, device="cuda")
        vr = torch.zeros_like(kr)
        idx = torch.arange(L - ring, L, device="cuda")
        kr[idx % ring] = inp.k[idx]
        vr[idx % ring] = inp.v[idx]
        k, v = kr, vr
        kw.update(ring_cap=ring)
    print(f"[case] f32 prefill hd{hd} T{T} L{L} window{window} ring{ring} n_seq{n_seq}", flush=True)
    got = attn.prefill(inp.q, k, v, **kw)
    torch.cuda.synchronize()
    ref = orc.attention(inp.q.cpu().numpy(), to_np_f16(inp.k), to_np_f16(inp.v), n_kv=n_kv, kv_len=inp.kv_len,
                        seq_kv_len=inp.seq_len.cpu().numpy(), seq_kv_offset=inp.seq_off.cpu().numpy(),
                        sinks=inp.sinks.cpu().numpy(), window=window)
    assert got.dtype == torch.float32
    assert_close(as_f64(got), ref.astype(np.float64), what="f32 prefill")


def test_far_rows_head_dim_128():
    # the key-range pass at Qwen3's shape (32 q heads, 4 kv heads, 4 drafts)
    from pelica_amd import workloads as wl

    cfg = wl.AttnConfig("far128", "decode", 32, 4, 128, 9000, q_tokens=4, seed=51)
    inp = wl.make_inputs(cfg, "cuda")
    res = 6137
    kw = dict(n_kv=4, kv_len=9000)
    a = attn.decode_partials_range(inp.q, inp.k[:res].clone(), inp.v[:res].clone(), key_begin=0, key_end=res, **kw)
    b = attn.decode_partials_range(inp.q, inp.k[res:].clone(), inp.v[res:].clone(), key_begin=res, key_end=9000, **kw)
    out = attn.partials_merge_batch(torch.stack([a.reshape(4, 32, 130), b.reshape(4, 32, 130)]).contiguous())
    torch.cuda.synchronize()
    ref = orc.attention(inp.q.cpu().numpy(), to_np_f16(inp.k), to_np_f16(inp.v), n_kv=4, kv_len=9000)
    assert_close(as_f64(out).reshape(ref.shape), ref.astype(np.float64), what="far rows hd128")


def test_strided_calls_in_graph_replays():
    # the call sites' layouts recorded into a HIP graph give the eager result
    # on every replay, with unrelated eager work between the replays
    T, L = 4, 5000
    act, kc, vc, sinks, table = _chain_inputs(T, L, seed=61)
    _step_before(act, kc, vc, table, T, L)
    q = _q_view(act, T)
    desc = attn.make_desc(N_HEAD, N_KV, HD, q_tokens=T, kv_len=L, q_token_stride=QKV_ROWS, out_token_stride=ATTW)
    ws = attn.new_workspace(desc)
    xo, out = _out_rows(T, torch.float32)
    attn.decode(q, kc, vc, n_kv=N_KV, kv_len=L, sinks=sinks, out=out, workspace=ws)
    eager_dec = out.clone()
    Tp = 160
    actp, kp, vp, sp, tp = _chain_inputs(Tp, Tp, seed=62)
    _step_before(actp, kp, vp, tp, Tp, Tp)
    qp = _q_view(actp, Tp)
    xp, outp = _out_rows(Tp, torch.float32)
    attn.prefill(qp, kp, vp, n_kv=N_KV, sinks=sp, window=128, out=outp)
    eager_pre = outp.clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attn.decode(q, kc, vc, n_kv=N_KV, kv_len=L, sinks=sinks, out=out, workspace=ws)
        attn.prefill(qp, kp, vp, n_kv=N_KV, sinks=sp, window=128, out=outp)
    for _ in range(3):
        out.zero_()
        outp.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_dec) and torch.equal(outp, eager_pre)
        _check_rest(xo)
        _check_rest(xp)
        _ = (act * 2).sum().item()  # unrelated eager work between replays
