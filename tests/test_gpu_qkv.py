"""GPU parity of pelica_attn_qkv_rope_cache (the step before attention:
qk_dec, src/moe_kernels.rs:304-378; ROPE_KV_T, src/oss_batch.rs:113-170)
against the CPU oracle on the same seeded inputs.

Bars: v rows bit-exact (the same f32 rounded to nearest-even f16); q within
1e-5 abs (rotation/norm in f32, contraction may differ by an ulp); k rows
within one f16 ulp of the oracle's; cache rows not addressed stay intact.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pelica_amd import attn
from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, to_np_f16
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu

SENTINEL = 0x7BCD  # an f16 bit pattern no input produces


def _case(n_seq, T, n_head, n_kv, hd, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    mk = lambda h: torch.randn(n_seq, T, h, hd, generator=g, device="cuda")
    return mk(n_head), mk(n_kv), mk(n_kv)


def _run_both(q, k, v, *, n_kv, kv_len, rows, table=None, rot=0, neox=True, table_split=0, q_norm=None,
              k_norm=None, seq_kv_len=None, seq_kv_offset=None, ring_cap=0, kv_row_stride=0):
    hd = q.shape[-1]
    stride = kv_row_stride or n_kv * hd
    kc = torch.full((rows, stride), 0, dtype=torch.int16, device="cuda")
    kc.fill_(SENTINEL)
    kc = kc.view(torch.float16)
    vc = kc.clone()
    qg = q.clone()
    attn.qkv_rope_cache(qg, k, v, kc, vc, n_kv=n_kv, kv_len=kv_len, table=table, rot=rot, neox=neox,
                        table_split=table_split, q_norm=q_norm, k_norm=k_norm, seq_kv_len=seq_kv_len,
                        seq_kv_offset=seq_kv_offset, ring_cap=ring_cap, kv_row_stride=kv_row_stride)
    torch.cuda.synchronize()
    kc0 = np.full((rows, stride), SENTINEL, np.uint16)
    vc0 = kc0.copy()
    qo, kco, vco = orc.qk_norm_rope_cache(
        q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), n_kv=n_kv, kv_len=kv_len,
        seq_kv_len=None if seq_kv_len is None else seq_kv_len.cpu().numpy(),
        seq_kv_offset=None if seq_kv_offset is None else seq_kv_offset.cpu().numpy(), ring_cap=ring_cap,
        kv_row_stride=kv_row_stride, k_cache=kc0, v_cache=vc0,
        rot=rot or hd, neox=neox, table=None if table is None else table.cpu().numpy(), table_split=table_split,
        q_norm=None if q_norm is None else q_norm.cpu().numpy(),
        k_norm=None if k_norm is None else k_norm.cpu().numpy())
    return (qg, kc, vc), (qo, kco, vco)


def _check(gpu, ref, what):
    qg, kc, vc = gpu
    qo, kco, vco = ref
    assert np.abs(qg.cpu().numpy().astype(np.float64) - qo).max() < 1e-5, what
    kg, vg = to_np_f16(kc), to_np_f16(vc)
    assert np.array_equal(vg, vco), what  # v: bit-exact, sentinel rows included
    untouched = kco == SENTINEL
    assert np.array_equal(kg[untouched], kco[untouched]), what
    a = kg[~untouched].view(np.float16).astype(np.float64)
    b = kco[~untouched].view(np.float16).astype(np.float64)
    ulp = np.maximum(np.abs(b), 6.1e-5) * 2.0 ** -10
    assert np.all(np.abs(a - b) <= ulp * 1.001), what


def test_gptoss_drafts_linear_and_ring():
    # gpt-oss: 64q/8kv hd64, NeoX pairs, direct table, 4 draft tokens
    q, k, v = _case(1, 4, 64, 8, 64, seed=1)
    table = torch.from_numpy(orc.rope_table(5000, 64)).cuda()
    print("[case] gpt-oss linear", flush=True)
    _check(*_run_both(q, k, v, n_kv=8, kv_len=5000, rows=5000, table=table), "linear")
    print("[case] gpt-oss ring", flush=True)
    _check(*_run_both(q, k, v, n_kv=8, kv_len=5000, rows=160, table=table, ring_cap=160), "ring")


def test_qwen3_norms_two_level_table_ragged_batch():
    # Qwen3: 32q/4kv hd128, per-head q/k RMS norms, the MoE engine's table
    q, k, v = _case(3, 1, 32, 4, 128, seed=2)
    split, n_hi = orc.rope_table(70000, 128, split=True)
    table = torch.from_numpy(split).cuda()
    g = torch.Generator(device="cuda").manual_seed(3)
    qn = torch.rand(128, generator=g, device="cuda") + 0.5
    kn = torch.rand(128, generator=g, device="cuda") + 0.5
    lens = torch.tensor([70000, 5, 31337], dtype=torch.int32, device="cuda")
    offs = torch.tensor([0, 70000, 70010], dtype=torch.int64, device="cuda")
    print("[case] qwen3 ragged", flush=True)
    _check(*_run_both(q, k, v, n_kv=4, kv_len=70000, rows=70010 + 31337, table=table, table_split=n_hi,
                      q_norm=qn, k_norm=kn, seq_kv_len=lens, seq_kv_offset=offs), "qwen3")


@pytest.mark.parametrize("hd,rot,neox", [(64, 32, False), (128, 64, True), (256, 256, False)])
def test_partial_rotary_interleaved_and_wide_heads(hd, rot, neox):
    q, k, v = _case(2, 2, 8, 2, hd, seed=hd + rot)
    table = torch.from_numpy(orc.rope_table(600, rot)).cuda()
    print(f"[case] hd{hd} rot{rot} neox{neox}", flush=True)
    _check(*_run_both(q, k, v, n_kv=2, kv_len=600, rows=1200, table=table, rot=rot, neox=neox,
                      kv_row_stride=2 * hd + 32), f"hd{hd}")


def test_no_rope_norm_only():
    q, k, v = _case(1, 3, 16, 16, 128, seed=5)
    w = torch.linspace(0.5, 1.5, 128, device="cuda")
    _check(*_run_both(q, k, v, n_kv=16, kv_len=50, rows=50, q_norm=w, k_norm=w), "norm only")


@pytest.mark.parametrize("pad", [0, 1])
def test_fused_qkv_rows_with_token_stride(pad):
    # the engine's activation rows [q heads | k heads | v heads] per token;
    # pad 1 makes the token stride odd (no 16-byte row accesses)
    n_head, n_kv, hd, T, L = 64, 8, 64, 3, 900
    qd, kd = n_head * hd, n_kv * hd
    g = torch.Generator(device="cuda").manual_seed(6)
    act = torch.randn(T, qd + 2 * kd + pad, generator=g, device="cuda")
    table = torch.from_numpy(orc.rope_table(L, hd)).cuda()
    kc = torch.zeros(L, kd, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    q_view = act[:, :qd]
    attn.qkv_rope_cache(q_view, act[:, qd:qd + kd], act[:, qd + kd:qd + 2 * kd], kc, vc, n_kv=n_kv, kv_len=L,
                        table=table, token_stride=qd + 2 * kd + pad, n_seq=1, q_tokens=T, n_head=n_head, hd=hd)
    torch.cuda.synchronize()
    a = act.cpu().numpy()
    q = a[:, :qd].reshape(1, T, n_head, hd)
    k = a[:, qd:qd + kd].reshape(1, T, n_kv, hd)
    v = a[:, qd + kd:qd + 2 * kd].reshape(1, T, n_kv, hd)
    # (q was rotated in place: recompute the oracle from the untouched k/v and the original q)
    g2 = torch.Generator(device="cuda").manual_seed(6)
    q0 = torch.randn(T, qd + 2 * kd + pad, generator=g2, device="cuda").cpu().numpy()[:, :qd].reshape(1, T, n_head, hd)
    qo, kco, vco = orc.qk_norm_rope_cache(q0, k, v, n_kv=n_kv, kv_len=L, table=table.cpu().numpy())
    assert np.abs(q.astype(np.float64) - qo).max() < 1e-5
    assert np.array_equal(to_np_f16(vc), vco)
    assert np.abs(as_f64(kc) - kco.view(np.float16).astype(np.float64)).max() < 4e-3


def test_then_decode_matches_the_oracle_chain():
    # the pair the engine runs: this step, then decode attention
    n_head, n_kv, hd, T, L = 64, 8, 64, 2, 3000
    cfg = wl.AttnConfig("chain", "decode", n_head, n_kv, hd, L, q_tokens=T, sinks=True, seed=11)
    inp = wl.make_inputs(cfg, "cuda")
    q, k, v = _case(1, T, n_head, n_kv, hd, seed=12)
    table = torch.from_numpy(orc.rope_table(L, hd)).cuda()
    kc, vc = inp.k.clone(), inp.v.clone()
    qg = q.clone()
    attn.qkv_rope_cache(qg, k, v, kc.view(L, -1), vc.view(L, -1), n_kv=n_kv, kv_len=L, table=table)
    out = attn.decode(qg, kc, vc, n_kv=n_kv, kv_len=L, sinks=inp.sinks)
    torch.cuda.synchronize()
    kco, vco = to_np_f16(inp.k).reshape(L, -1).copy(), to_np_f16(inp.v).reshape(L, -1).copy()
    qo, kco, vco = orc.qk_norm_rope_cache(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), n_kv=n_kv, kv_len=L,
                                          table=table.cpu().numpy(), k_cache=kco, v_cache=vco)
    ref = orc.attention(qo, kco, vco, n_kv=n_kv, kv_len=L, sinks=inp.sinks.cpu().numpy())
    assert_close(as_f64(out), ref.astype(np.float64), what="qkv step + decode")


def test_rejects_short_tables_and_odd_heads():
    q, k, v = _case(1, 1, 8, 8, 64, seed=7)
    kc = torch.zeros(100, 512, dtype=torch.float16, device="cuda")
    table = torch.from_numpy(orc.rope_table(50, 64)).cuda()
    with pytest.raises(attn.AttnError) as e:
        attn.qkv_rope_cache(q, k, v, kc, kc.clone(), n_kv=8, kv_len=100, table=table)
    assert e.value.code == attn.EINVAL and "rope table" in e.value.message
    q2, k2, v2 = _case(1, 1, 8, 8, 96, seed=8)
    with pytest.raises(attn.AttnError) as e:
        attn.qkv_rope_cache(q2, k2, v2, kc, kc.clone(), n_kv=8, kv_len=100)
    assert e.value.code == attn.EUNSUPPORTED
