"""GPU parity of pelica_attn_decode_partials (the VRAM rows' partial slots
that the CPU tier's slots complete, src/moe.rs:1600-1606,1713-1729) and of a
decode whose cache lives in host-visible (pinned) memory.

Tolerance (north star): max |gpu - oracle| <= 2e-3 and
||gpu - oracle||_2 / ||oracle||_2 <= 1e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pelica_amd import attn
from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, oracle_run, to_np_f16
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def _empty_slots(n, n_head, hd):
    e = np.zeros((n, n_head, hd + 2), np.float32)
    e[:, :, 0] = -3e38
    return e


@pytest.mark.parametrize("n_head,n_kv,hd,L,nv", [(64, 8, 64, 5000, 3000), (16, 16, 128, 2048, 1024),
                                                  (32, 4, 128, 9000, 8191), (64, 8, 64, 40000, 32768)])
def test_vram_partials_join_cpu_tier(n_head, n_kv, hd, L, nv):
    # keys [0, nv) on the GPU, [nv, L) on the CPU tier (cpu_attn chunks),
    # merged with the sinks in slot order == attention over all L keys
    print(f"[case] vram+cpu h{n_head}/{n_kv} hd{hd} L{L} nv{nv}", flush=True)
    cfg = wl.AttnConfig("tier", "decode", n_head, n_kv, hd, L, sinks=True, seed=nv)
    inp = wl.make_inputs(cfg, "cuda")
    gpu = attn.decode_partials(inp.q, inp.k[:nv].contiguous(), inp.v[:nv].contiguous(), n_kv=n_kv, kv_len=nv)
    torch.cuda.synchronize()
    q = inp.q.cpu().numpy()
    cpu = orc.partials(q, to_np_f16(inp.k), to_np_f16(inp.v), n_kv=n_kv, kv_len=L, k_begin=nv, k_end=L)
    slots = np.concatenate([gpu.cpu().numpy()[0], _empty_slots(2, n_head, hd), cpu])
    out = attn.partials_merge(torch.from_numpy(slots).cuda(), n_head=n_head, hd=hd, sinks=inp.sinks)
    torch.cuda.synchronize()
    assert_close(as_f64(out), as_f64(oracle_run(inp))[0, 0], what="vram + cpu tier")


@pytest.mark.parametrize("cfg", [wl.C3_FULL.scaled(kv_len=7000), wl.C3_SWA.scaled(kv_len=7000),
                                 wl.AttnConfig("drafts", "decode", 32, 4, 128, 3000, q_tokens=4, n_seq=3,
                                               ragged=(100, 3000), sinks=True, seed=7),
                                 wl.AttnConfig("short", "decode", 16, 16, 128, 100, sinks=True, seed=8)],
                         ids=lambda c: c.name)
def test_partials_merge_to_decode(cfg):
    # each token's slot merged alone with the sinks is the decode output
    print(f"[case] partials vs decode {cfg.name}", flush=True)
    inp = wl.make_inputs(cfg, "cuda")
    kw = dict(n_kv=cfg.n_kv, kv_len=inp.kv_len, window=cfg.window)
    if inp.ragged:
        kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    parts = attn.decode_partials(inp.q, inp.k, inp.v, **kw)
    torch.cuda.synchronize()
    assert parts.shape == (cfg.n_seq, cfg.q_tokens, cfg.n_head, cfg.hd + 2)
    ref = as_f64(oracle_run(inp))
    for s in range(cfg.n_seq):
        for t in range(cfg.q_tokens):
            out = attn.partials_merge(parts[s, t].contiguous(), n_head=cfg.n_head, hd=cfg.hd, sinks=inp.sinks)
            torch.cuda.synchronize()
            assert_close(as_f64(out), ref[s, t], what=f"{cfg.name} s{s} t{t}")


def test_partials_max_is_natural_log():
    # one key: M = q.k * scale (natural log), L = 1, O = v
    cfg = wl.AttnConfig("one", "decode", 8, 8, 64, 1, seed=9)
    inp = wl.make_inputs(cfg, "cuda")
    parts = attn.decode_partials(inp.q, inp.k, inp.v, n_kv=8, kv_len=1)
    torch.cuda.synchronize()
    p = parts.cpu().numpy()[0, 0].astype(np.float64)
    q = inp.q.cpu().numpy()[0, 0].astype(np.float64)
    k = inp.k.float().cpu().numpy()[0].astype(np.float64)
    v = inp.v.float().cpu().numpy()[0].astype(np.float64)
    m = np.einsum("hd,hd->h", q, k) / np.sqrt(64)
    assert np.abs(p[:, 0] - m).max() < 1e-3
    assert np.abs(p[:, 1] - 1).max() < 1e-6
    assert np.abs(p[:, 2:] - v).max() < 1e-6


def test_partials_need_a_buffer():
    inp = wl.make_inputs(wl.C3_FULL.scaled(kv_len=64), "cuda")
    desc = attn.make_desc(64, 8, 64, kv_len=64)
    lib = attn.load_library()
    rc = lib.pelica_attn_decode_partials(ctypes.byref(desc), inp.q.data_ptr(), inp.k.data_ptr(), inp.v.data_ptr(),
                                         None, None, 0, None)
    assert rc == attn.EINVAL and "parts" in lib.pelica_attn_last_error().decode()


def _hip():
    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    return None


def test_decode_reads_host_visible_cache():
    # the RAM tier read in place over the bus: K/V in pinned, device-mapped
    # host memory (hipHostMalloc, mapped), same result as from HBM
    hip = _hip()
    if hip is None:
        pytest.skip("libamdhip64 not loadable")
    cfg = wl.C3_FULL.scaled(kv_len=3000)
    inp = wl.make_inputs(cfg, "cuda")
    nbytes = inp.k.numel() * 2
    host, dev = [], []
    try:
        for t in (inp.k, inp.v):
            h = ctypes.c_void_p()
            assert hip.hipHostMalloc(ctypes.byref(h), ctypes.c_size_t(nbytes), ctypes.c_uint(0x2)) == 0
            host.append(h)
            d = ctypes.c_void_p()
            if hip.hipHostGetDevicePointer(ctypes.byref(d), h, ctypes.c_uint(0)) != 0 or not d.value:
                pytest.skip("no device mapping for pinned memory")
            dev.append(d)
            src = to_np_f16(t)
            ctypes.memmove(h.value, src.ctypes.data, nbytes)
        torch.cuda.synchronize()
        print(f"[case] host-visible cache {cfg.name}", flush=True)
        desc = attn.make_desc(64, 8, 64, kv_len=3000)
        lib = attn.load_library()
        need = lib.pelica_attn_workspace_bytes(ctypes.byref(desc))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(inp.q)
        rc = lib.pelica_attn_decode(ctypes.byref(desc), inp.q.data_ptr(), dev[0].value, dev[1].value,
                                    inp.sinks.data_ptr(), out.data_ptr(), ws.data_ptr(), need, None)
        assert rc == 0, lib.pelica_attn_last_error()
        torch.cuda.synchronize()
        assert_close(as_f64(out), as_f64(oracle_run(inp)), what="host-visible cache")
    finally:
        torch.cuda.synchronize()
        for h in host:
            hip.hipHostFree(h)


@pytest.mark.parametrize("n_head,n_kv,hd,T,L,nv", [(64, 8, 64, 4, 6000, 4000), (32, 4, 128, 4, 5000, 3000),
                                                    (32, 4, 128, 8, 2100, 2048)])
def test_draft_pass_joins_cpu_tier_batched(n_head, n_kv, hd, T, L, nv):
    # a draft-verify pass whose cache spills past the GPU: keys [0, nv) on
    # the GPU (every draft sees all of them), [nv, L) on the CPU tier (draft
    # t sees up to its own position L - T + t); one batched merge of all the
    # drafts' slots with the sinks == attention over the whole cache
    print(f"[case] drafts vram+cpu h{n_head}/{n_kv} hd{hd} T{T} L{L} nv{nv}", flush=True)
    cfg = wl.AttnConfig("tierT", "decode", n_head, n_kv, hd, L, q_tokens=T, sinks=True, seed=nv + T)
    inp = wl.make_inputs(cfg, "cuda")
    # the GPU's slot: the T drafts as T one-token rows over the same nv rows
    lens = torch.full((T,), nv, dtype=torch.int32, device="cuda")
    offs = torch.zeros(T, dtype=torch.int64, device="cuda")
    qg = inp.q.reshape(T, 1, n_head, hd).contiguous()
    gpu = attn.decode_partials(qg, inp.k[:nv].contiguous(), inp.v[:nv].contiguous(), n_kv=n_kv, kv_len=nv,
                               seq_kv_len=lens, seq_kv_offset=offs)
    torch.cuda.synchronize()
    q = inp.q.cpu().numpy()
    cpu = [orc.partials(q, to_np_f16(inp.k), to_np_f16(inp.v), n_kv=n_kv, kv_len=L, t=t, k_begin=nv, k_end=L)
           for t in range(T)]
    n_cpu = max(len(c) for c in cpu)
    slots = np.zeros((2 + n_cpu, T, n_head, hd + 2), np.float32)
    slots[:, :, :, 0] = -3e38
    slots[0] = gpu.cpu().numpy()[:, 0]
    for t, c in enumerate(cpu):     # slot 1 stays empty; each draft's chunks after it
        slots[2:2 + len(c), t] = c
    out = attn.partials_merge_batch(torch.from_numpy(slots).cuda(), sinks=inp.sinks)
    torch.cuda.synchronize()
    assert_close(as_f64(out), as_f64(oracle_run(inp))[0], what="drafts vram + cpu tier")


@pytest.mark.parametrize("n_parts", [1, 3, 700, 2500])
def test_partials_merge_batch_matches_per_token(n_parts):
    # the batched merge of (token, head) rows equals the one-token merge of
    # each row, and the fp64 merge formula (a textbook log-sum-exp), on
    # random slots with empties among them
    print(f"[case] merge batch n_parts {n_parts}", flush=True)
    rng = np.random.default_rng(n_parts)
    T, H, hd = 3, 16, 128
    parts = np.empty((n_parts, T, H, hd + 2), np.float32)
    parts[..., 0] = rng.normal(0, 4, (n_parts, T, H))
    parts[..., 1] = rng.uniform(0.5, 40, (n_parts, T, H))
    parts[..., 2:] = rng.normal(0, 3, (n_parts, T, H, hd))
    if n_parts > 2:
        parts[1::3, :, :, 0] = -3e38
    sinks = rng.normal(0, 1, H).astype(np.float32)
    dp = torch.from_numpy(parts).cuda()
    ds = torch.from_numpy(sinks).cuda()
    out = attn.partials_merge_batch(dp, sinks=ds)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    p = parts.astype(np.float64)
    M = np.maximum(p[..., 0].max(axis=0), sinks[None, :])
    w = np.exp(p[..., 0] - M[None])
    L = (p[..., 1] * w).sum(axis=0) + np.exp(sinks[None, :] - M)
    ref = (p[..., 2:] * w[..., None]).sum(axis=0) / L[..., None]
    assert_close(got, ref, what="batched merge vs fp64")
    for t in range(T):
        one = attn.partials_merge(dp[:, t].contiguous(), n_head=H, hd=hd, sinks=ds)
        torch.cuda.synchronize()
        assert np.array_equal(one.cpu().numpy(), out[t].cpu().numpy()), f"token {t}"
