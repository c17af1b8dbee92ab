"""Helpers of the GPU parity tests: run the HIP path through the C ABI
(pelica_amd.attn) and the CPU oracle on the same seeded inputs."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc
from pelica_amd import attn
from pelica_amd.workloads import AttnInputs


def to_np_f16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy().view(np.uint16)


def gpu_run(inp: AttnInputs, *, ring_cap=0, window=None, kv_row_stride=0, k=None, v=None, ragged=None):
    cfg = inp.cfg
    ragged = inp.ragged if ragged is None else ragged
    window = cfg.window if window is None else window
    k = inp.k if k is None else k
    v = inp.v if v is None else v
    kw = dict(n_kv=cfg.n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=window, ring_cap=ring_cap,
              kv_row_stride=kv_row_stride)
    if ragged:
        kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    fn = attn.prefill if cfg.kind == "prefill" else attn.decode
    out = fn(inp.q, k, v, **kw)
    torch.cuda.synchronize()
    return out


def oracle_run(inp: AttnInputs, *, ring_cap=0, window=None, kv_row_stride=0, k=None, v=None, t_begin=0, t_end=-1):
    cfg = inp.cfg
    window = cfg.window if window is None else window
    q = inp.q.cpu().numpy()
    if q.dtype == np.float16:
        q = q.view(np.uint16)
    k = to_np_f16(inp.k if k is None else k)
    v = to_np_f16(inp.v if v is None else v)
    sinks = None if inp.sinks is None else inp.sinks.cpu().numpy()
    offs = inp.seq_off.cpu().numpy() if (inp.ragged or not ring_cap) else None
    return orc.attention(q, k, v, n_kv=cfg.n_kv, kv_len=inp.kv_len, seq_kv_len=inp.seq_len.cpu().numpy(),
                         seq_kv_offset=offs, sinks=sinks, window=window, ring_cap=ring_cap,
                         kv_row_stride=kv_row_stride, t_begin=t_begin, t_end=t_end)


def as_f64(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu()
        if x.dtype == torch.float16:
            return x.float().numpy().astype(np.float64)
        return x.numpy().astype(np.float64)
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return x.view(np.float16).astype(np.float64)
    return x.astype(np.float64)
