"""fp64 brute-force attention and tolerance checks shared by the tests.

The brute force is the textbook definition, written independently of the
oracle: softmax over the visible keys (plus the sink logit in the
denominator), weighted sum of values, all in float64.
"""
from __future__ import annotations

import numpy as np

ATOL = 2e-3   # max |gpu - ref|
RTOL = 1e-3   # ||gpu - ref||_2 / ||ref||_2


def f16_bits_to_f64(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float64)


def brute_attention(q, k, v, *, n_kv, lens, offs=None, sinks=None, window=0, ring_cap=0, scale=None,
                    tokens=None):
    """q [n_seq, T, H, hd] (float), k/v [rows, n_kv, hd] (float), f64 out.
    ``tokens``: optional list of token indices to compute (others NaN)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64).reshape(-1, n_kv, q.shape[-1])
    v = np.asarray(v, np.float64).reshape(-1, n_kv, q.shape[-1])
    n_seq, T, H, hd = q.shape
    hpk = H // n_kv
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    if offs is None:
        per = ring_cap if ring_cap else lens[0]
        offs = [s * per for s in range(n_seq)]
    out = np.full(q.shape, np.nan)
    heads_kv = np.arange(H) // hpk
    for s in range(n_seq):
        for t in (range(T) if tokens is None else tokens):
            pos = lens[s] - T + t
            lo = max(0, pos + 1 - window) if window else 0
            j = np.arange(lo, pos + 1)
            rows = offs[s] + (j % ring_cap if ring_cap else j)
            kk = k[rows][:, heads_kv, :]          # [n, H, hd]
            vv = v[rows][:, heads_kv, :]
            sc = np.einsum("nhd,hd->hn", kk, q[s, t]) * scale   # [H, n]
            m = sc.max(axis=1)
            if sinks is not None:
                m = np.maximum(m, np.asarray(sinks, np.float64))
            p = np.exp(sc - m[:, None])
            den = p.sum(axis=1)
            if sinks is not None:
                den = den + np.exp(np.asarray(sinks, np.float64) - m)
            out[s, t] = np.einsum("hn,nhd->hd", p, vv) / den[:, None]
    return out


def errors(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    mask = ~np.isnan(ref)
    d = got[mask] - ref[mask]
    max_abs = float(np.abs(d).max()) if d.size else 0.0
    rel = float(np.linalg.norm(d) / max(np.linalg.norm(ref[mask]), 1e-30)) if d.size else 0.0
    return max_abs, rel


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    max_abs, rel = errors(got, ref)
    assert np.isfinite(np.asarray(got, np.float64)[~np.isnan(np.asarray(ref, np.float64))]).all(), f"{what}: non-finite"
    assert max_abs <= atol and rel <= rtol, f"{what}: max_abs {max_abs:.3g} (<= {atol}), rel {rel:.3g} (<= {rtol})"
    return max_abs, rel
