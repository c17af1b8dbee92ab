"""Pins of the CPU oracle (oracle/attn_oracle.c) — CPU only.

The reference ships no attention tests or fixtures (its only pins are
run-time checks that need a model and a Vulkan GPU), so the oracle is pinned
here against what the mathematics fixes: exhaustive half-float conversion,
exp accuracy, an independent fp64 brute force, closed forms (equal keys,
single key, sink identity, window >= context, GQA == replicated MHA), and the
reference's own structural pin — AVX2 and scalar chunk paths agree bit for
bit (src/moe.rs:1909-1913, check_attn).
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.refimpl import assert_close, brute_attention, f16_bits_to_f64


def rand_f16(rng, shape, scale=0.5):
    return (rng.standard_normal(shape) * scale).astype(np.float16).view(np.uint16)


# ---- scalar helpers -------------------------------------------------------

def test_f16_to_f32_exhaustive():
    L = orc.lib()
    allbits = np.arange(65536, dtype=np.uint16)
    want = allbits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in allbits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        rng.standard_normal(5000).astype(np.float32) * 1e-5,     # subnormal halves
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 6.1035156e-05, 5.96e-08, 2.98e-08,
                  np.inf, -np.inf, 1.0 + 2**-11, 1.0 + 3 * 2**-11], np.float32),
    ])
    L = orc.lib()
    got = np.array([L.orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_pexp_matches_exp():
    xs = np.linspace(-39.9, 0.0, 4001)
    got = np.array([orc.pexp(float(np.float32(x))) for x in xs])
    want = np.exp(xs.astype(np.float32).astype(np.float64))
    rel = np.abs(got - want) / want
    assert rel.max() < 4e-7
    assert orc.pexp(0.0) == 1.0
    assert orc.pexp(-40.5) == 0.0
    assert orc.pexp(-1e30) == 0.0


# ---- one chunk (cpu_attn::chunk) -------------------------------------------

@pytest.mark.parametrize("hd,n_kv,hpk,kv0,kv1,n", [
    (64, 8, 8, 0, 8, 256), (128, 4, 8, 1, 3, 97), (128, 16, 1, 0, 16, 64), (64, 2, 4, 1, 2, 5), (128, 1, 32, 0, 1, 1),
])
def test_chunk_avx2_equals_scalar_bitwise(hd, n_kv, hpk, kv0, kv1, n):
    rng = np.random.default_rng(hd * 1000 + n)
    k = rand_f16(rng, (n, n_kv * hd))
    v = rand_f16(rng, (n, n_kv * hd))
    q = (rng.standard_normal(((kv1 - kv0) * hpk, hd)) / math.sqrt(hd)).astype(np.float32)
    a = orc.chunk(hd, n_kv, hpk, kv0, kv1, k, v, q, path="scalar")
    b = orc.chunk(hd, n_kv, hpk, kv0, kv1, k, v, q, path="avx2")
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("hd,hpk", [(64, 8), (128, 4)])
def test_chunk_partials_vs_fp64(hd, hpk):
    rng = np.random.default_rng(7)
    n_kv, n = 2, 200
    k = rand_f16(rng, (n, n_kv * hd))
    v = rand_f16(rng, (n, n_kv * hd))
    q = (rng.standard_normal((n_kv * hpk, hd)) / math.sqrt(hd)).astype(np.float32)
    part = orc.chunk(hd, n_kv, hpk, 0, n_kv, k, v, q)
    kf = f16_bits_to_f64(k).reshape(n, n_kv, hd)
    vf = f16_bits_to_f64(v).reshape(n, n_kv, hd)
    for h in range(n_kv * hpk):
        g = h // hpk
        s = kf[:, g] @ q[h].astype(np.float64)
        M = s.max()
        p = np.exp(s - M)
        # the partial's max is a stream max: compare the normalised pieces
        w = math.exp(part[h, 0] - M)
        assert abs(part[h, 0] - M) < 1e-5
        assert abs(part[h, 1] / w - p.sum()) / p.sum() < 1e-5
        np.testing.assert_allclose(part[h, 2:] / w, p @ vf[:, g], rtol=1e-4, atol=1e-5)


def test_merge_head_closed_form():
    # two partials with known (M, L, O); sink adds e^{sink-M} to the denominator
    hd = 4
    parts = np.array([[1.0, 2.0, 2, 4, 6, 8], [3.0, 1.0, 1, 1, 1, 1]], np.float32)
    w = np.exp(np.array([1.0, 3.0]) - 3.0)
    L = 2.0 * w[0] + 1.0 * w[1]
    O = parts[0, 2:] * w[0] + parts[1, 2:] * w[1]
    np.testing.assert_allclose(orc.merge_head(parts), O / L, rtol=1e-6)
    sink = 2.5
    np.testing.assert_allclose(orc.merge_head(parts, sink), O / (L + math.exp(sink - 3.0)), rtol=1e-6)
    # an empty slot (max -3e38) carries no weight
    empty = np.zeros((1, hd + 2), np.float32)
    empty[0, 0] = -3e38
    np.testing.assert_allclose(orc.merge_head(np.concatenate([parts, empty])), O / L, rtol=1e-6)


# ---- whole attention --------------------------------------------------------

def _case(rng, n_seq, T, H, n_kv, hd, lens, ring_cap=0, f16q=False):
    rows = ring_cap * n_seq if ring_cap else sum(lens)
    k = rand_f16(rng, (rows, n_kv, hd))
    v = rand_f16(rng, (rows, n_kv, hd))
    q = rng.standard_normal((n_seq, T, H, hd)).astype(np.float32)
    if f16q:
        q = (q * 0.5).astype(np.float16).view(np.uint16)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64) if not ring_cap else \
        np.arange(n_seq, dtype=np.int64) * ring_cap
    return q, k, v, offs


@pytest.mark.parametrize("n_seq,T,H,n_kv,hd,lens,window,sinks", [
    (1, 1, 16, 16, 128, [700], 0, False),          # C1-like MHA
    (1, 1, 32, 4, 128, [1000], 0, False),          # C2-like GQA
    (1, 1, 64, 8, 64, [1500], 0, True),            # C3-like with sinks
    (1, 1, 64, 8, 64, [1500], 128, True),          # C3 window
    (3, 4, 32, 4, 128, [37, 600, 300], 0, False),  # C5-like ragged drafts
    (2, 3, 8, 2, 64, [5, 260], 7, True),           # tiny window, drafts
])
def test_attention_vs_fp64(n_seq, T, H, n_kv, hd, lens, window, sinks):
    rng = np.random.default_rng(sum(lens) + T)
    q, k, v, offs = _case(rng, n_seq, T, H, n_kv, hd, lens)
    sk = rng.standard_normal(H).astype(np.float32) if sinks else None
    got = orc.attention(q, k, v, n_kv=n_kv, seq_kv_len=np.array(lens, np.int32), seq_kv_offset=offs, sinks=sk,
                        window=window)
    ref = brute_attention(q, f16_bits_to_f64(k), f16_bits_to_f64(v), n_kv=n_kv, lens=lens, offs=offs, sinks=sk,
                          window=window)
    assert_close(got, ref, atol=2e-6, rtol=2e-6, what="oracle vs fp64")


def test_attention_ring_buffer():
    rng = np.random.default_rng(11)
    H, n_kv, hd, cap, L, T, W = 16, 4, 64, 160, 1000, 3, 128
    q = rng.standard_normal((1, T, H, hd)).astype(np.float32)
    # a linear cache, and the same keys placed in a ring at j % cap
    kl = rand_f16(rng, (L, n_kv, hd))
    vl = rand_f16(rng, (L, n_kv, hd))
    kr = np.zeros((cap, n_kv, hd), np.uint16)
    vr = np.zeros((cap, n_kv, hd), np.uint16)
    for j in range(L - cap, L):
        kr[j % cap], vr[j % cap] = kl[j], vl[j]
    a = orc.attention(q, kl, vl, n_kv=n_kv, kv_len=L, window=W)
    b = orc.attention(q, kr, vr, n_kv=n_kv, kv_len=L, window=W, ring_cap=cap)
    assert np.array_equal(a, b)


def test_prefill_f16_vs_fp64():
    rng = np.random.default_rng(3)
    T, H, n_kv, hd = 300, 16, 2, 64
    q, k, v, offs = _case(rng, 1, T, H, n_kv, hd, [T], f16q=True)
    sk = rng.standard_normal(H).astype(np.float32)
    for window in (0, 64):
        got = orc.attention(q, k, v, n_kv=n_kv, kv_len=T, sinks=sk, window=window)
        assert got.dtype == np.uint16
        ref = brute_attention(f16_bits_to_f64(q), f16_bits_to_f64(k), f16_bits_to_f64(v), n_kv=n_kv, lens=[T],
                              sinks=sk, window=window)
        # only the final f16 rounding separates them
        assert_close(f16_bits_to_f64(got), ref, atol=1e-3, rtol=6e-4, what=f"prefill window {window}")


def test_closed_forms():
    rng = np.random.default_rng(5)
    H, n_kv, hd, L = 8, 2, 64, 300
    q = rng.standard_normal((1, 1, H, hd)).astype(np.float32)
    # all keys equal -> uniform weights -> mean of V
    k = np.repeat(rand_f16(rng, (1, n_kv, hd)), L, axis=0)
    v = rand_f16(rng, (L, n_kv, hd))
    got = orc.attention(q, k, v, n_kv=n_kv, kv_len=L)
    want = f16_bits_to_f64(v).mean(axis=0)[np.arange(H) // (H // n_kv)]
    np.testing.assert_allclose(got[0, 0], want, rtol=2e-5, atol=2e-6)
    # a sink with all scores equal to s: out = mean(V) * n / (n + e^{sink - s})
    s_val = float((f16_bits_to_f64(k[0]) [np.arange(H) // (H // n_kv)] * q[0, 0]).sum(-1)[0] / math.sqrt(hd))
    sinks = np.full(H, 0.3, np.float32)
    got_s = orc.attention(q, k, v, n_kv=n_kv, kv_len=L, sinks=sinks)
    s_all = (f16_bits_to_f64(k[0])[np.arange(H) // (H // n_kv)] * q[0, 0]).sum(-1) / math.sqrt(hd)
    factor = L / (L + np.exp(0.3 - s_all))
    np.testing.assert_allclose(got_s[0, 0], want * factor[:, None], rtol=2e-5, atol=2e-6)
    assert s_val == pytest.approx(s_all[0])
    # one visible key -> that key's value
    got1 = orc.attention(q, k[:1], v[:1], n_kv=n_kv, kv_len=1)
    np.testing.assert_array_equal(got1[0, 0], f16_bits_to_f64(v[0])[np.arange(H) // (H // n_kv)].astype(np.float32))
    # window >= context is full attention
    k2 = rand_f16(rng, (L, n_kv, hd))
    a = orc.attention(q, k2, v, n_kv=n_kv, kv_len=L)
    b = orc.attention(q, k2, v, n_kv=n_kv, kv_len=L, window=L)
    assert np.array_equal(a, b)


def test_gqa_equals_replicated_mha():
    rng = np.random.default_rng(9)
    H, n_kv, hd, L = 16, 2, 128, 400
    q = rng.standard_normal((1, 1, H, hd)).astype(np.float32)
    k = rand_f16(rng, (L, n_kv, hd))
    v = rand_f16(rng, (L, n_kv, hd))
    g = orc.attention(q, k, v, n_kv=n_kv, kv_len=L)
    rep = np.arange(H) // (H // n_kv)
    m = orc.attention(q, np.ascontiguousarray(k[:, rep]), np.ascontiguousarray(v[:, rep]), n_kv=H, kv_len=L)
    assert np.array_equal(g, m)


def test_partials_merge_to_attention():
    # CPU-tier partials of every chunk, merged in order, give the attention
    rng = np.random.default_rng(13)
    H, n_kv, hd, L = 32, 4, 128, 1100
    q = rng.standard_normal((1, 1, H, hd)).astype(np.float32)
    k = rand_f16(rng, (L, n_kv, hd))
    v = rand_f16(rng, (L, n_kv, hd))
    sk = rng.standard_normal(H).astype(np.float32)
    parts = orc.partials(q, k, v, n_kv=n_kv, kv_len=L)
    assert parts.shape == (5, H, hd + 2)
    merged = np.stack([orc.merge_head(parts[:, h], sk[h]) for h in range(H)])
    full = orc.attention(q, k, v, n_kv=n_kv, kv_len=L, sinks=sk)
    assert np.array_equal(merged, full[0, 0])


def test_token_subrange_and_threads_are_consistent():
    rng = np.random.default_rng(17)
    T, H, n_kv, hd = 40, 8, 2, 64
    q, k, v, _ = _case(rng, 1, T, H, n_kv, hd, [T], f16q=True)
    full = orc.attention(q, k, v, n_kv=n_kv, kv_len=T, threads=1)
    part = orc.attention(q, k, v, n_kv=n_kv, kv_len=T, t_begin=10, t_end=20, threads=3)
    assert np.array_equal(full[:, 10:20], part[:, 10:20])
    assert not part[:, :10].any() and not part[:, 20:].any()
