"""Seeded random shapes through the C ABI against the CPU oracle: head dim,
GQA group size, kv head count (including counts the 8-wave decode shape
does not take), draft tokens, batch size and ragged lengths, windows,
sinks and prompt prefixes drawn together, so combinations that the
per-feature tests do not list are covered too.  The draw is fixed (seeded),
so a failure names a reproducible case.

Tolerance (north star): max |gpu - oracle| <= 2e-3 and
||gpu - oracle||_2 / ||oracle||_2 <= 1e-3.
"""
import random

import pytest

from pelica_amd import workloads as wl
from tests.gpu_util import as_f64, gpu_run, oracle_run
from tests.refimpl import assert_close

pytestmark = pytest.mark.gpu


def _decode_case(i):
    r = random.Random(1000 + i)
    hd = r.choice((64, 128))
    n_kv = r.choice((1, 2, 3, 4, 8))
    hpk = r.choice((1, 2, 4, 8))
    T = r.choice((1, 1, 2, 3, 4))
    n_seq = r.choice((1, 1, 2, 3))
    kv_len = r.randint(T, 3000)
    ragged = (r.randint(T, kv_len), kv_len) if n_seq > 1 and r.random() < 0.7 else None
    window = r.choice((0, 0, r.randint(1, kv_len + 8)))
    return wl.AttnConfig(f"rand_decode_{i}", "decode", n_kv * hpk, n_kv, hd, kv_len, q_tokens=T, n_seq=n_seq,
                         window=window, sinks=r.random() < 0.5, ragged=ragged, seed=5000 + i)


def _prefill_case(i):
    r = random.Random(2000 + i)
    hd = r.choice((64, 128))
    n_kv = r.choice((1, 2, 4, 8))
    hpk = r.choice((1, 2, 4, 8))
    T = r.randint(1, 300)
    prefix = r.choice((0, 0, r.randint(1, 500)))
    n_seq = r.choice((1, 1, 2))
    window = r.choice((0, 0, r.randint(1, T + prefix + 8)))
    return wl.AttnConfig(f"rand_prefill_{i}", "prefill", n_kv * hpk, n_kv, hd, T + prefix, q_tokens=T, n_seq=n_seq,
                         window=window, sinks=r.random() < 0.5, seed=6000 + i)


def _describe(c):
    return (f"{c.name}: hd{c.hd} h{c.n_head}/{c.n_kv} T{c.q_tokens} n_seq{c.n_seq} len{c.kv_len} "
            f"ragged{c.ragged} window{c.window} sinks{c.sinks}")


@pytest.mark.parametrize("i", range(32))
def test_random_decode(i):
    cfg = _decode_case(i)
    what = _describe(cfg)
    print(f"[case] {what}", flush=True)
    inp = wl.make_inputs(cfg, "cuda")
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what=what)


@pytest.mark.parametrize("i", range(24))
def test_random_prefill(i):
    cfg = _prefill_case(i)
    what = _describe(cfg)
    print(f"[case] {what}", flush=True)
    inp = wl.make_inputs(cfg, "cuda")
    assert_close(as_f64(gpu_run(inp)), as_f64(oracle_run(inp)), what=what)
