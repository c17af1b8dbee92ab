"""Write the golden fixtures of the attention path (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no attention fixtures, so these freeze the CPU oracle's
outputs (and an fp64 brute force next to them) on small seeded inputs that
cover each feature: GQA decode, sinks, windows, drafts, ragged batches, ring
caches and f16 prefill.  tests/test_golden.py checks the oracle reproduces
them bit for bit and stays within 2e-6 of the fp64 values; the GPU tests
check the HIP path against them.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402
from tests.refimpl import brute_attention, f16_bits_to_f64  # noqa: E402

CASES = {
    # name: (n_seq, T, H, n_kv, hd, lens, window, sinks, ring_cap, prefill)
    "decode_gqa_sinks": (1, 1, 16, 2, 64, [300], 0, True, 0, False),
    "decode_mha_hd128": (1, 1, 4, 4, 128, [257], 0, False, 0, False),
    "decode_window_drafts": (1, 3, 8, 2, 64, [200], 50, True, 0, False),
    "decode_ragged": (3, 2, 8, 1, 128, [2, 70, 300], 0, False, 0, False),
    "decode_ring": (1, 2, 8, 2, 64, [500], 64, True, 96, False),
    "prefill_causal_sinks": (1, 80, 8, 2, 64, [80], 0, True, 0, True),
    "prefill_window": (1, 70, 4, 1, 128, [100], 16, False, 0, True),
}


def make(name):
    n_seq, T, H, n_kv, hd, lens, window, sinks, ring, prefill = CASES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    rows = ring * n_seq if ring else sum(lens)
    k = (rng.standard_normal((rows, n_kv, hd)) * 0.5).astype(np.float16).view(np.uint16)
    v = (rng.standard_normal((rows, n_kv, hd)) * 0.5).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((n_seq, T, H, hd)).astype(np.float32)
    if prefill:
        q = (q * 0.5).astype(np.float16).view(np.uint16)
    sk = rng.standard_normal(H).astype(np.float32) if sinks else None
    offs = (np.arange(n_seq) * ring if ring else np.concatenate([[0], np.cumsum(lens)[:-1]])).astype(np.int64)
    lens = np.array(lens, np.int32)
    out = orc.attention(q, k, v, n_kv=n_kv, seq_kv_len=lens, seq_kv_offset=offs, sinks=sk, window=window,
                        ring_cap=ring)
    qf = f16_bits_to_f64(q) if prefill else q
    ref = brute_attention(qf, f16_bits_to_f64(k), f16_bits_to_f64(v), n_kv=n_kv, lens=list(lens), offs=list(offs),
                          sinks=sk, window=window, ring_cap=ring)
    arrays = dict(q=q, k=k, v=v, lens=lens, offs=offs, out=out, ref64=ref,
                  meta=np.array([n_seq, T, H, n_kv, hd, window, ring, int(prefill)], np.int64))
    if sk is not None:
        arrays["sinks"] = sk
    return arrays


if __name__ == "__main__":
    for name in CASES:
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **make(name))
        print("wrote", name)
