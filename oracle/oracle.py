"""ctypes binding of the CPU oracle (oracle/attn_oracle.c) — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module: it is the checker and the CPU baseline, never the product path.
Arrays are numpy; f16 tensors travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libattn_oracle.so")
CHUNK = 256

_lib = None


def build() -> str:
    """Compile the oracle (gcc, oracle/Makefile) and return the library path."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class OrcRope(ctypes.Structure):
    _fields_ = [
        ("rot", ctypes.c_int32),
        ("neox", ctypes.c_int32),
        ("table_split", ctypes.c_int32),
        ("table", ctypes.c_void_p),
    ]


class OrcDesc(ctypes.Structure):
    _fields_ = [
        ("n_head", ctypes.c_int32),
        ("n_kv", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("n_seq", ctypes.c_int32),
        ("q_tokens", ctypes.c_int32),
        ("seq_kv_len", ctypes.c_void_p),
        ("seq_kv_off", ctypes.c_void_p),
        ("kv_row_stride", ctypes.c_int64),
        ("window", ctypes.c_int32),
        ("ring_cap", ctypes.c_int32),
        ("scale", ctypes.c_float),
    ]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        L.orc_pexp.restype = ctypes.c_float
        L.orc_pexp.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        for name in ("orc_chunk", "orc_chunk_scalar"):
            f = getattr(L, name)
            f.restype = None
            f.argtypes = [i32, i32, i32, i32, i32, i32, vp, vp, vp, vp]
        L.orc_chunk_avx2.restype = i32
        L.orc_chunk_avx2.argtypes = [i32, i32, i32, i32, i32, i32, vp, vp, vp, vp]
        L.orc_merge_head.restype = None
        L.orc_merge_head.argtypes = [i32, i32, vp, ctypes.c_size_t, vp, vp]
        dp = ctypes.POINTER(OrcDesc)
        L.orc_attn.restype = i32
        L.orc_attn.argtypes = [dp, vp, vp, vp, vp, vp, i32, i32, i32]
        L.orc_attn_f16.restype = i32
        L.orc_attn_f16.argtypes = [dp, vp, vp, vp, vp, vp, i32, i32, i32]
        L.orc_partials.restype = i32
        L.orc_partials.argtypes = [dp, vp, vp, vp, i32, i32, i32, i32, vp, i32]
        L.orc_qk_norm_rope_cache.restype = i32
        L.orc_qk_norm_rope_cache.argtypes = [dp, ctypes.POINTER(OrcRope), vp, vp, vp, vp, vp, ctypes.c_float, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def pexp(x: float) -> float:
    return lib().orc_pexp(x)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def chunk(hd, n_kv, hpk, kv0, kv1, k, v, q, *, path="auto"):
    """cpu_attn::chunk: k, v uint16 [n, n_kv*hd]; q f32 heads of [kv0,kv1)
    (already scaled).  Returns f32 [(kv1-kv0)*hpk, hd+2]."""
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    q = _c(q, np.float32)
    n = k.size // (n_kv * hd)
    assert n <= CHUNK and v.size == k.size
    out = np.zeros(((kv1 - kv0) * hpk, hd + 2), np.float32)
    L = lib()
    args = (hd, n_kv, hpk, kv0, kv1, n, _p(k), _p(v), _p(q), _p(out))
    if path == "scalar":
        L.orc_chunk_scalar(*args)
    elif path == "avx2":
        if not L.orc_chunk_avx2(*args):
            raise RuntimeError("no AVX2/FMA/F16C on this CPU")
    else:
        L.orc_chunk(*args)
    return out


def merge_head(parts, sink=None):
    """Combine [n_parts, hd+2] partials of one head in order (with a sink)."""
    parts = _c(parts, np.float32)
    hd = parts.shape[-1] - 2
    out = np.zeros(hd, np.float32)
    s = None if sink is None else np.array([sink], np.float32)
    lib().orc_merge_head(hd, parts.shape[0], _p(parts), hd + 2, _p(s), _p(out))
    return out


def _desc(n_head, n_kv, hd, n_seq, q_tokens, seq_len, seq_off, row_stride, window, ring_cap, scale):
    d = OrcDesc()
    d.n_head, d.n_kv, d.hd, d.n_seq, d.q_tokens = n_head, n_kv, hd, n_seq, q_tokens
    d.seq_kv_len = _p(seq_len)
    d.seq_kv_off = _p(seq_off)
    d.kv_row_stride = row_stride or n_kv * hd
    d.window, d.ring_cap = window, ring_cap
    d.scale = scale if scale is not None else 1.0 / np.sqrt(hd)
    return d


def attention(q, k, v, *, n_kv, kv_len=None, seq_kv_len=None, seq_kv_offset=None, sinks=None, window=0,
              ring_cap=0, scale=None, kv_row_stride=0, t_begin=0, t_end=-1, threads=0):
    """Oracle attention.  q f32 [n_seq, T, n_head, hd] -> f32 (decode), or
    q uint16 (f16 bits) -> uint16 (prefill, f16 output).  k, v: uint16 cache
    rows.  Lengths default to kv_len for every sequence."""
    n_seq, T, n_head, hd = q.shape
    f16 = q.dtype == np.uint16
    q = _c(q, np.uint16 if f16 else np.float32)
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    if seq_kv_len is None:
        seq_kv_len = np.full(n_seq, kv_len, np.int32)
    seq_kv_len = _c(seq_kv_len, np.int32)
    if seq_kv_offset is not None:
        seq_kv_offset = _c(seq_kv_offset, np.int64)
    elif n_seq > 1:
        per = ring_cap if ring_cap else int(kv_len)
        seq_kv_offset = np.arange(n_seq, dtype=np.int64) * per
    s = _c(sinks, np.float32)
    d = _desc(n_head, n_kv, hd, n_seq, T, seq_kv_len, seq_kv_offset, kv_row_stride, window, ring_cap, scale)
    out = np.zeros(q.shape, q.dtype)
    fn = lib().orc_attn_f16 if f16 else lib().orc_attn
    rc = fn(ctypes.byref(d), _p(q), _p(k), _p(v), _p(s), _p(out), t_begin, t_end, threads)
    if rc != 0:
        raise ValueError("oracle rejected the descriptor")
    return out


def partials(q, k, v, *, n_kv, kv_len, s=0, t=0, k_begin=0, k_end=None, sinks=None, window=0, scale=None,
             threads=0):
    """CPU-tier partials of keys [k_begin, k_end) for one token: one
    [n_head, hd+2] slot per 256-position chunk (natural-log max)."""
    n_seq, T, n_head, hd = q.shape
    q = _c(q, np.float32)
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    lens = np.full(n_seq, kv_len, np.int32)
    offs = np.arange(n_seq, dtype=np.int64) * kv_len
    d = _desc(n_head, n_kv, hd, n_seq, T, lens, offs, 0, window, 0, scale)
    k_end = kv_len if k_end is None else k_end
    n_slots = (k_end - 1) // CHUNK - k_begin // CHUNK + 1
    out = np.zeros((max(n_slots, 0), n_head, hd + 2), np.float32)
    n = lib().orc_partials(ctypes.byref(d), _p(q), _p(k), _p(v), s, t, k_begin, k_end, _p(out), threads)
    if n < 0:
        raise ValueError("oracle rejected the descriptor")
    return out[:n]


def rope_table(n_pos, rot, base=10000.0, split=False):
    """(cos, sin) table [rows, rot/2, 2] f32 for plain rotary angles
    theta = pos * base^(-2j/rot), computed in f64 like the engines' tables
    (src/oss.rs:1320-1349, src/moe.rs:484-519, without YaRN).  split=True
    gives the two-level layout: rows pos = 256 i (i < n_hi), then pos = p
    (p < 256); returns (table, n_hi)."""
    half = rot // 2
    freq = base ** (-(2.0 * np.arange(half)) / rot)
    if split:
        n_hi = -(-n_pos // 256)
        pos = np.concatenate([256.0 * np.arange(n_hi), np.arange(256.0)])
    else:
        n_hi = 0
        pos = np.arange(float(n_pos))
    th = pos[:, None] * freq[None, :]
    t = np.stack([np.cos(th), np.sin(th)], -1).astype(np.float32)
    return (t, n_hi) if split else t


def qk_norm_rope_cache(q, k, v, *, n_kv, kv_len=None, seq_kv_len=None, seq_kv_offset=None, ring_cap=0,
                       kv_row_stride=0, cache_rows=None, k_cache=None, v_cache=None, rot=None, neox=True,
                       table=None, table_split=0, q_norm=None, k_norm=None, eps=1e-6):
    """Oracle of the step before attention.  q f32 [n_seq, T, n_head, hd]
    (returned rotated), k, v f32 [n_seq, T, n_kv, hd]; the new rows land in
    uint16 (f16 bits) caches, returned (given ones are updated)."""
    n_seq, T, n_head, hd = q.shape
    q = np.array(q, np.float32, copy=True)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    if seq_kv_len is None:
        seq_kv_len = np.full(n_seq, kv_len, np.int32)
    seq_kv_len = _c(seq_kv_len, np.int32)
    if seq_kv_offset is None:
        span = ring_cap or int(seq_kv_len.max())
        seq_kv_offset = np.arange(n_seq, dtype=np.int64) * span
    seq_kv_offset = _c(seq_kv_offset, np.int64)
    stride = kv_row_stride or n_kv * hd
    if k_cache is None:
        rows = cache_rows or int(seq_kv_offset.max()) + (ring_cap or int(seq_kv_len.max()))
        k_cache = np.zeros((rows, stride), np.uint16)
        v_cache = np.zeros((rows, stride), np.uint16)
    d = _desc(n_head, n_kv, hd, n_seq, T, seq_kv_len, seq_kv_offset, stride, 0, ring_cap, None)
    r = None
    if table is not None:
        table = _c(table, np.float32)
        r = OrcRope(rot or hd, 1 if neox else 0, table_split, _p(table))
    qn = _c(q_norm, np.float32)
    kn = _c(k_norm, np.float32)
    rc = lib().orc_qk_norm_rope_cache(ctypes.byref(d), None if r is None else ctypes.byref(r), _p(q), _p(k), _p(v),
                                      _p(qn), _p(kn), eps, _p(k_cache), _p(v_cache))
    if rc != 0:
        raise ValueError("oracle rejected the descriptor")
    return q, k_cache, v_cache
