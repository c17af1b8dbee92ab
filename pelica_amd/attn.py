"""Host binding of libpelica_attn.so (include/pelica_attn.h) for torch tensors.

The reference has no single attention function: its engines record WGSL
dispatches (src/moe.rs:1343,1364 decode; src/oss.rs:675-694 gpt-oss decode and
drafts; src/oss.rs:734-741 prompt) and its CPU tier calls
``cpu_attn::chunk(&Shape, kv, k, v, q, out)`` (src/cpu_attn.rs:72).  This
module mirrors that surface: ``Shape`` is ``cpu_attn::Shape``
(src/cpu_attn.rs:13-26), ``decode`` / ``decode_partials`` / ``prefill`` /
``partials_merge`` are the C entry points.  Errors come back as ``AttnError`` carrying the C status
and the library's message (the reference returns ``anyhow::Result`` from its
engine calls).

There is no CPU fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
EHIP = -3
EWORKSPACE = -4

#: every symbol include/pelica_attn.h declares
EXPORTS = (
    "pelica_attn_version",
    "pelica_attn_last_error",
    "pelica_attn_reload_tuning",
    "pelica_attn_workspace_bytes",
    "pelica_attn_workspace_init",
    "pelica_attn_decode",
    "pelica_attn_decode_noalloc",
    "pelica_attn_decode_partials",
    "pelica_attn_decode_partials_range",
    "pelica_attn_mla_workspace_bytes",
    "pelica_attn_mla",
    "pelica_attn_prefill",
    "pelica_attn_prefill_f32",
    "pelica_attn_prefill_round",
    "pelica_attn_prefill_round_f32",
    "pelica_attn_partials_merge",
    "pelica_attn_partials_merge_batch",
    "pelica_attn_qkv_rope_cache",
    "pelica_attn_prof_enable",
    "pelica_attn_prof_read",
)

#: kernel ids of the per-kernel timing records
PROF_KERNELS = {1: "decode_split", 2: "decode_combine", 3: "prefill", 4: "partials_merge", 5: "qkv_rope_cache"}


class AttnError(RuntimeError):
    """A failed libpelica_attn call: ``code`` is the C status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"pelica_attn error {code}: {message}")
        self.code = code
        self.message = message


@dataclass(frozen=True)
class Shape:
    """``cpu_attn::Shape``: dims per head, kv heads, query heads per kv head."""

    hd: int
    n_kv: int
    hpk: int

    def row(self) -> int:
        """f16 values per cache row (one position's keys or values)."""
        return self.n_kv * self.hd

    @property
    def n_head(self) -> int:
        return self.n_kv * self.hpk


class Rope(ctypes.Structure):
    """``PelicaRope``: rotary dims, NeoX pairing, table layout and rows."""

    _fields_ = [
        ("rot", ctypes.c_int32),
        ("neox", ctypes.c_int32),
        ("table_split", ctypes.c_int32),
        ("table_rows", ctypes.c_int32),
        ("table", ctypes.c_void_p),
    ]


class ProfRecord(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int32), ("ms", ctypes.c_float)]


# PelicaAttnDesc.flags: decode runs its key-split kernel only (measurement)
FLAG_SPLIT_ONLY = 1


class AttnDesc(ctypes.Structure):
    """``PelicaAttnDesc`` (field meanings in include/pelica_attn.h)."""

    _fields_ = [
        ("n_head", ctypes.c_int32),
        ("n_kv", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("n_seq", ctypes.c_int32),
        ("q_tokens", ctypes.c_int32),
        ("kv_len", ctypes.c_int32),
        ("seq_kv_len", ctypes.c_void_p),
        ("seq_kv_offset", ctypes.c_void_p),
        ("kv_row_stride", ctypes.c_int64),
        ("window", ctypes.c_int32),
        ("ring_cap", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("q_token_stride", ctypes.c_int64),
        ("out_token_stride", ctypes.c_int64),
    ]


_lib = None


def library_path() -> str:
    return os.environ.get("PELICA_ATTN_LIB", os.path.join(_HERE, "lib", "libpelica_attn.so"))


def load_library() -> ctypes.CDLL:
    """Load libpelica_attn.so once.  Raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise AttnError(EHIP, f"{path} is not built (run __graft_entry__.build() or make -C pelica_amd/csrc)")
    try:  # the HIP runtime torch ships must be the one the library binds to
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
    dp = ctypes.POINTER(AttnDesc)
    lib.pelica_attn_version.restype = ctypes.c_int
    lib.pelica_attn_version.argtypes = []
    lib.pelica_attn_last_error.restype = ctypes.c_char_p
    lib.pelica_attn_last_error.argtypes = []
    lib.pelica_attn_reload_tuning.restype = ctypes.c_int
    lib.pelica_attn_reload_tuning.argtypes = []
    lib.pelica_attn_workspace_bytes.restype = sz
    lib.pelica_attn_workspace_bytes.argtypes = [dp]
    lib.pelica_attn_workspace_init.restype = ctypes.c_int
    lib.pelica_attn_workspace_init.argtypes = [vp, sz, vp]
    lib.pelica_attn_decode.restype = ctypes.c_int
    lib.pelica_attn_decode.argtypes = [dp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pelica_attn_decode_noalloc.restype = ctypes.c_int
    lib.pelica_attn_decode_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, vp]
    lib.pelica_attn_decode_partials.restype = ctypes.c_int
    lib.pelica_attn_decode_partials.argtypes = [dp, vp, vp, vp, vp, vp, sz, vp]
    lib.pelica_attn_decode_partials_range.restype = ctypes.c_int
    lib.pelica_attn_decode_partials_range.argtypes = [dp, vp, vp, vp, i32, i32, vp, vp, sz, vp]
    lib.pelica_attn_prefill.restype = ctypes.c_int
    lib.pelica_attn_prefill.argtypes = [dp, vp, vp, vp, vp, vp, vp]
    lib.pelica_attn_prefill_f32.restype = ctypes.c_int
    lib.pelica_attn_prefill_f32.argtypes = [dp, vp, vp, vp, vp, vp, vp]
    lib.pelica_attn_mla_workspace_bytes.restype = sz
    lib.pelica_attn_mla_workspace_bytes.argtypes = [dp]
    lib.pelica_attn_mla.restype = ctypes.c_int
    lib.pelica_attn_mla.argtypes = [dp, vp, vp, vp, vp, sz, vp]
    lib.pelica_attn_prefill_round.restype = ctypes.c_int
    lib.pelica_attn_prefill_round.argtypes = [dp, vp, vp, vp, i32, i32, vp, vp, i32, vp, vp]
    lib.pelica_attn_prefill_round_f32.restype = ctypes.c_int
    lib.pelica_attn_prefill_round_f32.argtypes = [dp, vp, vp, vp, i32, i32, vp, vp, i32, vp, vp]
    lib.pelica_attn_qkv_rope_cache.restype = ctypes.c_int
    lib.pelica_attn_qkv_rope_cache.argtypes = [dp, ctypes.POINTER(Rope), vp, vp, vp, ctypes.c_int64, vp, vp,
                                               ctypes.c_float, vp, vp, vp]
    lib.pelica_attn_partials_merge.restype = ctypes.c_int
    lib.pelica_attn_partials_merge.argtypes = [i32, i32, i32, vp, vp, vp, vp]
    lib.pelica_attn_partials_merge_batch.restype = ctypes.c_int
    lib.pelica_attn_partials_merge_batch.argtypes = [i32, i32, i32, i32, vp, vp, vp, vp]
    lib.pelica_attn_prof_enable.restype = ctypes.c_int
    lib.pelica_attn_prof_enable.argtypes = [ctypes.c_int]
    lib.pelica_attn_prof_read.restype = ctypes.c_int
    lib.pelica_attn_prof_read.argtypes = [ctypes.POINTER(ProfRecord), ctypes.c_int]
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != OK:
        msg = load_library().pelica_attn_last_error().decode(errors="replace")
        raise AttnError(rc, msg)


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream_ptr(stream) -> Optional[int]:
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


def make_desc(n_head: int, n_kv: int, hd: int, *, n_seq: int = 1, q_tokens: int = 1, kv_len: int,
              seq_kv_len=None, seq_kv_offset=None, kv_row_stride: int = 0, window: int = 0,
              ring_cap: int = 0, scale: Optional[float] = None, flags: int = 0, q_token_stride: int = 0,
              out_token_stride: int = 0) -> AttnDesc:
    d = AttnDesc()
    d.n_head, d.n_kv, d.hd = n_head, n_kv, hd
    d.n_seq, d.q_tokens, d.kv_len = n_seq, q_tokens, kv_len
    d.seq_kv_len = _ptr(seq_kv_len)
    d.seq_kv_offset = _ptr(seq_kv_offset)
    d.kv_row_stride = kv_row_stride
    d.window, d.ring_cap = window, ring_cap
    d.scale = 0.0 if scale is None else float(scale)
    d.flags = flags
    d.q_token_stride, d.out_token_stride = q_token_stride, out_token_stride
    return d


def token_stride(t) -> int:
    """The descriptor's token stride for a [n_seq, T, n_head, hd] tensor:
    0 when it is contiguous, else the elements between consecutive tokens
    (s * T + t) of a view whose heads are contiguous — e.g. the queries left
    in place in fused [q | k | v] rows.  Raises for other layouts."""
    if t.is_contiguous():
        return 0
    n_seq, T, n_head, hd = t.shape
    if t.stride(3) != 1 or (n_head > 1 and t.stride(2) != hd):
        raise AttnError(EINVAL, f"token rows need contiguous heads, got strides {tuple(t.stride())}")
    st = t.stride(1) if T > 1 else t.stride(0)
    if n_seq > 1 and T > 1 and t.stride(0) != T * st:
        raise AttnError(EINVAL, f"tokens of all sequences need one stride, got strides {tuple(t.stride())}")
    return st


def _validate_lens(seq_kv_len, seq_kv_offset):
    import torch

    if seq_kv_len is not None:
        assert seq_kv_len.dtype == torch.int32 and seq_kv_len.is_cuda and seq_kv_len.is_contiguous()
    if seq_kv_offset is not None:
        assert seq_kv_offset.dtype == torch.int64 and seq_kv_offset.is_cuda and seq_kv_offset.is_contiguous()


def workspace_bytes(desc: AttnDesc) -> int:
    n = load_library().pelica_attn_workspace_bytes(ctypes.byref(desc))
    if n == 0:
        msg = load_library().pelica_attn_last_error().decode(errors="replace")
        if msg:
            raise AttnError(EINVAL, msg)
    return n


def new_workspace(desc: AttnDesc, device="cuda"):
    """A workspace for decode calls with this descriptor (uninitialised:
    the calls need no particular contents)."""
    import torch

    return torch.empty(max(workspace_bytes(desc), 16), dtype=torch.uint8, device=device)


def decode(q, k, v, *, n_kv: int, kv_len: int, sinks=None, window: int = 0, ring_cap: int = 0,
           scale: Optional[float] = None, seq_kv_len=None, seq_kv_offset=None, kv_row_stride: int = 0,
           out=None, workspace=None, stream=None, split_only: bool = False):
    """Decode attention.  q: f32 [n_seq, q_tokens, n_head, hd] (CUDA);
    k, v: f16 cache rows (any shape, contiguous); returns f32 like q.
    split_only (measurement): run the key-split kernel only
    (PELICA_ATTN_FLAG_SPLIT_ONLY); the result is then not written."""
    import torch

    assert q.dtype == torch.float32 and q.dim() == 4 and q.is_cuda
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.is_contiguous() and v.is_contiguous()
    _validate_lens(seq_kv_len, seq_kv_offset)
    n_seq, T, n_head, hd = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    assert out.dtype == torch.float32 and out.shape == q.shape
    desc = make_desc(n_head, n_kv, hd, n_seq=n_seq, q_tokens=T, kv_len=kv_len, seq_kv_len=seq_kv_len,
                     seq_kv_offset=seq_kv_offset, kv_row_stride=kv_row_stride, window=window,
                     ring_cap=ring_cap, scale=scale, flags=FLAG_SPLIT_ONLY if split_only else 0,
                     q_token_stride=token_stride(q), out_token_stride=token_stride(out))
    lib = load_library()
    need = lib.pelica_attn_workspace_bytes(ctypes.byref(desc))
    if need == 0:
        msg = lib.pelica_attn_last_error().decode(errors="replace")
        if msg:
            raise AttnError(EINVAL, msg)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        # (the contents need no initialisation)
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    if sinks is not None:
        assert sinks.dtype == torch.float32 and sinks.is_cuda and sinks.numel() == n_head
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib.pelica_attn_decode(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v), _ptr(sinks), _ptr(out),
                                  _ptr(workspace), ws_bytes, _stream_ptr(stream)))
    return out


#: scratch bytes of the no-allocation decode (PELICA_ATTN_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 16 << 20


def decode_noalloc(q, k, v, *, n_kv: int, kv_len: int, sinks=None, window: int = 0, ring_cap: int = 0,
                   scale: Optional[float] = None, seq_kv_len=None, seq_kv_offset=None, kv_row_stride: int = 0,
                   out=None, stream=None):
    """``decode`` through pelica_attn_decode_noalloc: no workspace, the
    library's per-device static scratch (calls on one GPU must not overlap)."""
    import torch

    assert q.dtype == torch.float32 and q.dim() == 4 and q.is_cuda
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.is_contiguous() and v.is_contiguous()
    _validate_lens(seq_kv_len, seq_kv_offset)
    n_seq, T, n_head, hd = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    desc = make_desc(n_head, n_kv, hd, n_seq=n_seq, q_tokens=T, kv_len=kv_len, seq_kv_len=seq_kv_len,
                     seq_kv_offset=seq_kv_offset, kv_row_stride=kv_row_stride, window=window,
                     ring_cap=ring_cap, scale=scale, q_token_stride=token_stride(q),
                     out_token_stride=token_stride(out))
    if sinks is not None:
        assert sinks.dtype == torch.float32 and sinks.is_cuda and sinks.numel() == n_head
    _check(load_library().pelica_attn_decode_noalloc(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v), _ptr(sinks),
                                                     _ptr(out), _stream_ptr(stream)))
    return out


def decode_partials(q, k, v, *, n_kv: int, kv_len: int, window: int = 0, ring_cap: int = 0,
                    scale: Optional[float] = None, seq_kv_len=None, seq_kv_offset=None, kv_row_stride: int = 0,
                    parts=None, workspace=None, stream=None):
    """Partials of the keys this cache holds: f32 [n_seq, q_tokens, n_head,
    hd + 2] slots {M (natural log), L, O} in merge_dec's format, no sinks
    (they join in ``partials_merge`` with the CPU tier's slots)."""
    import torch

    assert q.dtype == torch.float32 and q.dim() == 4 and q.is_cuda
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.is_contiguous() and v.is_contiguous()
    _validate_lens(seq_kv_len, seq_kv_offset)
    n_seq, T, n_head, hd = q.shape
    desc = make_desc(n_head, n_kv, hd, n_seq=n_seq, q_tokens=T, kv_len=kv_len, seq_kv_len=seq_kv_len,
                     seq_kv_offset=seq_kv_offset, kv_row_stride=kv_row_stride, window=window,
                     ring_cap=ring_cap, scale=scale, q_token_stride=token_stride(q))
    lib = load_library()
    if parts is None:
        parts = torch.empty(n_seq, T, n_head, hd + 2, dtype=torch.float32, device=q.device)
    workspace, ws_bytes = _decode_workspace(lib, desc, workspace, q.device)
    _check(lib.pelica_attn_decode_partials(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v), _ptr(parts),
                                           _ptr(workspace), ws_bytes, _stream_ptr(stream)))
    return parts


def _decode_workspace(lib, desc, workspace, device):
    """(workspace, bytes): the caller's, or a new one when it is missing or
    too small for this descriptor's plan."""
    import torch

    need = lib.pelica_attn_workspace_bytes(ctypes.byref(desc))
    if need == 0:
        msg = lib.pelica_attn_last_error().decode(errors="replace")
        if msg:
            raise AttnError(EINVAL, msg)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    return workspace, 0 if workspace is None else workspace.numel() * workspace.element_size()


def decode_partials_range(q, k_rows, v_rows, *, n_kv: int, kv_len: int, key_begin: int, key_end: int,
                          window: int = 0, scale: Optional[float] = None, kv_row_stride: int = 0, parts=None,
                          workspace=None, stream=None):
    """Partials over key positions [key_begin, key_end) whose cache rows
    start at k_rows / v_rows (row 0 = position key_begin), one sequence:
    f32 [1, q_tokens, n_head, hd + 2] slots like ``decode_partials``.  Two
    such calls (VRAM rows, far rows) and ``partials_merge_batch`` are the
    reference's attn_s over resident and far keys."""
    import torch

    assert q.dtype == torch.float32 and q.dim() == 4 and q.is_cuda and q.shape[0] == 1
    assert k_rows.dtype == v_rows.dtype == torch.float16 and k_rows.is_contiguous() and v_rows.is_contiguous()
    n_seq, T, n_head, hd = q.shape
    desc = make_desc(n_head, n_kv, hd, n_seq=1, q_tokens=T, kv_len=kv_len, kv_row_stride=kv_row_stride,
                     window=window, scale=scale, q_token_stride=token_stride(q))
    lib = load_library()
    if parts is None:
        parts = torch.empty(1, T, n_head, hd + 2, dtype=torch.float32, device=q.device)
    workspace, ws_bytes = _decode_workspace(lib, desc, workspace, q.device)
    _check(lib.pelica_attn_decode_partials_range(ctypes.byref(desc), _ptr(q), _ptr(k_rows), _ptr(v_rows),
                                                 key_begin, key_end, _ptr(parts), _ptr(workspace), ws_bytes,
                                                 _stream_ptr(stream)))
    return parts


def qkv_rope_cache(q, k, v, k_cache, v_cache, *, n_kv: int, kv_len: int, table=None, rot: int = 0,
                   neox: bool = True, table_split: int = 0, q_norm=None, k_norm=None, eps: float = 1e-6,
                   seq_kv_len=None, seq_kv_offset=None, ring_cap: int = 0, kv_row_stride: int = 0,
                   token_stride: int = 0, n_seq: Optional[int] = None, q_tokens: Optional[int] = None,
                   n_head: Optional[int] = None, hd: Optional[int] = None, stream=None):
    """The step before attention (qk_dec / ROPE_KV_T): per-head RMS norm of
    q and k (when q_norm / k_norm are given), rope on q and k (table: f32
    [rows, rot/2, 2] cos/sin), q rotated in place, k and v rows into the f16
    caches.  q: f32 [n_seq, T, n_head, hd], k, v: f32 [n_seq, T, n_kv, hd]
    (or views into one fused buffer with ``token_stride``; then pass the
    shape keywords).  Returns q."""
    import torch

    if n_seq is None:
        n_seq, q_tokens, n_head, hd = q.shape
    assert q.dtype == k.dtype == v.dtype == torch.float32 and q.is_cuda
    assert k_cache.dtype == v_cache.dtype == torch.float16
    _validate_lens(seq_kv_len, seq_kv_offset)
    desc = make_desc(n_head, n_kv, hd, n_seq=n_seq, q_tokens=q_tokens, kv_len=kv_len, seq_kv_len=seq_kv_len,
                     seq_kv_offset=seq_kv_offset, kv_row_stride=kv_row_stride, ring_cap=ring_cap)
    rp = None
    if table is not None:
        assert table.dtype == torch.float32 and table.is_cuda and table.is_contiguous()
        rot = rot or hd
        rp = Rope(rot, 1 if neox else 0, table_split, table.shape[0], table.data_ptr())
    lib = load_library()
    _check(lib.pelica_attn_qkv_rope_cache(ctypes.byref(desc), None if rp is None else ctypes.byref(rp), _ptr(q),
                                          _ptr(k), _ptr(v), token_stride, _ptr(q_norm), _ptr(k_norm), eps,
                                          _ptr(k_cache), _ptr(v_cache), _stream_ptr(stream)))
    return q


def prefill(q, k, v, *, n_kv: int, kv_len: Optional[int] = None, sinks=None, window: int = 0,
            ring_cap: int = 0, scale: Optional[float] = None, seq_kv_len=None, seq_kv_offset=None,
            kv_row_stride: int = 0, out=None, stream=None):
    """Prompt attention.  q: f16 (pelica_attn_prefill) or f32
    (pelica_attn_prefill_f32) [n_seq, T, n_head, hd], contiguous or token
    rows of a wider buffer; k, v: f16 cache rows; kv_len defaults to T (a
    prompt that starts the cache).  Returns q's dtype (or fills ``out``, which
    may be a strided view too)."""
    import torch

    assert q.dtype in (torch.float16, torch.float32) and q.dim() == 4 and q.is_cuda
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.is_contiguous() and v.is_contiguous()
    _validate_lens(seq_kv_len, seq_kv_offset)
    n_seq, T, n_head, hd = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    assert out.dtype == q.dtype and out.shape == q.shape
    desc = make_desc(n_head, n_kv, hd, n_seq=n_seq, q_tokens=T, kv_len=T if kv_len is None else kv_len,
                     seq_kv_len=seq_kv_len, seq_kv_offset=seq_kv_offset, kv_row_stride=kv_row_stride,
                     window=window, ring_cap=ring_cap, scale=scale, q_token_stride=token_stride(q),
                     out_token_stride=token_stride(out))
    if sinks is not None:
        assert sinks.dtype == torch.float32 and sinks.is_cuda and sinks.numel() == n_head
    lib = load_library()
    fn = lib.pelica_attn_prefill if q.dtype == torch.float16 else lib.pelica_attn_prefill_f32
    _check(fn(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v), _ptr(sinks), _ptr(out), _stream_ptr(stream)))
    return out


def mla(q, latent, *, kv_len: int, scale: Optional[float] = None, seq_kv_len=None, seq_kv_offset=None,
        kv_row_stride: int = 0, out=None, workspace=None, stream=None):
    """MLA latent attention: q f32 [n_seq, T, n_head, 512] (absorbed
    queries), latent f16 cache rows of 512 (keys = values); causal.
    Returns f32 like q."""
    import torch

    assert q.dtype == torch.float32 and q.dim() == 4 and q.is_cuda and q.shape[-1] == 512
    assert latent.dtype == torch.float16 and latent.is_contiguous()
    _validate_lens(seq_kv_len, seq_kv_offset)
    n_seq, T, n_head, hd = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    desc = make_desc(n_head, 1, hd, n_seq=n_seq, q_tokens=T, kv_len=kv_len, seq_kv_len=seq_kv_len,
                     seq_kv_offset=seq_kv_offset, kv_row_stride=kv_row_stride, scale=scale,
                     q_token_stride=token_stride(q), out_token_stride=token_stride(out))
    lib = load_library()
    need = lib.pelica_attn_mla_workspace_bytes(ctypes.byref(desc))
    if need == 0:
        msg = lib.pelica_attn_last_error().decode(errors="replace")
        if msg:
            raise AttnError(EINVAL, msg)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib.pelica_attn_mla(ctypes.byref(desc), _ptr(q), _ptr(latent), _ptr(out), _ptr(workspace), ws_bytes,
                               _stream_ptr(stream)))
    return out


def prefill_round(q, k_rows, v_rows, state, *, n_kv: int, kv_len: int, key_begin: int, key_end: int,
                  first: bool, sinks=None, window: int = 0, scale: Optional[float] = None,
                  kv_row_stride: int = 0, out=None, stream=None):
    """Prompt attention over one round of keys [key_begin, key_end) (rows of
    those positions in k_rows / v_rows), folded into ``state`` (f32 [1, T,
    n_head, hd + 2]: M natural-log, L, O); ``out`` (q's dtype: f16, or f32
    through pelica_attn_prefill_round_f32) gets the output so far when
    given.  Returns out (or None)."""
    import torch

    assert q.dtype in (torch.float16, torch.float32) and q.dim() == 4 and q.is_cuda
    assert k_rows.dtype == v_rows.dtype == torch.float16 and k_rows.is_contiguous() and v_rows.is_contiguous()
    n_seq, T, n_head, hd = q.shape
    assert state.dtype == torch.float32 and state.numel() == n_seq * T * n_head * (hd + 2)
    assert out is None or (out.dtype == q.dtype and out.shape == q.shape)
    desc = make_desc(n_head, n_kv, hd, n_seq=n_seq, q_tokens=T, kv_len=kv_len, kv_row_stride=kv_row_stride,
                     window=window, scale=scale, q_token_stride=token_stride(q),
                     out_token_stride=0 if out is None else token_stride(out))
    lib = load_library()
    fn = lib.pelica_attn_prefill_round if q.dtype == torch.float16 else lib.pelica_attn_prefill_round_f32
    _check(fn(ctypes.byref(desc), _ptr(q), _ptr(k_rows), _ptr(v_rows), key_begin, key_end, _ptr(sinks), _ptr(state),
              1 if first else 0, _ptr(out), _stream_ptr(stream)))
    return out


def partials_merge(parts, *, n_head: int, hd: int, sinks=None, out=None, stream=None):
    """Combine partial slots [n_parts, n_head, hd + 2] (max, sum, O) in slot
    order with optional sinks into f32 [n_head, hd]."""
    import torch

    assert parts.dtype == torch.float32 and parts.is_cuda and parts.is_contiguous()
    n_parts = parts.numel() // (n_head * (hd + 2))
    assert n_parts * n_head * (hd + 2) == parts.numel()
    if out is None:
        out = torch.empty(n_head, hd, dtype=torch.float32, device=parts.device)
    lib = load_library()
    _check(lib.pelica_attn_partials_merge(n_head, hd, n_parts, _ptr(parts), _ptr(sinks), _ptr(out),
                                          _stream_ptr(stream)))
    return out


def partials_merge_batch(parts, *, sinks=None, out=None, stream=None):
    """Combine partial slots [n_parts, n_tokens, n_head, hd + 2] per (token,
    head) in slot order with optional sinks into f32 [n_tokens, n_head, hd]
    (ATTN_M over all the pass's tokens)."""
    import torch

    assert parts.dtype == torch.float32 and parts.is_cuda and parts.is_contiguous() and parts.dim() == 4
    n_parts, n_tok, n_head, hp = parts.shape
    hd = hp - 2
    if out is None:
        out = torch.empty(n_tok, n_head, hd, dtype=torch.float32, device=parts.device)
    assert out.dtype == torch.float32 and out.is_contiguous() and out.numel() == n_tok * n_head * hd
    if sinks is not None:
        assert sinks.dtype == torch.float32 and sinks.is_cuda and sinks.numel() == n_head
    lib = load_library()
    _check(lib.pelica_attn_partials_merge_batch(n_tok, n_head, hd, n_parts, _ptr(parts), _ptr(sinks), _ptr(out),
                                                _stream_ptr(stream)))
    return out


def reload_tuning() -> None:
    """Re-read the planner's PELICA_ATTN_* environment switches (they are
    otherwise read once per process)."""
    _check(load_library().pelica_attn_reload_tuning())


def default_scale(hd: int) -> float:
    return 1.0 / math.sqrt(hd)


def prof_enable(on: bool = True) -> None:
    """Per-kernel GPU timing of the library's launches (HIP events)."""
    _check(load_library().pelica_attn_prof_enable(1 if on else 0))


def prof_read(max_records: int = 1 << 14) -> list:
    """[(kernel name, ms), ...] of the launches timed since the last read."""
    buf = (ProfRecord * max_records)()
    n = load_library().pelica_attn_prof_read(buf, max_records)
    if n < 0:
        _check(n)
    return [(PROF_KERNELS.get(buf[i].kernel, str(buf[i].kernel)), buf[i].ms) for i in range(n)]
