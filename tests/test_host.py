"""Host-side checks that need no GPU: the C ABI library loads and exports what
include/pelica_attn.h declares, descriptors are validated with the documented
status codes, and the workload byte/flop counts match BASELINE's figures."""
import ctypes
import os
import re

import pytest

from pelica_amd import attn
from pelica_amd import workloads as wl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "pelica_attn.h")).read()
    return sorted(set(re.findall(r"\b(pelica_attn_\w+)\s*\(", text)))


def test_header_matches_binding_list():
    assert header_functions() == sorted(attn.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = attn.load_library()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.pelica_attn_version() == 2


def _desc(**kw):
    base = dict(n_head=64, n_kv=8, hd=64, n_seq=1, q_tokens=1, kv_len=32768)
    base.update(kw)
    n_head, n_kv, hd = base.pop("n_head"), base.pop("n_kv"), base.pop("hd")
    return attn.make_desc(n_head, n_kv, hd, **base)


def test_workspace_sizes():
    # gpt-oss decode: 8 kv heads x 8 rows x splits x (2 + 64) floats
    n = attn.workspace_bytes(_desc())
    assert n > 0 and n % 4 == 0
    # a single split needs no workspace
    assert attn.workspace_bytes(_desc(kv_len=64, n_kv=64, n_head=64)) == 0


def test_split_only_flag_is_decode_only():
    lib = attn.load_library()
    d = _desc()
    base = attn.workspace_bytes(d)
    d.flags = attn.FLAG_SPLIT_ONLY
    # decode accepts it (same workspace), unknown bits are rejected
    assert lib.pelica_attn_workspace_bytes(ctypes.byref(d)) == base
    d.flags = 2
    assert lib.pelica_attn_workspace_bytes(ctypes.byref(d)) == 0
    assert "flags" in lib.pelica_attn_last_error().decode()
    # every other entry point rejects it before touching the GPU
    d.flags = attn.FLAG_SPLIT_ONLY
    rc = lib.pelica_attn_prefill(ctypes.byref(d), 16, 16, 16, None, 16, None)
    assert rc == attn.EINVAL and "flags" in lib.pelica_attn_last_error().decode()
    rc = lib.pelica_attn_decode_partials(ctypes.byref(d), 16, 16, 16, 16, None, 0, None)
    assert rc == attn.EINVAL and "flags" in lib.pelica_attn_last_error().decode()


@pytest.mark.parametrize("kw,code", [
    (dict(hd=96), attn.EUNSUPPORTED),
    (dict(n_head=60), attn.EINVAL),
    (dict(kv_len=0), attn.EINVAL),
    (dict(q_tokens=4, kv_len=3), attn.EINVAL),
    (dict(window=-1), attn.EINVAL),
    (dict(ring_cap=100, window=0, kv_len=1000), attn.EINVAL),
    (dict(kv_row_stride=12), attn.EINVAL),
])
def test_invalid_descriptors(kw, code):
    lib = attn.load_library()
    d = _desc(**kw)
    assert lib.pelica_attn_workspace_bytes(ctypes.byref(d)) == 0
    msg = lib.pelica_attn_last_error().decode()
    assert msg, kw
    # the decode entry point reports the same status before touching the GPU
    rc = lib.pelica_attn_decode(ctypes.byref(d), 16, 16, 16, None, 16, None, 0, None)
    assert rc == code, (kw, rc, lib.pelica_attn_last_error())


def test_null_and_misaligned_pointers():
    lib = attn.load_library()
    d = _desc(kv_len=64, n_kv=64)
    assert lib.pelica_attn_decode(ctypes.byref(d), None, 16, 16, None, 16, None, 0, None) == attn.EINVAL
    assert lib.pelica_attn_decode(ctypes.byref(d), 8, 16, 16, None, 16, None, 0, None) == attn.EINVAL
    assert b"aligned" in lib.pelica_attn_last_error()
    assert lib.pelica_attn_prefill(ctypes.byref(d), 16, None, 16, None, 16, None) == attn.EINVAL
    assert lib.pelica_attn_partials_merge(0, 64, 1, 16, None, 16, None) == attn.EINVAL


def test_workspace_too_small_is_reported():
    lib = attn.load_library()
    d = _desc()
    need = lib.pelica_attn_workspace_bytes(ctypes.byref(d))
    rc = lib.pelica_attn_decode(ctypes.byref(d), 16, 16, 16, None, 16, 16, need - 16, None)
    assert rc == attn.EWORKSPACE


def test_baseline_work_counts():
    # the work of each benchmark shape: K/V bytes of a decode call, flops of a
    # prefill (4 hd per visible query-key pair, causal pairs with the diagonal)
    assert wl.kv_bytes(wl.C1) == 16_793_600
    assert wl.kv_bytes(wl.C2) == 16_809_984
    assert wl.kv_bytes(wl.C3_FULL) == 67_141_632
    assert wl.kv_bytes(wl.C3_SWA) == 294_912
    assert wl.attn_flops(wl.C4_FULL) == 137_472_507_904
    assert wl.attn_flops(wl.C4_SWA) == 8_456_765_440
    lens = wl.seq_lengths(wl.C5)
    assert len(lens) == 32 and all(512 <= n <= 16384 for n in lens)
    assert wl.kv_bytes(wl.C5) == sum(lens) * 2048 + 2 * 2_097_152


def test_shape_mirror():
    sh = attn.Shape(hd=128, n_kv=4, hpk=8)
    assert sh.row() == 512 and sh.n_head == 32


def test_small_inputs_are_deterministic():
    a = wl.make_inputs(wl.C3_FULL.scaled(kv_len=256))
    b = wl.make_inputs(wl.C3_FULL.scaled(kv_len=256))
    assert (a.q == b.q).all() and (a.k == b.k).all() and (a.sinks == b.sinks).all()


def test_partials_merge_batch_arguments():
    lib = attn.load_library()
    f = lib.pelica_attn_partials_merge_batch
    assert f(0, 8, 64, 1, 16, None, 16, None) == attn.EINVAL       # no tokens
    assert f(2, 8, 63, 1, 16, None, 16, None) == attn.EINVAL       # odd hd
    assert f(2, 8, 2048, 1, 16, None, 16, None) == attn.EINVAL     # hd too large
    assert f(2, 8, 64, 0, 16, None, 16, None) == attn.EINVAL       # no slots
    assert f(2, 8, 64, 1, None, None, 16, None) == attn.EINVAL     # no parts
    assert f(2, 8, 64, 1, 12, None, 16, None) == attn.EINVAL       # misaligned
    assert b"aligned" in lib.pelica_attn_last_error()


def test_planner_switches_are_read_once():
    # the workspace size is fixed by the environment at the first plan
    import subprocess
    import sys

    code = ("import ctypes, os\n"
            "from pelica_amd import attn\n"
            "d = attn.make_desc(64, 8, 64, kv_len=32768)\n"
            "a = attn.workspace_bytes(d)\n"
            "os.environ['PELICA_ATTN_SPLIT_BLOCKS'] = '1'\n"
            "b = attn.workspace_bytes(d)\n"
            "print(a == b and a > 0)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.stdout.strip() == "True", r.stderr


def test_noalloc_decode_rejects_oversize_pass():
    # a pass whose partials exceed the static scratch is refused before any
    # GPU call (a 64-sequence stream-K verify batch at 64K keys: ~77 MB)
    d = _desc(n_head=32, n_kv=4, hd=128, n_seq=64, q_tokens=4, kv_len=1 << 16)
    d.seq_kv_len, d.seq_kv_offset = 256, 512   # device tables (not read by the planner)
    need = attn.workspace_bytes(d)
    assert need > attn.NOALLOC_SCRATCH_BYTES
    lib = attn.load_library()
    rc = lib.pelica_attn_decode_noalloc(ctypes.byref(d), 16, 16, 16, None, 16, None)
    assert rc == attn.EWORKSPACE and b"scratch" in lib.pelica_attn_last_error()
    d.flags = attn.FLAG_SPLIT_ONLY
    assert lib.pelica_attn_decode_noalloc(ctypes.byref(d), 16, 16, 16, None, 16, None) == attn.EINVAL


def test_noalloc_scratch_size_matches_header():
    text = open(os.path.join(ROOT, "include", "pelica_attn.h")).read()
    m = re.search(r"#define PELICA_ATTN_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == attn.NOALLOC_SCRATCH_BYTES


def test_package_exports_every_public_binding():
    """Every public function of the binding module is re-exported by the package."""
    import inspect

    import pelica_amd

    public = {n for n, f in inspect.getmembers(attn, inspect.isfunction)
              if not n.startswith("_") and f.__module__ == attn.__name__}
    assert public <= set(pelica_amd.__all__), sorted(public - set(pelica_amd.__all__))
    for n in pelica_amd.__all__:
        assert getattr(pelica_amd, n) is getattr(attn, n)


def test_descriptor_layout_matches_the_c_header(tmp_path):
    # the ctypes mirror and the C struct agree field by field (gcc on the header)
    src = tmp_path / "layout.c"
    fields = [f for f, _ in attn.AttnDesc._fields_]
    body = "".join(f'printf("{f} %zu\\n", offsetof(PelicaAttnDesc, {f}));\n' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "pelica_attn.h"\n'
                   'int main(void) {\n' + body + 'printf("size %zu\\n", sizeof(PelicaAttnDesc));\nreturn 0;\n}\n')
    exe = tmp_path / "layout"
    import subprocess

    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), "-o", str(exe), str(src)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    for f in fields:
        assert int(out[f]) == getattr(attn.AttnDesc, f).offset, f
    assert int(out["size"]) == ctypes.sizeof(attn.AttnDesc)


@pytest.mark.parametrize("field,value", [
    ("q_token_stride", 64 * 64 - 4),     # below a token's heads
    ("q_token_stride", 64 * 64 + 2),     # rows no longer 16-byte aligned
    ("q_token_stride", 1 << 20),         # past the kernels' 32-bit block offsets
    ("out_token_stride", 64 * 64 + 1),
])
def test_token_strides_are_validated(field, value):
    lib = attn.load_library()
    d = _desc(q_tokens=4)
    setattr(d, field, value)
    for rc in (lib.pelica_attn_decode(ctypes.byref(d), 16, 16, 16, None, 16, None, 0, None),
               lib.pelica_attn_decode_partials(ctypes.byref(d), 16, 16, 16, 16, None, 0, None),
               lib.pelica_attn_prefill_f32(ctypes.byref(d), 16, 16, 16, None, 16, None)):
        assert rc == attn.EINVAL and field.encode() in lib.pelica_attn_last_error()
    # f16 prefill rows: a multiple of 8 values (4 is enough for f32 rows)
    d = _desc(q_tokens=4)
    setattr(d, field, 64 * 64 + 4)
    assert lib.pelica_attn_prefill(ctypes.byref(d), 16, 16, 16, None, 16, None) == attn.EINVAL
    assert field.encode() in lib.pelica_attn_last_error()


def test_token_stride_of_views():
    import torch

    rows = torch.zeros(2, 3, (64 + 2 * 8) * 64)
    q = rows[..., :64 * 64].view(2, 3, 64, 64)
    assert attn.token_stride(q) == (64 + 2 * 8) * 64
    assert attn.token_stride(torch.zeros(2, 3, 64, 64)) == 0
    assert attn.token_stride(rows[:, :1, :64 * 64].view(2, 1, 64, 64)) == (64 + 2 * 8) * 64 * 3
    with pytest.raises(attn.AttnError):
        attn.token_stride(torch.zeros(2, 3, 64, 128)[..., :64])


def test_key_range_arguments():
    lib = attn.load_library()
    f = lib.pelica_attn_decode_partials_range
    d = _desc(q_tokens=4, kv_len=20000)
    assert f(ctypes.byref(d), 16, 16, 16, 0, 0, 16, None, 0, None) == attn.EINVAL           # empty
    assert f(ctypes.byref(d), 16, 16, 16, 100, 20001, 16, None, 0, None) == attn.EINVAL     # past kv_len
    assert f(ctypes.byref(d), 16, 16, 16, -1, 50, 16, None, 0, None) == attn.EINVAL         # negative
    assert f(ctypes.byref(d), 16, 16, 16, 0, 50, None, None, 0, None) == attn.EINVAL        # no parts
    d2 = _desc(q_tokens=4, kv_len=20000, n_seq=2)
    assert f(ctypes.byref(d2), 16, 16, 16, 0, 50, 16, None, 0, None) == attn.EINVAL
    assert b"one sequence" in lib.pelica_attn_last_error()


def test_recorded_traffic_follows_the_kernel_sources(tmp_path, monkeypatch):
    # bench.py reports roofline.traffic from the committed counter summary
    # only while the kernel's sources hash as they did when it was measured
    import bench

    lines = [ln.split() for ln in open(bench.TRAFFIC_PROFILE).read().splitlines() if ln.startswith("traffic ")]
    assert {f[1] for f in lines} >= {"c3_gptoss_decode_full", "c4_gptoss_prefill_full"}
    for f in lines:
        assert len(f) == 4 and int(f[2]) > 0 and f[3].startswith("src=")
        got, note = bench.recorded_traffic(f[1])
        fresh = f[3] == "src=" + bench.sources_hash(bench.TRAFFIC_KERNELS[f[1]][1])
        assert (got == int(f[2])) == fresh, note
    stale = tmp_path / "t.md"
    stale.write_text("traffic c3_gptoss_decode_full 123 src=000000000000\n")
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", str(stale))
    assert bench.recorded_traffic("c3_gptoss_decode_full")[0] is None
