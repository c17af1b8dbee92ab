"""Pins of the CPU oracle of the step before attention (oracle/qkv_oracle.c:
qk_dec, src/moe_kernels.rs:304-378; ROPE_KV_T, src/oss_batch.rs:113-170),
each against something the mathematics fixes rather than the same formula:
rotation as complex multiplication, norm preservation, position 0 as the
identity, angle addition of the two-level table, RMS of a normalised head,
f16 rounding against numpy's, and the cache row addressing."""
import numpy as np
import pytest

from oracle import oracle as orc


def _inputs(n_seq, T, n_head, n_kv, hd, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_seq, T, n_head, hd)).astype(np.float32)
    k = rng.standard_normal((n_seq, T, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n_seq, T, n_kv, hd)).astype(np.float32)
    return q, k, v


def _f16(bits):
    return bits.view(np.float16).astype(np.float64)


def _rope_complex(x, pos, rot, neox, base=10000.0):
    """fp64 rotation as complex multiplication by e^{i theta_j}."""
    x = x.astype(np.float64).copy()
    half = rot // 2
    th = pos * base ** (-(2.0 * np.arange(half)) / rot)
    if neox:
        z = x[..., :half] + 1j * x[..., half:rot]
    else:
        z = x[..., 0:rot:2] + 1j * x[..., 1:rot:2]
    z = z * np.exp(1j * th)
    if neox:
        x[..., :half], x[..., half:rot] = z.real, z.imag
    else:
        x[..., 0:rot:2], x[..., 1:rot:2] = z.real, z.imag
    return x


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("hd,rot", [(64, 64), (128, 128), (64, 32)])
def test_rope_is_complex_rotation(neox, hd, rot):
    L, T = 300, 3
    q, k, v = _inputs(1, T, 4, 2, hd, seed=hd + rot)
    table = orc.rope_table(L, rot)
    qo, kc, vc = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=L, table=table, rot=rot, neox=neox)
    for t in range(T):
        pos = L - T + t
        want = _rope_complex(q[0, t], pos, rot, neox)
        assert np.abs(qo[0, t] - want).max() < 2e-5
        assert np.abs(_f16(kc[pos].reshape(2, hd)) - _rope_complex(k[0, t], pos, rot, neox)).max() < 4e-3
        # dims past rot untouched
        assert np.array_equal(qo[0, t][..., rot:], q[0, t][..., rot:])


def test_position_zero_is_identity_and_norms_are_kept():
    q, k, v = _inputs(1, 1, 8, 2, 64, seed=3)
    table = orc.rope_table(1, 64)
    qo, kc, _ = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=1, table=table)
    assert np.array_equal(qo, q)
    assert np.array_equal(kc[0], k[0, 0].reshape(-1).astype(np.float16).view(np.uint16))
    table = orc.rope_table(5000, 64)
    q, k, v = _inputs(1, 1, 8, 2, 64, seed=4)
    qo, _, _ = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=5000, table=table)
    half = 32
    n_in = np.hypot(q[..., :half].astype(np.float64), q[..., half:])
    n_out = np.hypot(qo[..., :half].astype(np.float64), qo[..., half:])
    assert np.abs(n_in - n_out).max() < 1e-5


def test_two_level_table_is_angle_addition():
    L = 70000
    q, k, v = _inputs(1, 2, 4, 2, 128, seed=5)
    direct = orc.rope_table(L, 128)
    split, n_hi = orc.rope_table(L, 128, split=True)
    a, ka, _ = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=L, table=direct)
    b, kb, _ = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=L, table=split, table_split=n_hi)
    assert np.abs(a - b).max() < 5e-5
    assert np.abs(_f16(ka[L - 2:]) - _f16(kb[L - 2:])).max() < 4e-3


def test_rms_norm():
    q, k, v = _inputs(1, 2, 4, 2, 128, seed=6)
    ones = np.ones(128, np.float32)
    qo, kc, vc = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=2, q_norm=ones, k_norm=ones, eps=0.0)
    rms = np.sqrt(np.mean(qo.astype(np.float64) ** 2, axis=-1))
    assert np.abs(rms - 1).max() < 1e-6
    w = np.random.default_rng(7).standard_normal(128).astype(np.float32)
    qo, _, _ = orc.qk_norm_rope_cache(q, k, v, n_kv=2, kv_len=2, q_norm=w, eps=1e-6)
    x = q.astype(np.float64)
    want = x / np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + 1e-6) * w
    assert np.abs(qo - want).max() < 1e-5
    # v rows are never normalised: exact f16 rounding of the input
    assert np.array_equal(vc[:2].reshape(2, 2, 128), v[0].astype(np.float16).view(np.uint16))
    # a zero head stays zero (eps keeps the scale finite)
    z = np.zeros_like(q)
    qo, _, _ = orc.qk_norm_rope_cache(z, k, v, n_kv=2, kv_len=2, q_norm=w, eps=1e-6)
    assert not np.any(qo)


def test_cache_rows_linear_ring_ragged_and_stride():
    n_seq, T, hd, n_kv = 3, 4, 64, 2
    q, k, v = _inputs(n_seq, T, 4, n_kv, hd, seed=8)
    lens = np.array([4, 9, 13], np.int32)
    offs = np.array([0, 20, 40], np.int64)
    stride = n_kv * hd + 16
    _, kc, vc = orc.qk_norm_rope_cache(q, k, v, n_kv=n_kv, kv_len=13, seq_kv_len=lens, seq_kv_offset=offs,
                                       kv_row_stride=stride, cache_rows=60)
    written = set()
    for s in range(n_seq):
        for t in range(T):
            row = offs[s] + lens[s] - T + t
            written.add(row)
            assert np.array_equal(vc[row, :n_kv * hd], v[s, t].reshape(-1).astype(np.float16).view(np.uint16))
            assert np.array_equal(kc[row, :n_kv * hd], k[s, t].reshape(-1).astype(np.float16).view(np.uint16))
    assert not np.any(kc[:, n_kv * hd:]) and not np.any(vc[:, n_kv * hd:])
    assert not any(np.any(vc[r]) for r in range(60) if r not in written)
    # ring: position p in row p % cap
    cap, L = 8, 30
    _, kc, vc = orc.qk_norm_rope_cache(q[:1], k[:1], v[:1], n_kv=n_kv, kv_len=L, ring_cap=cap)
    for t in range(T):
        assert np.array_equal(vc[(L - T + t) % cap], v[0, t].reshape(-1).astype(np.float16).view(np.uint16))
