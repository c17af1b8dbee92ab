"""The benchmark shapes as seeded synthetic inputs.

Every tensor comes from ``torch.Generator`` seeded per config, drawn on the
requested device, so tests and the benchmark see the same kind of data:
Q ~ N(0,1) f32 (f16 for prefill), K/V ~ N(0,1)*0.5 in f16, sinks ~ N(0,1).
Config 2 RMS-normalises Q and K per head (unit gain, eps 1e-6) before K is
rounded to f16 and leaves V at N(0,1).
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Optional

import torch


@dataclass(frozen=True)
class AttnConfig:
    name: str
    kind: str  # "decode" | "prefill"
    n_head: int
    n_kv: int
    hd: int
    kv_len: int  # keys per sequence (max for ragged batches)
    q_tokens: int = 1
    n_seq: int = 1
    window: int = 0
    sinks: bool = False
    kv_scale: float = 0.5
    rms_norm_qk: bool = False
    ragged: Optional[tuple] = None  # (lo, hi) inclusive key-length range per sequence
    seed: int = 0
    note: str = field(default="", compare=False)

    def scaled(self, **kw) -> "AttnConfig":
        return replace(self, **kw)


C1 = AttnConfig("c1_olmoe_decode", "decode", 16, 16, 128, 2048, seed=1,
                note="OLMoE-1B-7B decode: 16q/16kv MHA, hd128, ctx 2048")
C2 = AttnConfig("c2_qwen3_gqa_decode", "decode", 32, 4, 128, 8192, kv_scale=1.0, rms_norm_qk=True, seed=2,
                note="Qwen3-30B-A3B decode: 32q/4kv, hd128, ctx 8192, RMS-normed q/k")
C3_FULL = AttnConfig("c3_gptoss_decode_full", "decode", 64, 8, 64, 32768, sinks=True, seed=3,
                     note="gpt-oss-20b decode, full layer: 64q/8kv, hd64, ctx 32768, sinks")
C3_SWA = C3_FULL.scaled(name="c3_gptoss_decode_swa128", window=128,
                        note="gpt-oss-20b decode, sliding-window-128 layer")
C4_FULL = AttnConfig("c4_gptoss_prefill_full", "prefill", 64, 8, 64, 4096, q_tokens=4096, sinks=True, seed=4,
                     note="gpt-oss-20b causal prefill, 4096 tokens, full causal")
C4_SWA = C4_FULL.scaled(name="c4_gptoss_prefill_swa128", window=128,
                        note="gpt-oss-20b causal prefill, 4096 tokens, window 128")
C5 = AttnConfig("c5_qwen3_spec_decode", "decode", 32, 4, 128, 16384, q_tokens=4, n_seq=32, ragged=(512, 16384),
                seed=5, note="Qwen3 batched speculative verify: 32 seqs x 4 drafts, ragged 512..16384")

CONFIGS = {c.name: c for c in (C1, C2, C3_FULL, C3_SWA, C4_FULL, C4_SWA, C5)}


def _rms_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


@dataclass
class AttnInputs:
    cfg: AttnConfig
    q: torch.Tensor           # [n_seq, T, n_head, hd] f32 (decode) / f16 (prefill)
    k: torch.Tensor           # [rows, n_kv, hd] f16
    v: torch.Tensor
    sinks: Optional[torch.Tensor]
    seq_len: torch.Tensor     # [n_seq] int32 (same device)
    seq_off: torch.Tensor     # [n_seq] int64 first cache row
    kv_len: int               # max keys per sequence

    @property
    def ragged(self) -> bool:
        return self.cfg.ragged is not None


def seq_lengths(cfg: AttnConfig) -> list:
    if cfg.ragged is None:
        return [cfg.kv_len] * cfg.n_seq
    g = torch.Generator().manual_seed(cfg.seed * 7919 + 17)
    lo, hi = cfg.ragged
    return torch.randint(lo, hi + 1, (cfg.n_seq,), generator=g).tolist()


def make_inputs(cfg: AttnConfig, device="cpu") -> AttnInputs:
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    lens = seq_lengths(cfg)
    rows = sum(lens)
    offs = [0]
    for n in lens[:-1]:
        offs.append(offs[-1] + n)
    T = cfg.q_tokens
    q = torch.randn(cfg.n_seq, T, cfg.n_head, cfg.hd, generator=g, device=dev, dtype=torch.float32)
    k = torch.randn(rows, cfg.n_kv, cfg.hd, generator=g, device=dev, dtype=torch.float32)
    v = torch.randn(rows, cfg.n_kv, cfg.hd, generator=g, device=dev, dtype=torch.float32)
    if cfg.rms_norm_qk:
        q = _rms_norm(q)
        k = _rms_norm(k)
    else:
        k = k * cfg.kv_scale
    v = v * cfg.kv_scale
    if cfg.kind == "prefill":
        q = (q * cfg.kv_scale).to(torch.float16)
    sinks = torch.randn(cfg.n_head, generator=g, device=dev, dtype=torch.float32) if cfg.sinks else None
    return AttnInputs(cfg, q.contiguous(), k.to(torch.float16).contiguous(), v.to(torch.float16).contiguous(),
                      sinks, torch.tensor(lens, dtype=torch.int32, device=dev),
                      torch.tensor(offs, dtype=torch.int64, device=dev), max(lens))


def kv_bytes(cfg: AttnConfig, lens=None) -> int:
    """Algorithmic bytes of one decode call: K and V once per kv head, Q in, O out."""
    lens = seq_lengths(cfg) if lens is None else lens
    if cfg.window:
        keys = [min(n, cfg.window + cfg.q_tokens - 1) for n in lens]
    else:
        keys = lens
    kv = sum(keys) * cfg.n_kv * cfg.hd * 2 * 2
    qo = 2 * cfg.n_seq * cfg.q_tokens * cfg.n_head * cfg.hd * (4 if cfg.kind == "decode" else 2)
    return kv + qo


def attn_flops(cfg: AttnConfig, lens=None) -> int:
    """4 * hd * (visible query-key pairs), causal pairs including the diagonal."""
    lens = seq_lengths(cfg) if lens is None else lens
    pairs = 0
    for n in lens:
        for t in range(cfg.q_tokens):
            pos = n - cfg.q_tokens + t
            lo = max(0, pos + 1 - cfg.window) if cfg.window else 0
            pairs += pos - lo + 1
    return 4 * cfg.hd * cfg.n_head * pairs
