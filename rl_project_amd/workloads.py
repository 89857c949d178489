"""Seeded synthetic inputs of the sampler's benchmark workloads.

Each workload is one step of the sampling path on synthetic logits of the
shape and distribution stated for it (no model, no dataset).  Inputs are
generated on the CPU from ``torch.Generator().manual_seed(seed)`` so that the
same seed gives the same tensors on every machine, then moved to ``device``.

    plumbing_f32_4x512        B=4, V=512 fp32 N(0, 3^2); T .8, top-k 50,
                              top-p .9, penalty 1.1 over 32 uniform ids/row
    uniform_f32_64x32000      B=64, V=32000 fp32 N(0, 2^2) + 1% spikes of +8;
                              T .7, top-k 50, top-p .95, min-p .05, penalty
                              1.15 over 512 ids/row; 4 stop ids
    hetero_bf16_256x128256    B=256, V=128256 bf16 N(0, 2.5^2); per row
                              T~U[.1,1.5], top-k in {0,1,20,50,200},
                              top-p~U[.5,1], min-p in {0,.02,.1},
                              penalty~U[1,1.3] over 2048 Zipf(1.1) ids
    softcap_zipf_f32_512x262144  B=512, V=262144 fp32
                              -1.2 ln(rank) + N(0, .5^2), ranks permuted per
                              row; soft-cap 30, top-p .9, T 1
    spec_f32_32x5x128256      B=32 sequences x 5 drafts, V=128256 fp32;
                              target 2 Z1, draft 2(.8 Z1 + .6 Z2); T .8,
                              top-p .95 on both; drafts drawn from the draft
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

WORKLOADS = (
    "plumbing_f32_4x512",
    "uniform_f32_64x32000",
    "hetero_bf16_256x128256",
    "softcap_zipf_f32_512x262144",
    "spec_f32_32x5x128256",
)


@dataclass
class SampleWorkload:
    name: str
    logits: torch.Tensor                 # [B, V]
    temperature: torch.Tensor            # float32 [B]
    top_k: torch.Tensor                  # int32 [B] (0 = off)
    top_p: torch.Tensor                  # float32 [B] (1 = off)
    min_p: torch.Tensor                  # float32 [B] (0 = off)
    repetition_penalty: torch.Tensor     # float32 [B] (1 = off)
    history: Optional[torch.Tensor]      # int32 [B, H] or None
    stop_ids: Optional[torch.Tensor]     # int32 [S] or None
    uniforms: torch.Tensor               # float32 [B]
    softcap: float = 0.0

    @property
    def batch(self) -> int:
        return self.logits.size(0)

    @property
    def vocab(self) -> int:
        return self.logits.size(1)

    def kwargs(self) -> Dict[str, object]:
        """Keyword arguments of ``sample_tokens`` for this workload."""
        return dict(temperature=self.temperature, top_k=self.top_k, top_p=self.top_p, min_p=self.min_p,
                    repetition_penalty=self.repetition_penalty, history=self.history, stop_ids=self.stop_ids,
                    uniforms=self.uniforms, softcap=self.softcap)

    def algorithmic_bytes(self) -> int:
        """Compulsory HBM traffic of one step: logits once, history ids,
        24 B/row of parameters and uniform, 9 B/row of token + finished."""
        B, V = self.logits.shape
        hist = 0 if self.history is None else self.history.numel() * 4
        return B * V * self.logits.element_size() + hist + 24 * B + 9 * B

    def to(self, device) -> "SampleWorkload":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return SampleWorkload(self.name, mv(self.logits), mv(self.temperature), mv(self.top_k), mv(self.top_p),
                              mv(self.min_p), mv(self.repetition_penalty), mv(self.history), mv(self.stop_ids),
                              mv(self.uniforms), self.softcap)


@dataclass
class SpecWorkload:
    name: str
    target: torch.Tensor          # [B, K+1, V]
    draft: torch.Tensor           # [B, K, V]
    draft_ids: torch.Tensor       # int64 [B, K]
    u_accept: torch.Tensor        # float32 [B, K]
    u_resample: torch.Tensor      # float32 [B]
    temperature: float = 0.8
    top_p: float = 0.95
    extra: Dict[str, object] = field(default_factory=dict)
    top_k: int = 0                # 0 = off (the reference's default speculative filter is top-k 50)

    def algorithmic_bytes(self) -> int:
        B, K = self.draft_ids.shape
        return (self.target.numel() + self.draft.numel()) * self.target.element_size() + B * K * (8 + 4) + B * 4 \
            + B * 4 + B * (K + 1) * 8

    def to(self, device) -> "SpecWorkload":
        return SpecWorkload(self.name, self.target.to(device), self.draft.to(device), self.draft_ids.to(device),
                            self.u_accept.to(device), self.u_resample.to(device), self.temperature, self.top_p,
                            dict(self.extra), self.top_k)


def zipf_ids(g: torch.Generator, shape, V: int, s: float) -> torch.Tensor:
    """Finite Zipf(s) over ranks 1..V (CDF table + searchsorted); id = rank - 1."""
    ranks = torch.arange(1, V + 1, dtype=torch.float64)
    cdf = torch.cumsum(ranks.pow(-s), 0)
    cdf = cdf / cdf[-1].clone()
    u = torch.rand(*shape, generator=g, dtype=torch.float64)
    return torch.searchsorted(cdf, u).clamp(max=V - 1).to(torch.int32)


def _full(B, v, dtype=torch.float32):
    return torch.full((B,), v, dtype=dtype)


def make(name: str, seed: int = 0, batch: Optional[int] = None, vocab: Optional[int] = None):
    """Build workload ``name`` on the CPU; ``batch``/``vocab`` shrink it for tests."""
    g = torch.Generator().manual_seed(seed)
    if name == "plumbing_f32_4x512":
        B, V = batch or 4, vocab or 512
        x = torch.randn(B, V, generator=g) * 3.0
        hist = torch.randint(0, V, (B, 32), generator=g, dtype=torch.int32)
        return SampleWorkload(name, x, _full(B, 0.8), _full(B, 50, torch.int32), _full(B, 0.9), _full(B, 0.0),
                              _full(B, 1.1), hist, None, torch.rand(B, generator=g))
    if name == "uniform_f32_64x32000":
        B, V = batch or 64, vocab or 32000
        x = torch.randn(B, V, generator=g) * 2.0
        x += 8.0 * (torch.rand(B, V, generator=g) < 0.01)
        hist = torch.randint(0, V, (B, 512), generator=g, dtype=torch.int32)
        stop = torch.randint(0, V, (4,), generator=g, dtype=torch.int32)
        return SampleWorkload(name, x, _full(B, 0.7), _full(B, 50, torch.int32), _full(B, 0.95), _full(B, 0.05),
                              _full(B, 1.15), hist, stop, torch.rand(B, generator=g))
    if name == "hetero_bf16_256x128256":
        B, V = batch or 256, vocab or 128256
        x = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
        T = 0.1 + 1.4 * torch.rand(B, generator=g)
        K = torch.tensor([0, 1, 20, 50, 200], dtype=torch.int32)[torch.randint(0, 5, (B,), generator=g)]
        P = 0.5 + 0.5 * torch.rand(B, generator=g)
        MP = torch.tensor([0.0, 0.02, 0.1])[torch.randint(0, 3, (B,), generator=g)]
        RP = 1.0 + 0.3 * torch.rand(B, generator=g)
        hist = zipf_ids(g, (B, 2048), V, 1.1)
        return SampleWorkload(name, x, T, K, P, MP, RP, hist, None, torch.rand(B, generator=g))
    if name == "softcap_zipf_f32_512x262144":
        B, V = batch or 512, vocab or 262144
        x = torch.empty(B, V)
        for b in range(B):
            ranks = torch.randperm(V, generator=g).to(torch.float32) + 1.0
            x[b] = -1.2 * torch.log(ranks) + 0.5 * torch.randn(V, generator=g)
        return SampleWorkload(name, x, _full(B, 1.0), _full(B, 0, torch.int32), _full(B, 0.9), _full(B, 0.0),
                              _full(B, 1.0), None, None, torch.rand(B, generator=g), softcap=30.0)
    raise KeyError(f"unknown sampling workload {name!r}")


def make_spec(name: str = "spec_f32_32x5x128256", seed: int = 0, batch: Optional[int] = None,
              vocab: Optional[int] = None, k: int = 5, draft_sampler=None) -> SpecWorkload:
    """Correlated target/draft logits; drafts are drawn from the filtered draft
    distribution with ``draft_sampler(draft [B*K, V], u [B*K]) -> ids`` (the
    inverse-CDF selection rule; callers pass the GPU sampler or the oracle)."""
    if name != "spec_f32_32x5x128256":
        raise KeyError(name)
    g = torch.Generator().manual_seed(seed)
    B, V = batch or 32, vocab or 128256
    z1 = torch.randn(B, k + 1, V, generator=g)
    z2 = torch.randn(B, k, V, generator=g)
    target = 2.0 * z1
    draft = 2.0 * (0.8 * z1[:, :k] + 0.6 * z2)
    u_draft = torch.rand(B * k, generator=g)
    u_acc = torch.rand(B, k, generator=g)
    u_res = torch.rand(B, generator=g)
    if draft_sampler is None:
        ids = torch.zeros(B, k, dtype=torch.int64)
    else:
        ids = draft_sampler(draft.reshape(B * k, V), u_draft).view(B, k).to(torch.int64).cpu()
    return SpecWorkload(name, target, draft, ids, u_acc, u_res, 0.8, 0.95, {"u_draft": u_draft})
