"""Full-distribution log-probability statistics on MI355X (one fused pass per
row): the RL-side consumers of the same ``[B, T, V]`` logits scan as the
sampler.

Drop-ins with the reference's signatures and results (float32, shapes
``[B, T]``):

* ``token_logprobs_from_logits(logits, labels)`` -- ``models/policy.py:47-50``
* ``entropy_from_logits(logits)`` -- ``training/common/logprobs.py:65-68``
* ``kl_full_distribution(new_logits, ref_logits)`` -- ``training/common/logprobs.py:58-62``

``row_stats`` returns any combination of them (plus log-sum-exp) from one
read of the logits.  Logits must be on the ROCm device; there is no CPU path.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import RowStatsArgs, check, lib, ptr
from .sampling import _DTYPES

IGNORE_INDEX = -100  # F.cross_entropy's default ignore_index


@dataclass
class RowStats:
    logprob: Optional[torch.Tensor]   # float32 [...]
    entropy: Optional[torch.Tensor]
    kl: Optional[torch.Tensor]
    lse: Optional[torch.Tensor]


def _rows(x: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm device (no CPU fallback)")
    if x.dtype not in _DTYPES:
        raise NotImplementedError(f"{name} dtype {x.dtype} is not supported (float32, bfloat16, float16)")
    if x.dim() < 1:
        raise ValueError(f"{name} must have a vocabulary dimension")
    x2 = x.reshape(-1, x.size(-1))
    if x2.stride(-1) != 1 or (x2.size(0) > 1 and x2.stride(0) < x2.size(1)):
        x2 = x2.contiguous()
    return x2


def row_stats(logits: torch.Tensor, labels: Optional[torch.Tensor] = None, ref_logits: Optional[torch.Tensor] = None,
              *, entropy: bool = False, lse: bool = False, ignore_index: int = IGNORE_INDEX,
              check_labels: bool = True) -> RowStats:
    """Per-row statistics of ``logits [..., V]`` in one pass: the log-prob of
    ``labels [...]`` (if given), the entropy (``entropy=True``), KL(logits ||
    ref_logits) (if ``ref_logits`` is given) and log-sum-exp (``lse=True``)."""
    x = _rows(logits, "logits")
    lead = logits.shape[:-1]
    R, V = x.shape
    dev = x.device
    y = None
    if ref_logits is not None:
        if ref_logits.shape != logits.shape or ref_logits.dtype != logits.dtype:
            raise ValueError("ref_logits must match logits in shape and dtype")
        y = _rows(ref_logits, "ref_logits")
    lab = None
    if labels is not None:
        if tuple(labels.shape) != tuple(lead):
            raise ValueError(f"labels {tuple(labels.shape)} must be {tuple(lead)}")
        lab = labels.to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
        if check_labels and R > 0:
            bad = ((lab < 0) & (lab != ignore_index)) | (lab >= V)
            if bool(bad.any()):
                raise IndexError(f"target {int(lab[bad][0])} is out of bounds for {V} classes")
    out = lambda on: torch.empty(R, dtype=torch.float32, device=dev) if on else None  # noqa: E731
    o_lp, o_h, o_kl, o_lse = out(lab is not None), out(entropy), out(y is not None), out(lse)
    a = RowStatsArgs()
    a.struct_size = ctypes.sizeof(RowStatsArgs)
    a.dtype = _DTYPES[x.dtype]
    a.logits, a.ref_logits = x.data_ptr(), ptr(y)
    a.rows, a.vocab = R, V
    a.ld = x.stride(0) if R > 1 else V
    a.ref_ld = (y.stride(0) if R > 1 else V) if y is not None else 0
    a.labels, a.ignore_index = ptr(lab), int(ignore_index)
    a.out_logprob, a.out_entropy, a.out_kl, a.out_lse = ptr(o_lp), ptr(o_h), ptr(o_kl), ptr(o_lse)
    check(lib().fl_row_stats(ctypes.byref(a), _lib.stream_handle(dev)), "fl_row_stats")
    _keep = (x, y, lab)  # noqa: F841  (alive until the launch has consumed them)
    shape = lambda t: None if t is None else t.view(lead)  # noqa: E731
    return RowStats(shape(o_lp), shape(o_h), shape(o_kl), shape(o_lse))


def token_logprobs_from_logits(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """Per-token ``log p(label)`` of ``logits [B, T, V]``, ``labels [B, T]``
    (``-cross_entropy`` of the float32 logits; reference ``policy.py:47-50``)."""
    return row_stats(logits, labels).logprob


def entropy_from_logits(logits: torch.Tensor) -> torch.Tensor:
    """Per-position entropy ``[B, T]`` of the full distribution (reference
    ``training/common/logprobs.py:65-68``)."""
    return row_stats(logits, entropy=True).entropy


def kl_full_distribution(new_logits: torch.Tensor, ref_logits: torch.Tensor) -> torch.Tensor:
    """Exact per-token ``KL(new || ref)`` from full-vocabulary logits ``[B, T, V]``
    (reference ``training/common/logprobs.py:58-62``)."""
    return row_stats(new_logits, ref_logits=ref_logits).kl
