"""CPU restatement of the reference's full-distribution log-probability
statistics (test infrastructure only: the reference the MI355X kernels are
compared with, never part of the product path).

Each function follows one reference function line by line, in float32 on
the CPU as the reference computes after ``.float()``:

* ``token_logprobs_from_logits``  src/forgeline/models/policy.py:47-50
* ``entropy_from_logits``         src/forgeline/training/common/logprobs.py:65-68
* ``kl_full_distribution``        src/forgeline/training/common/logprobs.py:58-62
* ``logsumexp``                   the normaliser the three share

Pinned in tests/test_oracle.py by closed forms (uniform rows, two-point
rows), float64 brute force on small inputs, shift invariance and the
cross-entropy ignore_index convention.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def token_logprobs_from_logits(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """``-F.cross_entropy(logits.reshape(-1, V).float(), labels.reshape(-1), reduction="none")``
    reshaped to ``labels``' shape (policy.py:47-50; ignore_index -100 gives -0.0)."""
    V = logits.size(-1)
    lp = -F.cross_entropy(logits.reshape(-1, V).float(), labels.reshape(-1).long(), reduction="none")
    return lp.reshape(labels.shape)


def entropy_from_logits(logits: torch.Tensor) -> torch.Tensor:
    """``-(exp(lp) * lp).sum(-1)`` with ``lp = log_softmax(logits.float())`` (logprobs.py:65-68)."""
    lp = torch.log_softmax(logits.float(), dim=-1)
    return -(lp.exp() * lp).sum(-1)


def kl_full_distribution(new_logits: torch.Tensor, ref_logits: torch.Tensor) -> torch.Tensor:
    """``(exp(new_lp) * (new_lp - ref_lp)).sum(-1)`` (logprobs.py:58-62)."""
    new_lp = torch.log_softmax(new_logits.float(), dim=-1)
    ref_lp = torch.log_softmax(ref_logits.float(), dim=-1)
    return (new_lp.exp() * (new_lp - ref_lp)).sum(-1)


def logsumexp(logits: torch.Tensor) -> torch.Tensor:
    return torch.logsumexp(logits.float(), dim=-1)
