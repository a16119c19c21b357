"""cross_entropy (reference kernels/cross_entropy.py:52-67, csrc/cross_entropy_op.cu:10-62,92-116):
the mean over non-ignored targets of -log softmax(logits)[target], with F.cross_entropy's
ignore_index default of -100."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check
from .backward import CrossEntropyFunction, needs_grad


def cross_entropy_fwd(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100):
    """(loss, lse, n_valid): loss is the fp32 mean over targets != ignore_index (0 when none is, as the
    reference's clamp(min=1) gives); lse (N,) fp32 is each row's log-sum-exp (0 for an ignored row);
    n_valid (1,) int32 counts the valid targets. All on the device, no host synchronisation. A target
    outside [0, V) other than ignore_index is skipped like an ignored one and recorded on the device
    (kernels.raise_device_errors)."""
    check("cross_entropy", logits)
    if logits.dim() != 2:
        raise ValueError(f"cross_entropy: logits must be (N, V), got {tuple(logits.shape)}")
    N, V = logits.shape
    if targets.shape != (N,) or not targets.is_cuda or targets.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"cross_entropy: targets must be an integer ({N},) device tensor")
    lg = logits.contiguous()
    tg = targets.to(torch.int64).contiguous()
    per_token = torch.empty(N, dtype=torch.float32, device=lg.device)
    lse = torch.empty(N, dtype=torch.float32, device=lg.device)
    loss = torch.empty((), dtype=torch.float32, device=lg.device)
    n_valid = torch.empty(1, dtype=torch.int32, device=lg.device)
    _lib.call("q3_cross_entropy", lg.data_ptr(), tg.data_ptr(), per_token.data_ptr(), lse.data_ptr(),
              loss.data_ptr(), n_valid.data_ptr(), N, V, int(ignore_index), _lib.dtype_code(lg.dtype),
              _lib.status_word(lg.device).data_ptr(), _lib.stream())
    return loss, lse, n_valid


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100) -> torch.Tensor:
    """Mean cross-entropy of (N, V) logits against (N,) int64 targets; fp32 0-dim result (the
    reference divides its fp32 per-token losses by the valid count). Differentiable in logits."""
    if needs_grad(logits):
        return CrossEntropyFunction.apply(logits, targets, ignore_index)
    return cross_entropy_fwd(logits, targets, ignore_index)[0]
