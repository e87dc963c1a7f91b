"""Write-proposal arithmetic on the HIP path.

Mirrors ``proposal_delta`` of S/runtime/dense.py:11-14 (S/ =
projects/gl-sdm/src/gl_sdm/): same name, argument order and meaning, fp32
result ``mass * ((exp(log_decay) - 1) * rows + weights * beta * (target -
exp(log_decay) * prediction))`` evaluated as separate fp32 operations in the
reference's order.  Operand shapes are the stack's: rows ``[..., H, k, D]``,
weights ``[..., H, k]``, prediction/target ``[..., H, D]``, beta/log_decay
``[..., H, 1]``, mass ``[...]``.

Under autograd (training with writes) the same operations run as device
tensor ops, so that gradients reach every operand; the HIP kernel is
forward-only.
"""
import torch

from ..memory.backends import hip


def proposal_delta(rows, weights, prediction, target, beta, log_decay, mass):
    operands = (rows, weights, prediction, target, beta, log_decay, mass)
    if torch.is_grad_enabled() and any(t.requires_grad for t in operands):
        hip.require_cuda(*operands)
        decay = log_decay.exp()
        error = beta * (target.float() - decay * prediction)
        spread = (decay[..., None] - 1) * rows + weights[..., None] * error[..., None, :]
        return mass[..., None, None, None] * spread
    return hip.proposal_delta(rows.contiguous(), weights.contiguous(), prediction.contiguous(),
                              target.contiguous(), beta.contiguous(), log_decay.contiguous(), mass.contiguous())
