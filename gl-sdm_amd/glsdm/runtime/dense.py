"""Write-proposal arithmetic on the HIP path.

Mirrors ``proposal_delta`` of S/runtime/dense.py:11-14 (S/ =
projects/gl-sdm/src/gl_sdm/): same name, argument order and meaning, fp32
result ``mass * ((exp(log_decay) - 1) * rows + weights * beta * (target -
exp(log_decay) * prediction))`` evaluated as separate fp32 operations in the
reference's order.  Operand shapes are the stack's: rows ``[..., H, k, D]``,
weights ``[..., H, k]``, prediction/target ``[..., H, D]``, beta/log_decay
``[..., H, 1]``, mass ``[...]``.
"""
from ..memory.backends import hip


def proposal_delta(rows, weights, prediction, target, beta, log_decay, mass):
    return hip.proposal_delta(rows.contiguous(), weights.contiguous(), prediction.contiguous(),
                              target.contiguous(), beta.contiguous(), log_decay.contiguous(), mass.contiguous())
