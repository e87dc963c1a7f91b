"""One untied global layer: routed read of the chunk snapshot, mixing, MLP,
and its write proposal (S/layers/global_layer.py:13-54, S/ =
projects/gl-sdm/src/gl_sdm/)."""
import torch
from torch import nn
import torch.nn.functional as F

from .. import _native as N
from ..memory import routing
from ..memory.proposals import layer_proposal, log_proposal
from .block import check_reg_mode, regulariser, zero
from .common import MLP, RMSNorm, linear, linear_group
from .router import GlobalRouter


def write_gates(b_lin, d_lin):
    """``(sigmoid(b) [..., 1], -softplus(d - 4) [..., 1])`` in fp32 from the beta and
    decay projections' outputs, in one HIP launch (``glsdm_write_gates``)."""
    b_lin, d_lin = b_lin.contiguous(), d_lin.contiguous()
    beta = torch.empty(b_lin.shape, dtype=torch.float32, device=b_lin.device)
    log_decay = torch.empty_like(beta)
    N.call("glsdm_write_gates", N.ptr(b_lin), N.ptr(d_lin), N.dtype_code(b_lin), b_lin.numel(), N.ptr(beta),
           N.ptr(log_decay), N.stream(b_lin.device))
    return beta.unsqueeze(-1), log_decay.unsqueeze(-1)


class GlobalLayer(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        check_reg_mode(cfg)
        dim = cfg["hidden_size"]
        self.attn = GlobalRouter(cfg)
        self.norm1, self.norm2 = RMSNorm(dim), RMSNorm(dim)
        self.mlp = MLP(dim, cfg.get("intermediate_size"))
        self.reg_mode = cfg.get("reg_mode", "baseline")

    def forward(self, x, snapshot, physical=None):
        """``x + proj(read_norm(read))`` then ``+ mlp(norm2(x))``; the read routes the
        factor scores ``q(norm1(x))`` through the snapshot.  The reference widens
        them with ``.float()`` first; the route takes the projection's bf16 output
        as is and orders it exactly as its fp32 widening."""
        B, T, _ = x.shape
        router = self.attn
        dtype = router.q.weight.dtype
        scores = linear(router.q, self.norm1.cast(x, dtype)).view(B, T, router.heads, -1)
        # outside autograd the read rounds its fp32 sums to the projection dtype itself
        grad = torch.is_grad_enabled() and (x.requires_grad or snapshot.values.requires_grad)
        readings, _, _ = routing.routed_read(self, snapshot.values, scores, router.num_reads, physical,
                                             out_dtype=torch.float32 if grad else dtype)
        x = linear(router.proj, router.read_norm(readings.to(dtype)).flatten(-2), x)
        x = self.mlp(self.norm2.cast(x, dtype), residual=x)
        return x, regulariser(x, self.reg_mode), zero(x)

    def propose(self, x, snapshot, offset, layer_idx, chunk_size, num_layers, physical=None, log=None):
        """Write proposal of the chunk's tokens against ``snapshot``.

        Each token-head's delta against the rows its write route picks is
        ``(exp(g) - 1) * row + w * beta * (target - exp(g) * prediction)`` with
        mass 1, with no averaging over tokens or layers; collisions commit in
        (address, position in chunk, layer) order through the keys.  Outside
        autograd the deltas stay deferred: the commit forms them from the rows
        it touches; with a proposal ``log`` (the stack's inference path) the
        gates, keys and error terms go straight into the log in one launch.
        Under autograd (training with writes) they are materialised as the
        reference does, so gradients flow through the commit into later
        chunks' reads.
        """
        training = torch.is_grad_enabled() and (x.requires_grad or snapshot.values.requires_grad)
        B, T, _ = x.shape
        router = self.attn
        zk = self.norm1.cast(x, router.k.weight.dtype)
        scores = linear(router.k, zk).view(B, T, router.heads, -1)
        prediction, index, weights = routing.routed_read(self, snapshot.values, scores, router.num_writes, physical)
        vdt = router.v.weight.dtype
        dense = zk if vdt == zk.dtype else self.norm1.cast(x, vdt)
        target, b_lin, d_lin = linear_group((router.v, router.beta, router.decay), dense)
        target = target.view(B, T, router.heads, router.head_dim)
        if log is not None and not training and b_lin.is_cuda and b_lin.dtype in (torch.float32, torch.bfloat16):
            return log_proposal(log, snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx,
                                chunk_size, num_layers)
        if training or not b_lin.is_cuda or b_lin.dtype not in (torch.float32, torch.bfloat16):
            beta = b_lin.float().sigmoid().unsqueeze(-1)
            log_decay = -F.softplus(d_lin.float() - 4).unsqueeze(-1)
        else:
            beta, log_decay = write_gates(b_lin, d_lin)
        return layer_proposal(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx,
                              chunk_size, num_layers, deferred=not training)
