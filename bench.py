"""Benchmark of the GL-SDM memory operator on one MI355X (headline config).

Workload: B=8 requests, T=2048 tokens in 4 commit
epochs of C=512, H=8 heads, bank M=65536 slots per head (half=256, L=512
factor scores per head), key dim dk=128, value dim D=128 (H*D = 1024), top-k
16, bf16 bank/queries/deltas, fp32 accumulation.  One step = all 4 epochs of:

  score+route(read queries) -> snapshot read               (read path)
  score+route+keys(write queries) -> commit                 (write path)

(score+route is one fused kernel: MFMA scores feed the top-k through LDS; the
write route's kernel also emits the proposal addresses and collision keys)

with the bank updated in place at every 512-token clock (donated commit).
``--write-path proposals`` replaces the synthetic deltas by the stack's write
path (S/layers/global_layer.py:42-54): routed read of the write route
(prediction) -> proposal error terms -> fused proposal commit, whose deltas
are formed inside the commit; ``proposals-materialised`` runs the same work
the reference's way (gather rows -> materialised fp32 deltas -> commit).
Inputs are synthetic, generated on the CPU with a seeded generator and copied
to HBM before the timed region.  Prints one JSON line (see the driver
contract); rank 0 only, one GPU.
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gl-sdm_amd"))

HBM_PEAK = 8.0e12          # B/s, MI355X
MFMA_BF16_PEAK = 2.5e15    # FLOP/s dense bf16

CONFIGS = {
    # the reference's CPU-runnable case (fp32, one epoch)
    1: dict(B=2, T=512, C=512, H=1, half=64, dk=64, D=256, k=8, dtype=torch.float32, skew=False),
    # the headline roofline config
    2: dict(B=8, T=2048, C=512, H=8, half=256, dk=128, D=128, k=16, dtype=torch.bfloat16, skew=False),
    # 2^20-slot bank, Zipf(1.1)-skewed routes over 4096 product clusters
    3: dict(B=4, T=4096, C=512, H=1, half=1024, dk=128, D=512, k=32, dtype=torch.bfloat16, skew=True),
}
CFG = CONFIGS[2]

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this
# workload, scaled by a 256 MiB copy measured in the same run (FETCH x 1.9998,
# WRITE x 1.0); source: profiles/glsdm_kernels.config2.hbm-traffic.md.  Re-measured
# whenever a kernel of the path changes.
TRAFFIC_PER_LAUNCH = {
    "score_route": (4911.6 * 1.9998 + 7782.4) * 1024,
    "read": (67885.0 * 1.9998 + 16384.0) * 1024,
    # glsdm_commit on the bucket path: tile bucketing, bucket sort, segment
    "commit": ((2094.6 + 2601.8 + 132820.3) * 1.9998 + (6144.1 + 4100.5 + 120860.8)) * 1024,
}


def _zipf_queries(g, B, T, H, centres, dk, s=1.1):
    """Queries around product cluster z = (z0, z1) with z ~ Zipf(s) over a seeded rank permutation."""
    n = centres[0].shape[0]
    p = torch.arange(1, n * n + 1, dtype=torch.float64).pow(-s)
    perm = torch.randperm(n * n, generator=g)
    z = perm[torch.multinomial(p / p.sum(), B * T * H, replacement=True, generator=g)]
    q = centres[0][z // n] + centres[1][z % n] + 0.05 * torch.randn(B * T * H, dk, generator=g)
    return torch.nn.functional.normalize(q, dim=-1).view(B, T, H, dk)


def make_inputs(cfg, seed=0):
    """Seeded CPU generation in a fixed order, then the config's dtype."""
    g = torch.Generator("cpu").manual_seed(seed)
    B, T, H, half, dk, D, k = (cfg[x] for x in ("B", "T", "H", "half", "dk", "D", "k"))
    dt = cfg["dtype"]
    norm = torch.nn.functional.normalize
    if cfg["skew"]:
        centres = [norm(torch.randn(64, dk, generator=g), dim=-1) for _ in range(2)]
        sub = [norm(centres[f][torch.arange(half) % 64] + 0.05 * torch.randn(half, dk, generator=g), dim=-1)
               for f in range(2)]
        keys = torch.cat(sub).view(1, 2 * half, dk).expand(H, -1, -1).contiguous()
    else:
        keys = norm(torch.randn(H, 2 * half, dk, generator=g), dim=-1)
    bank = (torch.randn(H, half * half, D, generator=g) * 0.02).to(dt)
    if cfg["skew"]:
        qr = _zipf_queries(g, B, T, H, centres, dk)
        qw = _zipf_queries(g, B, T, H, centres, dk)
    else:
        qr = norm(torch.randn(B, T, H, dk, generator=g), dim=-1)
        qw = norm(torch.randn(B, T, H, dk, generator=g), dim=-1)
    delta = (torch.randn(B, T, H, k, D, generator=g) * 0.02).to(dt)
    return keys.bfloat16(), bank, qr.bfloat16(), qw.bfloat16(), delta


WRITE_PATHS = {
    "deltas": "commit of synthetic deltas",
    "proposals": "write read + proposal error + fused proposal commit",
    "proposals-materialised": "write read + row gather + proposal deltas + commit",
}


def make_write_operands(cfg, seed=1):
    """Value targets (config dtype), gates beta/log_decay [B, T, H, 1] (as
    S/layers/global_layer.py:47-49 forms them) for the proposal write path."""
    g = torch.Generator("cpu").manual_seed(seed)
    B, T, H, D = (cfg[x] for x in ("B", "T", "H", "D"))
    target = (torch.randn(B, T, H, D, generator=g) * 0.1).to(cfg["dtype"])
    beta = torch.randn(B, T, H, 1, generator=g).sigmoid()
    log_decay = -torch.nn.functional.softplus(torch.randn(B, T, H, 1, generator=g) - 4)
    return target, beta, log_decay


class Pipeline:
    """Preallocated buffers and direct C-ABI calls for the 4-epoch workload.

    Two schedules of the same work (``--schedule``; ``auto`` picks overlap when a
    step has more than one epoch, serial otherwise):
    * overlap: scoring+routing never reads the bank, so the route stream
      computes epoch e+1's read and write routes and proposal keys while the
      memory stream runs epoch e's read and commit.  The memory stream waits for
      an epoch's routes with an event; read(e+1) follows commit(e) in stream
      order, so every read still sees the bank version of its epoch.  The write
      route's proposal keys come from a separate keys launch on the route stream
      (faster beside the memory kernels than the fused route-with-keys, measured);
    * serial: every call on one stream, epoch after epoch (one-epoch steps gain
      nothing from the cross-stream waits).  The per-call durations reported
      next to the step time come from a separate serial pass.
    """

    def __init__(self, cfg, device, write_path="deltas", backward=False, overlay=False, split_commit=False,
                 route_parts=0):
        from glsdm import _native as N
        self.N, self.cfg, self.dev, self.write_path, self.backward = N, cfg, device, write_path, backward
        self.overlay = overlay
        if split_commit and (overlay or write_path != "deltas"):
            raise SystemExit("--split-commit runs the dense bank with synthetic deltas only")
        self.split_commit = split_commit
        keys, bank, qr, qw, delta = make_inputs(cfg)
        B, T, C, H, half, dk, D, k = (cfg[x] for x in ("B", "T", "C", "H", "half", "dk", "D", "k"))
        self.epochs = T // C
        self.keys = keys.to(device)
        self.bank = bank.unsqueeze(0).expand(B, -1, -1, -1).contiguous().to(device)   # per-request replicas
        split = lambda x: [x[:, e * C:(e + 1) * C].contiguous().to(device) for e in range(self.epochs)]
        self.qr, self.qw, self.delta = split(qr), split(qw), split(delta)
        per_epoch = lambda dt: [torch.empty(B, C, H, k, dtype=dt, device=device) for _ in range(self.epochs)]
        self.idx, self.w = per_epoch(torch.int64), per_epoch(torch.float32)
        self.widx, self.ww = per_epoch(torch.int64), per_epoch(torch.float32)
        self.addr, self.ckeys = per_epoch(torch.int64), per_epoch(torch.int64)
        self.out = torch.empty(B, C, H, D, dtype=torch.float32, device=device)
        self.rows = B * H * half * half
        self.E = B * C * H * k
        size = ctypes.c_size_t(0)
        N.call("glsdm_commit_workspace_bytes", self.E, self.rows, ctypes.byref(size))
        self.ws = torch.empty(size.value, dtype=torch.uint8, device=device)
        # split commit: one workspace per epoch, since the route stream sorts epoch e+1's
        # entries while the memory stream still applies epoch e's from its workspace
        self.cws = [torch.empty(size.value, dtype=torch.uint8, device=device)
                    for _ in range(self.epochs if split_commit else 0)]
        N.call("glsdm_score_route_workspace_bytes", B, C, H, half, k, ctypes.byref(size))
        # one route workspace: both routing calls of an epoch run on the same stream, one after the other
        self.route_ws = torch.empty(max(size.value, 8), dtype=torch.uint8, device=device)
        self.unique = torch.zeros(1, dtype=torch.int64, device=device)
        if write_path != "deltas":
            self.delta = None
            target, beta, log_decay = make_write_operands(cfg)
            self.target, self.beta, self.log_decay = split(target), split(beta), split(log_decay)
            self.pred = torch.empty(B, C, H, D, dtype=torch.float32, device=device)
            self.error = torch.empty(B, C, H, D, dtype=torch.float32, device=device)
            self.decay = torch.empty(B, C, H, dtype=torch.float32, device=device)
            self.mass = torch.ones(B, C, dtype=torch.float32, device=device)
            if write_path == "proposals-materialised":
                self.rows_buf = torch.empty(B, C, H, k, D, dtype=self.bank.dtype, device=device)
                self.dbuf = torch.empty(B, C, H, k, D, dtype=torch.float32, device=device)
        if overlay:
            if write_path != "deltas" or backward:
                raise SystemExit("--bank overlay runs the BASELINE protocol only (deltas, no backward)")
            # one shared base [H, S, D]; per step a fresh request batch: map reset to -1, pool emptied
            self.base = bank.to(device)
            self.bank = None
            self.map = torch.full((B, H, half * half), -1, dtype=torch.int32, device=device)
            self.pool = torch.empty(self.epochs * self.E, D, dtype=self.base.dtype, device=device)
        if backward:
            # read backward into the learned [H, S, D] bank's fp32 gradient: the
            # requests' replicas fold onto one row (address h*S + slot)
            g = torch.Generator("cpu").manual_seed(2)
            self.grad_out = (torch.randn(B, C, H, D, generator=g) * 0.01).to(device)
            self.grad_w = torch.empty(B, C, H, k, dtype=torch.float32, device=device)
            self.grad_scores = torch.empty(B, C, H, 2 * half, dtype=torch.float32, device=device)
            self.grad_bank = torch.zeros(H * half * half, D, dtype=torch.float32, device=device)
            self.fold = [torch.empty(B, C, H, k, dtype=torch.int64, device=device) for _ in range(self.epochs)]
            N.call("glsdm_commit_workspace_bytes", self.E, H * half * half, ctypes.byref(size))
            self.bw_ws = torch.empty(size.value, dtype=torch.uint8, device=device)
        self.mem_stream = torch.cuda.current_stream(device)
        self.route_stream = torch.cuda.Stream(device)          # default priority
        # overlap schedule: each route call launched over `route_parts` consecutive request
        # ranges (default 1: whole launches)
        parts = max(1, route_parts)
        while parts > 1 and B % parts:
            parts -= 1
        self.route_parts = parts
        self.routed = [torch.cuda.Event() for _ in range(self.epochs)]
        self.consumed = [torch.cuda.Event() for _ in range(self.epochs)]
        for ev in self.consumed:
            ev.record(self.mem_stream)
        self.timers = None
        self.only = None     # time only this call name (None: every call)
        # the read's entry point: glsdm_read keeps up to four route entries per lane group
        # in flight; glsdm_read_narrow keeps one and is small enough that the route kernel's
        # waves still fit beside its waves, which the overlap schedule needs (set by main)
        self.read_entry = "glsdm_read"

    def _timed(self, name, stream, fn):
        if self.timers is None or (self.only is not None and name != self.only):
            return fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        self.timers.setdefault(name, []).append((a, b))

    def routes(self, e, stream):
        if stream is self.route_stream:
            return self.routes_parts(e, stream)
        N, c, p, st = self.N, self.cfg, self.N.ptr, self.N.ctypes.c_void_p(stream.cuda_stream)
        B, C, H, half, dk, k = (c[x] for x in ("B", "C", "H", "half", "dk", "k"))
        self._timed("score_route", stream, lambda: N.call(
            "glsdm_score_route", p(self.qr[e]), p(self.keys), B, C, H, dk, half, k, N.TIE_HIGHEST, None,
            p(self.idx[e]), p(self.w[e]), p(self.route_ws), self.route_ws.numel(), st))
        # the write route also emits its proposal addresses and keys addr*C + t (one launch)
        self._timed("score_route_keys", stream, lambda: N.call(
            "glsdm_score_route_keys", p(self.qw[e]), p(self.keys), B, C, H, dk, half, k, N.TIE_HIGHEST, 0, C, 1, 0,
            p(self.widx[e]), p(self.ww[e]), p(self.addr[e]), p(self.ckeys[e]), p(self.route_ws),
            self.route_ws.numel(), st))

    def routes_parts(self, e, stream):
        """The overlap schedule's routes: the read and write routes (each launched over
        `route_parts` request ranges; the same routes bit for bit, requests are
        independent), then the write route's proposal addresses and keys from one
        `glsdm_proposal_keys` launch over the epoch.  Beside the memory stream this
        runs faster than the write route emitting its keys itself
        (`glsdm_score_route_keys`, which the serial schedule uses): 0.78 vs 0.92 ms
        per config-2 step, measured; the memory stream's commit then takes 132 µs
        instead of 152."""
        N, c, st = self.N, self.cfg, self.N.ctypes.c_void_p(stream.cuda_stream)
        B, C, H, half, dk, k = (c[x] for x in ("B", "C", "H", "half", "dk", "k"))
        n = B // self.route_parts
        at = lambda t, i: N.ctypes.c_void_p(t[i * n:(i + 1) * n].data_ptr())
        for q, idx, w in ((self.qr[e], self.idx[e], self.w[e]), (self.qw[e], self.widx[e], self.ww[e])):
            name = "score_route" if q is self.qr[e] else "score_route_keys"
            for i in range(self.route_parts):
                self._timed(name, stream, lambda: N.call(
                    "glsdm_score_route", at(q, i), N.ptr(self.keys), n, C, H, dk, half, k, N.TIE_HIGHEST, None,
                    at(idx, i), at(w, i), N.ptr(self.route_ws), self.route_ws.numel(), st))
        self._timed("score_route_keys", stream, lambda: N.call(
            "glsdm_proposal_keys", N.ptr(self.widx[e]), B, C, H, k, half * half, 0, C, 1, 0, N.ptr(self.addr[e]),
            N.ptr(self.ckeys[e]), st))

    def prepare(self, e, stream):
        """Split commit, first half: group epoch e's entries by address (reads only
        the write route's addresses, never the bank) into the epoch's workspace."""
        N, p, st = self.N, self.N.ptr, self.N.ctypes.c_void_p(stream.cuda_stream)
        self._timed("commit_prepare", stream, lambda: N.call(
            "glsdm_commit_prepare", self.rows, p(self.addr[e]), self.E, p(self.cws[e]), self.cws[e].numel(), st))

    def memory(self, e, stream, count_unique=False, split=False):
        N, c, p, st = self.N, self.cfg, self.N.ptr, self.N.ctypes.c_void_p(stream.cuda_stream)
        B, C, H, half, D, k = (c[x] for x in ("B", "C", "H", "half", "D", "k"))
        dt = N.dtype_code(self.base if self.overlay else self.bank)
        uq = p(self.unique) if count_unique else None
        if self.overlay:
            dt = N.dtype_code(self.base)
            S = half * half
            self._timed("read", stream, lambda: N.call(
                "glsdm_overlay_read", p(self.base), dt, p(self.map), p(self.pool), B, H, S, D, C, k, p(self.idx[e]),
                p(self.w[e]), p(self.out), N.F32, st))
            self._timed("commit", stream, lambda: N.call(
                "glsdm_overlay_commit", p(self.base), dt, B, H, S, D, p(self.map), p(self.pool),
                self.pool.shape[0], e * self.E, p(self.addr[e]), p(self.delta[e]), dt, p(self.ckeys[e]),
                self.E, p(self.ws), self.ws.numel(), uq, st))
            return
        self._timed("read", stream, lambda: N.call(
            self.read_entry, p(self.bank), dt, B, H, half * half, D, C, k, p(self.idx[e]), p(self.w[e]),
            p(self.out), N.F32, st))
        if self.backward:
            S = half * half
            self._timed("read_bw_weights", stream, lambda: N.call(
                "glsdm_read_backward_weights", p(self.bank), dt, B, H, S, D, C, k, p(self.idx[e]),
                p(self.grad_out), p(self.grad_w), st))
            self._timed("route_bw", stream, lambda: N.call(
                "glsdm_route_backward", p(self.idx[e]), p(self.w[e]), p(self.grad_w), B * C * H, half, k,
                p(self.grad_scores), st))
            # [B, C, H, k] seen as one request of B*C tokens: addresses h*S + slot
            self._timed("fold", stream, lambda: N.call(
                "glsdm_absolute_addresses", p(self.idx[e]), 1, B * C, H, k, S, p(self.fold[e]), st))
            self._timed("read_bw_rows", stream, lambda: N.call(
                "glsdm_read_backward_rows", p(self.grad_bank), H * S, D, p(self.fold[e]), self.E, k,
                p(self.w[e]), p(self.grad_out), p(self.bw_ws), self.bw_ws.numel(), st))
        if self.write_path == "deltas" and split:
            self._timed("commit", stream, lambda: N.call(
                "glsdm_commit_apply", p(self.bank), dt, self.rows, D, p(self.delta[e]), dt, p(self.ckeys[e]),
                self.E, p(self.cws[e]), self.cws[e].numel(), uq, st))
            return
        if self.write_path == "deltas":
            self._timed("commit", stream, lambda: N.call(
                "glsdm_commit", p(self.bank), dt, self.rows, D, p(self.addr[e]), p(self.delta[e]), dt,
                p(self.ckeys[e]), self.E, p(self.ws), self.ws.numel(), uq, st))
            return
        R = B * C * H
        # the write route's routed read: the proposal's prediction
        self._timed("write_read", stream, lambda: N.call(
            self.read_entry, p(self.bank), dt, B, H, half * half, D, C, k, p(self.widx[e]), p(self.ww[e]),
            p(self.pred), N.F32, st))
        if self.write_path == "proposals":
            self._timed("proposal_error", stream, lambda: N.call(
                "glsdm_proposal_error", R, D, p(self.pred), p(self.target[e]), N.dtype_code(self.target[e]),
                p(self.beta[e]), p(self.log_decay[e]), p(self.error), p(self.decay), st))
            self._timed("commit", stream, lambda: N.call(
                "glsdm_commit_proposals", p(self.bank), dt, self.rows, D, p(self.addr[e]), p(self.ckeys[e]),
                self.E, k, p(self.ww[e]), p(self.error), p(self.decay), p(self.mass), H, p(self.ws),
                self.ws.numel(), uq, st))
            return
        self._timed("gather", stream, lambda: N.call(
            "glsdm_gather_rows", p(self.bank), dt, self.rows, D, p(self.addr[e]), self.E, p(self.rows_buf), st))
        self._timed("proposal_delta", stream, lambda: N.call(
            "glsdm_proposal_delta", p(self.rows_buf), dt, R, k, D, p(self.ww[e]), p(self.pred),
            p(self.target[e]), N.dtype_code(self.target[e]), p(self.beta[e]), p(self.log_decay[e]),
            p(self.mass), H, p(self.dbuf), st))
        self._timed("commit", stream, lambda: N.call(
            "glsdm_commit", p(self.bank), dt, self.rows, D, p(self.addr[e]), p(self.dbuf), N.F32,
            p(self.ckeys[e]), self.E, p(self.ws), self.ws.numel(), uq, st))

    def new_batch(self):
        """Overlay mode: a fresh snapshot of the base for the step's requests (map and pool reset)."""
        if self.overlay:
            self.map.fill_(-1)

    def step_serial(self):
        self.new_batch()
        for e in range(self.epochs):
            self.routes(e, self.mem_stream)
            self.memory(e, self.mem_stream)

    def step(self):
        rs, ms = self.route_stream, self.mem_stream
        self.new_batch()
        for e in range(self.epochs):
            rs.wait_event(self.consumed[e])   # the previous step's read/commit of epoch e is done with its routes
            self.routes(e, rs)
            if self.split_commit:
                self.prepare(e, rs)
            self.routed[e].record(rs)
        for e in range(self.epochs):
            ms.wait_event(self.routed[e])
            self.memory(e, ms, split=self.split_commit)
            self.consumed[e].record(ms)

    def unique_rows(self):
        """Touched rows U per epoch (untimed serial pass on a scratch copy of the bank)."""
        saved = self.bank
        self.bank = None if self.overlay else saved.clone()
        self.new_batch()
        out = []
        for e in range(self.epochs):
            self.unique.zero_()
            self.routes(e, self.mem_stream)
            self.memory(e, self.mem_stream, count_unique=True)
            torch.cuda.synchronize()
            out.append(int(self.unique.item()))
        self.bank = saved
        return out


def algorithmic_bytes(cfg, unique, write_path="deltas"):
    """HBM bytes per epoch: (read incl. queries, read kernel, [commit launch per
    epoch], other write-path work).  Bank and deltas in the config's dtype.

    ``deltas``: the commit reads the synthetic deltas, addresses and keys and
    each touched row twice.  Proposal write paths add the write route's read
    (k rows, fp32 prediction, index/weights) and the error terms' inputs
    (prediction fp32, target, gates) as other work; their commit launch reads
    each error row and decay/mass once plus weight, address and key per entry
    (``proposals``), or the materialised fp32 deltas, addresses and keys
    (``proposals-materialised``: the gather and delta kernels are that
    path's own overhead and are not counted as algorithmic)."""
    B, C, H, dk, D, k = (cfg[x] for x in ("B", "C", "H", "dk", "D", "k"))
    sv = torch.tensor([], dtype=cfg["dtype"]).element_size()
    rows = B * C * H
    read_kernel = rows * (k * D * sv + D * 4 + k * 12)           # gathers + fp32 out + idx/w
    read = read_kernel + rows * dk * 2                            # + queries read once
    E = rows * k
    rmw = [2 * u * D * sv for u in unique]
    if write_path == "deltas":
        return read, read_kernel, [E * D * sv + E * 16 + x for x in rmw], 0
    other = read_kernel + rows * (D * 4 + D * sv + 12)
    if write_path == "proposals":
        return read, read_kernel, [rows * (D * 4 + 8) + E * 20 + x for x in rmw], other
    return read, read_kernel, [E * D * 4 + E * 16 + x for x in rmw], other


def literal_scoring(cfg, dev, reps=20):
    """The reference's literal scoring projection for one epoch of the workload:
    ``router.q`` as a bf16 Linear [B*C, d_model] x [d_model, H*L] on hipBLASLt
    (d_model = H*D, S/layers/global_layer.py:26), and the route of its bf16
    output as is (glsdm_route, 32-bit keys).  Returns the GEMM's MFMA rate and
    both calls' times (HIP events on the current stream)."""
    from glsdm import _native as N
    from glsdm.memory.backends import hip
    B, C, H, half, D, k = (cfg[x] for x in ("B", "C", "H", "half", "D", "k"))
    d_model, L, n = H * D, 2 * half, B * C
    g = torch.Generator("cpu").manual_seed(5)
    x = torch.nn.functional.normalize(torch.randn(n, d_model, generator=g), dim=-1).bfloat16().to(dev)
    # the Linear's weight [H*L, d_model], stored transposed and contiguous for a plain NN product
    w_t = (torch.randn(H * L, d_model, generator=g) * d_model ** -0.5).bfloat16().t().contiguous().to(dev)
    scores = torch.empty(n, H * L, dtype=torch.bfloat16, device=dev)
    index = torch.empty(n * H, k, dtype=torch.int64, device=dev)
    weights = torch.empty(n * H, k, dtype=torch.float32, device=dev)
    ws = hip.route_workspace(n * H, half, k, dev)
    stream = N.stream(dev)

    def gemm():
        torch.matmul(x, w_t, out=scores)

    def route():
        N.call("glsdm_route", N.ptr(scores), N.BF16, n * H, half, k, N.TIE_HIGHEST, N.ptr(index),
               N.ptr(weights), N.ptr(ws), 0 if ws is None else ws.numel(), stream)

    def timed(fn):
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    ms_gemm, ms_route = timed(gemm), timed(route)
    flops = 2 * n * d_model * H * L
    return {"flops_per_call": flops, "gemm_ms_per_call": round(ms_gemm, 5),
            "achieved_TFLOPs": round(flops / (ms_gemm * 1e-3) / 1e12, 1),
            "frac": round(flops / (ms_gemm * 1e-3) / MFMA_BF16_PEAK, 4),
            "route_ms_per_call": round(ms_route, 5),
            "shape": f"[{n}, {d_model}] x [{d_model}, {H * L}] bf16 -> bf16 scores, route k={k} over {n * H} rows",
            "note": "the reference's router.q Linear (hipBLASLt) and the route of its bf16 output, per epoch"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, budget_s=20.0):
    """The reference's CPU path, timed on the host cores: ``oracle/torch_oracle``,
    the reference's own torch op sequence (factor scores q @ K^T per head; route
    and read of S/memory/routing.py:10-28; the keyed stable sort, segment_reduce
    and index_copy of S/memory/transactions.py:89-96, a new bank per commit),
    fp32 (the reference's only state dtype) on the workload's bf16-rounded
    inputs, all B requests, torch's intra-op threads.  One warmup epoch, then
    whole epochs until ``budget_s``; tokens/s = B*C / median epoch time
    (P/scripts/benchmark_memory.py:82-97 takes the median too)."""
    from oracle import torch_oracle
    keys, bank, qr, qw, delta = make_inputs(cfg)
    B, C, H, half, D, k = (cfg[x] for x in ("B", "C", "H", "half", "D", "k"))
    epochs = cfg["T"] // C
    values = bank.float().unsqueeze(0).expand(B, -1, -1, -1).contiguous()     # per-request replicas
    kf = keys.float()
    pos = torch.arange(C).view(1, C, 1, 1).expand(B, C, H, k).reshape(-1)

    def epoch(e, values):
        sl = slice(e * C, (e + 1) * C)
        _, idx, w = torch_oracle.routed_read(values, torch.einsum("bthe,hle->bthl", qr[:, sl].float(), kf), k)
        widx, _ = torch_oracle.route(torch.einsum("bthe,hle->bthl", qw[:, sl].float(), kf), k)
        addr = torch_oracle.absolute_addresses(values, widx).reshape(-1)
        new = torch_oracle.commit(values.reshape(-1, D), addr, delta[:, sl].float().reshape(-1, D), addr * C + pos)
        return new.view_as(values)

    values = epoch(0, values)                                                   # warmup
    times, e, t0 = [], 1, time.perf_counter()
    while len(times) < 2 or time.perf_counter() - t0 < budget_s:
        t = time.perf_counter()
        values = epoch(e % epochs, values)
        times.append(time.perf_counter() - t)
        e += 1
    med = statistics.median(times)
    return {"value": B * C / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"{len(times)} whole epochs of the workload after 1 warmup (B={B} requests x {C} tokens "
                      f"each; score + route + read + write route + commit with a new bank per commit), "
                      f"median {med:.3f} s per epoch; oracle/torch_oracle: the reference's torch op sequence, "
                      f"fp32, {torch.get_num_threads()} threads"}


# the physical stack (S/layers/stack.py) with
# 16 distinct layers alternating local (window 512, 16 heads) and global, d_model 1024,
# head_dim 64 (so 16 memory heads of value dim 64), top-k 16, 512-token clock
STACK = dict(arch_type="gl_sdm", vocab_size=32000, hidden_size=1024, head_dim=64, num_hidden_layers=16,
             dtype="bfloat16", gl_layer_pattern=["local", "global"], gl_reads=16, gl_writes=16,
             gl_chunk_size=512, gl_local_window=512, gl_memory_backend="hip", residual_dtype="float32")
STACK_CONFIGS = {
    4: dict(STACK, gl_slots=262144, B=4, T=8192),
    # 64 streams of a 2^20-slot bank: bf16 request snapshots (64 x 2 GiB)
    5: dict(STACK, gl_slots=1048576, gl_state_dtype="bfloat16", B=64, prompt=512, decode_steps=4096),
}
MEMORY_CALLS = ("routed_snapshot_read", "commit_proposals")     # + ProposalLog.append (the proposals)


def stack_flops_per_token(cfg):
    """Dense multiply-adds x 2 per token of the stack forward: every Linear once (global
    layers: q, and k/v/beta/decay/proj for the write path), windowed attention
    (QK^T and AV over at most `window` keys) and the vocabulary head."""
    d, V, W = cfg["hidden_size"], cfg["vocab_size"], cfg["gl_local_window"]
    inner = cfg.get("intermediate_size") or 4 * d
    H = d // cfg["head_dim"]
    L = 2 * int(round(cfg["gl_slots"] ** 0.5))
    mlp = 3 * d * inner
    local = 5 * d * d + mlp + 2 * W * d
    glob = 2 * d * H * L + 2 * d * d + 2 * d * H + mlp
    pattern = cfg["gl_layer_pattern"]
    n = cfg["num_hidden_layers"]
    n_global = sum(pattern[i % len(pattern)] == "global" for i in range(n))
    return 2 * ((n - n_global) * local + n_global * glob + d * V)


class CallTimer:
    """HIP events around the memory operator's entry points (torch's current stream,
    the stream the library launches on)."""

    def __init__(self, module, names):
        self.module, self.names, self.orig, self.events = module, names, {}, {}

    def __enter__(self):
        for n in self.names:
            f = getattr(self.module, n)
            self.orig[n] = f

            def wrapped(*a, _f=f, _n=n, **kw):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                out = _f(*a, **kw)
                e.record()
                self.events.setdefault(_n, []).append((s, e))
                return out
            setattr(self.module, n, wrapped)
        return self

    def __exit__(self, *exc):
        for n, f in self.orig.items():
            setattr(self.module, n, f)

    def totals(self, per):
        torch.cuda.synchronize()
        return {n: round(sum(a.elapsed_time(b) for a, b in v) / per, 4) for n, v in self.events.items()}


def stack_model(cfg, dev):
    from glsdm.model import create_model
    model_cfg = {k: v for k, v in cfg.items() if k not in ("B", "T", "prompt", "decode_steps")}
    torch.manual_seed(0)
    with torch.device(dev):
        model = create_model(model_cfg)     # random init, drawn on the device
    return model.eval()


def device_copy_rate(dev, nbytes=1 << 30, reps=10):
    """Bytes moved per second (read + write) by a 1 GiB device-to-device copy: the
    practical streaming ceiling that the HBM roofline fractions are read against."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    rate = 2 * nbytes / (a.elapsed_time(b) / reps * 1e-3)
    del src, dst
    return rate


def full_stack_rate(dev, steps=2, warmup=1):
    """Config 4's full-stack forward, reported beside the
    headline memory-op line: tokens/s of Model.prefill on the whole batch."""
    cfg = STACK_CONFIGS[4]
    model = stack_model(cfg, dev)
    inputs = torch.randint(cfg["vocab_size"], (cfg["B"], cfg["T"]), generator=torch.Generator("cpu").manual_seed(0))
    inputs = inputs.to(dev)
    for _ in range(warmup):
        model.prefill(inputs)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        model.prefill(inputs)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    del model
    torch.cuda.empty_cache()
    return {"value": round(cfg["B"] * cfg["T"] / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 3),
            "steps": steps, "warmup": warmup,
            "workload": "BASELINE configs[3]: 16-layer stack (8 local window-512 / 8 global, M=262144, k=16), "
                        "d_model 1024, B=4, T=8192, bf16 random init; one step = Model.prefill of the batch "
                        "(bench.py --config 4 reports it alone with its breakdown)"}


def stack_main(args, dev):
    from glsdm.memory.backends import hip
    cfg = STACK_CONFIGS[args.config]
    model = stack_model(cfg, dev)
    g = torch.Generator("cpu").manual_seed(0)
    B = cfg["B"]
    per_token = stack_flops_per_token(cfg)
    workload = (f"GL-SDM stack, BASELINE configs[{args.config - 1}]: 16 layers (local window 512 / global) "
                f"d_model 1024, 16 heads, M={cfg['gl_slots']}, value dim 1024 (16 x 64), top-k 16, clock 512, "
                f"vocab 32000, bf16 weights, {'fp32' if cfg.get('gl_state_dtype', 'float32') == 'float32' else 'bf16'}"
                " request snapshots, random init")
    base = {"metric": "GL-SDM mem-op tokens/s + % HBM roofline (read+commit); full-stack tokens/s",
            "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic (uniform random token ids, seeded; random-init weights)"}
    if args.config == 4:
        T = cfg["T"]
        inputs = torch.randint(cfg["vocab_size"], (B, T), generator=g).to(dev)
        for _ in range(args.warmup):
            model.prefill(inputs)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            model.prefill(inputs)
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps
        from glsdm.memory import ProposalLog
        with CallTimer(hip, MEMORY_CALLS) as timer, CallTimer(ProposalLog, ("append",)) as appends:
            model.prefill(inputs)
        mem = {**timer.totals(1), **{"proposal_append": v for v in appends.totals(1).values()}}
        flops = per_token * B * T
        result = dict(base, value=round(B * T / (ms * 1e-3), 1), steps=args.steps, warmup=args.warmup,
                      ms_per_step=round(ms, 3),
                      config={"workload": workload + "; one step = Model.prefill of the whole batch (new request "
                              "caches, 16 chunks, 16 commits)", "B": B, "T": T, "layers": 16, "d_model": 1024,
                              "slots": cfg["gl_slots"], "top_k": 16, "parallelism": "single GPU"},
                      roofline={"kernel": "whole forward (hipBLASLt GEMMs dominate)", "bound": "mfma",
                                "achieved": round(flops / (ms * 1e-3) / 1e12, 1), "peak": MFMA_BF16_PEAK / 1e12,
                                "unit": "TFLOP/s", "frac": round(flops / (ms * 1e-3) / MFMA_BF16_PEAK, 4),
                                "traffic": None, "flops_per_step": flops},
                      memory_op_ms_per_step=mem, memory_op_share=round(sum(mem.values()) / ms, 4))
        print(json.dumps(result))
        return
    # config 5: prompt prefill, then one-token decode steps with a commit every 512 tokens
    steps = args.decode_steps or cfg["decode_steps"]
    decode = decode_run(model, cfg, dev, steps)
    p50 = decode["p50_ms"]
    result = dict(base, value=round(B / (p50 * 1e-3), 1), steps=steps, warmup=0, ms_per_step=p50,
                  higher_is_better=True,
                  config={"workload": workload + f"; {B} streams, {cfg['prompt']}-token prompt, {steps} decode "
                          "steps of one token per stream, commit every 512 steps", "B": B, "prompt": cfg["prompt"],
                          "decode_steps": steps, "slots": cfg["gl_slots"], "parallelism": "single GPU"},
                  decode=decode, roofline=None)
    print(json.dumps(result))


def decode_record(dev):
    """Config 5 decode, reported beside the headline line:
    all of the config's decode steps (bench.py --config 5 reports it alone)."""
    cfg = STACK_CONFIGS[5]
    model = stack_model(cfg, dev)
    out = decode_run(model, cfg, dev, cfg["decode_steps"])
    del model
    torch.cuda.empty_cache()
    out["workload"] = ("BASELINE configs[4]: 16-layer stack (8 global, M=2^20, k=16, bf16 request snapshots), "
                       "d_model 1024, 64 streams, 512-token prompt then 4096 one-token decode steps, a commit "
                       "every 512; bf16 random init")
    return out


def decode_run(model, cfg, dev, steps):
    """Config 5's decode: the prompt's prefill (one commit), then ``steps`` one-token
    decode steps of every stream (a commit every 512 tokens); per-step times from
    HIP events on the current stream, so each step's host work and launches are in it."""
    B, P = cfg["B"], cfg["prompt"]
    g = torch.Generator("cpu").manual_seed(0)
    prompt = torch.randint(cfg["vocab_size"], (B, P), generator=g).to(dev)
    tokens = torch.randint(cfg["vocab_size"], (B, steps), generator=g).to(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _, cache = model.prefill(prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    commit_steps = []
    for s in range(steps):
        marks[s].record()
        model.decode(tokens[:, s:s + 1], cache)
        if cache[0].tokens % cfg["gl_chunk_size"] == 0:
            commit_steps.append(s)
    marks[steps].record()
    torch.cuda.synchronize()
    dur = [marks[s].elapsed_time(marks[s + 1]) for s in range(steps)]
    in_commit = set(commit_steps)
    plain = sorted(d for s, d in enumerate(dur) if s not in in_commit)
    commits = [dur[s] for s in commit_steps]
    n_global = sum(p == "global" for p in cfg["gl_layer_pattern"]) * cfg["num_hidden_layers"] \
        // len(cfg["gl_layer_pattern"])
    heads = cfg["hidden_size"] // cfg["head_dim"]
    return {"streams": B, "prompt": P, "decode_steps": steps,
            "p50_ms": round(statistics.median(dur), 4), "p50_ms_without_commit": round(statistics.median(plain), 4),
            "p90_ms": round(sorted(dur)[int(0.9 * steps)], 4),
            "tokens_per_s_at_p50": round(B / (statistics.median(dur) * 1e-3), 1),
            "commit_steps": len(commits),
            "commit_step_ms_mean": round(statistics.mean(commits), 3) if commits else None,
            "commit_step_ms_max": round(max(commits), 3) if commits else None,
            "commit_entries": B * cfg["gl_chunk_size"] * n_global * heads * cfg["gl_writes"],
            "prefill_s": round(prefill_s, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, choices=(1, 2, 3, 4, 5), default=2,
                    help="BASELINE.json configs[config-1]; 2 (the headline) is the default; 4 and 5 run the "
                         "layer stack (full forward / decode)")
    ap.add_argument("--decode-steps", type=int, default=None,
                    help="config 5: decode steps (default 4096, the config's)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--schedule", choices=("auto", "serial", "overlap"), default="auto",
                    help="overlap: routes of later epochs on a second stream while the memory stream reads and "
                         "commits; serial: every call on one stream; auto (default): overlap when a step has "
                         "more than one epoch (with one, the next step's routes wait for this step's commit "
                         "anyway, and the cross-stream waits only add latency)")
    ap.add_argument("--compare-schedules", action="store_true",
                    help="also time the other schedule (reported as ms_per_step_other_schedule)")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-full-stack", action="store_true",
                    help="skip the config-4 full-stack forward reported beside the headline line")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the config-5 decode record reported beside the headline line")
    ap.add_argument("--backward", action="store_true",
                    help="also run the read's backward every epoch: weights' and factor scores' gradients, and "
                         "the bank rows' gradient folded into the learned [H, S, D] bank (reported alongside; "
                         "not the BASELINE protocol)")
    ap.add_argument("--bank", choices=("dense", "overlay"), default="dense",
                    help="dense: the per-request replicated bank (default); overlay: one shared base plus each "
                         "request's touched rows, a fresh batch snapshot per step (map reset instead of a clone)")
    ap.add_argument("--write-path", choices=("deltas", "proposals", "proposals-materialised"), default="deltas",
                    help="deltas: synthetic deltas (the BASELINE protocol, default); proposals: the stack's write "
                         "path with the fused proposal commit; proposals-materialised: the same work with "
                         "gathered rows and stored fp32 deltas")
    ap.add_argument("--route-parts", type=int, default=1,
                    help="overlap schedule: launch each route call over this many request ranges")
    ap.add_argument("--split-commit", action="store_true",
                    help="overlap schedule: sort each epoch's write entries on the route stream "
                         "(glsdm_commit_prepare) and apply them on the memory stream (glsdm_commit_apply); "
                         "the serial pass keeps the one-call glsdm_commit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed region, copy 256 MiB device-to-device 3 times (a kernel of known "
                         "traffic for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the operator shards by request/head with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    if args.config in STACK_CONFIGS:
        stack_main(args, dev)
        return
    cfg = CONFIGS[args.config]
    pipe = Pipeline(cfg, dev, args.write_path, args.backward, args.bank == "overlay", args.split_commit,
                    args.route_parts)
    if args.schedule == "auto":
        args.schedule = "overlap" if pipe.epochs > 1 else "serial"
    unique = pipe.unique_rows()
    run = pipe.step if args.schedule == "overlap" else pipe.step_serial
    other = pipe.step_serial if args.schedule == "overlap" else pipe.step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    read_choice = None
    if args.schedule == "overlap":
        # Which read runs beside the route stream: the wide read (several route entries
        # per lane group in flight) is faster alone, but where its waves leave a SIMD no
        # room for a wave of the 248-VGPR fused route kernel the two streams run nearly in
        # turn (config 2: 0.92 vs 0.76 ms per step); the narrow read fits beside it.  The
        # split-path routes of other shapes fit beside either.  Chosen by timing both
        # (untimed: the best of 3 windows of 5 steps each).
        read_choice = {}
        for entry in ("glsdm_read_narrow", "glsdm_read"):
            pipe.read_entry = entry
            best = None
            for _ in range(3):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                a.record()
                for _ in range(5):
                    run()
                b.record()
                torch.cuda.synchronize()
                t = a.elapsed_time(b) / 5
                best = t if best is None else min(best, t)
            read_choice[entry] = round(best, 4)
        pipe.read_entry = min(read_choice, key=read_choice.get)
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()

    # instrumented pass: events around every call, to find the dominant call
    pipe.timers = {}
    for _ in range(2):
        run()
    torch.cuda.synchronize()
    pre = {n: statistics.mean(a.elapsed_time(b) for a, b in v) * len(v) for n, v in pipe.timers.items()}
    # the metric's roofline term is the HBM roofline of read + commit: `roofline` reports
    # the larger of those two calls; the fused scoring + route (MFMA, selection-bound) is
    # reported beside it in `scoring_mfma`
    dominant = pipe.only = max(("read", "commit"), key=lambda n: pre.get(n, 0.0))

    ms_other = None
    if args.compare_schedules:
        # the other schedule, timed the same way (reported for comparison)
        for _ in range(args.warmup):
            other()
        pipe.timers = {}
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            other()
        end.record()
        torch.cuda.synchronize()
        ms_other = start.elapsed_time(end) / args.steps
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()

    # timed region: events only around the dominant call's launches
    pipe.timers = {}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        run()
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_step = total_ms / args.steps
    dominant_ms = {n: statistics.mean(a.elapsed_time(b) for a, b in v) for n, v in pipe.timers.items()}
    # all calls, from a second instrumented pass on one stream: each call's own
    # duration without the other stream's kernels beside it (reported, and the
    # isolated roofline; not the timed region's)
    pipe.timers, pipe.only = {}, None
    for _ in range(3):
        pipe.step_serial()
    torch.cuda.synchronize()
    per_call = {n: statistics.mean(a.elapsed_time(b) for a, b in v) for n, v in pipe.timers.items()}
    calls = {n: len(v) // 3 for n, v in pipe.timers.items()}

    tokens = cfg["B"] * cfg["T"]
    read_b, read_kernel_b, commit_b, other_b = algorithmic_bytes(cfg, unique, args.write_path)
    epochs = pipe.epochs
    alg_total = epochs * (read_b + other_b) + sum(commit_b)
    # dominant call's duration: in the timed region (the schedule as run, `roofline`)
    # and alone on one stream (the serial pass, `roofline_isolated`)
    isolated_ms = per_call[dominant]
    t_timed = dominant_ms[dominant]
    if dominant == "read":
        bytes_launch, t_launch = read_kernel_b, t_timed * 1e-3
        roof = {"kernel": f"read_kernel ({pipe.read_entry})", "bound": "hbm", "unit": "GB/s", "peak": HBM_PEAK / 1e9}
        achieved = bytes_launch / t_launch / 1e9
    elif dominant == "commit":
        bytes_launch, t_launch = statistics.mean(commit_b), t_timed * 1e-3
        entry = "glsdm_commit_proposals" if args.write_path == "proposals" else "glsdm_commit"
        steps = ("tile bucketing + bucket sort + segment" if pipe.rows >= 1 << 16
                 else "prep + pack + LSD passes + segment")
        one_call = f"{entry} ({steps})"
        if pipe.split_commit and args.schedule == "overlap":
            # the timed launch is the apply; the sort (which reads the addresses) ran on the route stream
            bytes_launch -= pipe.E * 8
            entry, steps = "glsdm_commit_apply", "segment; sort by glsdm_commit_prepare on the route stream"
        roof = {"kernel": f"{entry} ({steps})", "bound": "hbm",
                "unit": "GB/s",
                "peak": HBM_PEAK / 1e9}
        achieved = bytes_launch / t_launch / 1e9
    else:
        # fused scoring + selection: the MFMA contraction is the only dense work
        flops = 2 * cfg["B"] * cfg["C"] * cfg["H"] * 2 * cfg["half"] * cfg["dk"]
        t_launch = per_call["score_route"] * 1e-3
        roof = {"kernel": "score_route_kernel (glsdm_score_route)", "bound": "mfma", "unit": "TFLOP/s",
                "peak": MFMA_BF16_PEAK / 1e12}
        achieved = flops / t_launch / 1e12
        bytes_launch = None
    traffic = TRAFFIC_PER_LAUNCH.get(dominant) if args.config == 2 and args.write_path == "deltas" else None
    roof.update({"achieved": round(achieved, 1), "frac": round(achieved / roof["peak"], 4),
                 "traffic": None if traffic is None else int(traffic),
                 "ms_per_launch": round(t_timed, 5)})
    roof_iso = None
    if bytes_launch is not None:
        # the serial pass runs the one-call commit: all of its bytes
        b_iso = statistics.mean(commit_b) if dominant == "commit" else bytes_launch
        a_iso = b_iso / (isolated_ms * 1e-3) / 1e9
        roof_iso = {"kernel": one_call if dominant == "commit" else roof["kernel"],
                    "achieved": round(a_iso, 1), "frac": round(a_iso / roof["peak"], 4),
                    "ms_per_launch": round(isolated_ms, 5),
                    "note": "the same call alone on one stream (serial pass); `roofline` is measured in the "
                            "timed region, where the route stream's kernels run beside it"}

    scoring_flops = 2 * cfg["B"] * cfg["C"] * cfg["H"] * 2 * cfg["half"] * cfg["dk"]
    memory_calls = ("read", "commit", "write_read", "proposal_error", "gather", "proposal_delta")
    rc_time = sum(per_call[n] * calls[n] for n in memory_calls if n in per_call) * 1e-3
    result = {
        "metric": "GL-SDM mem-op tokens/s + % HBM roofline (read+commit); full-stack tokens/s",
        "value": round(tokens / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "schedule": args.schedule,
        "split_commit": pipe.split_commit and args.schedule == "overlap",
        "route_parts": pipe.route_parts if args.schedule == "overlap" else 1,
        "read_entry": pipe.read_entry,
        "read_choice_ms_per_step": read_choice,
        "ms_per_step_other_schedule": None if ms_other is None else round(ms_other, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg["dtype"] == torch.bfloat16 else "f32",
        "data": "synthetic (seeded CPU generator, BASELINE.json config protocol)",
        "config": {"workload": f"memory op, BASELINE configs[{args.config - 1}]: B={cfg['B']} T={cfg['T']} "
                               f"({epochs} epochs of {cfg['C']}) H={cfg['H']} M={cfg['half'] ** 2} dk={cfg['dk']} "
                               f"D={cfg['D']} k={cfg['k']} {'bf16' if cfg['dtype'] == torch.bfloat16 else 'fp32'}"
                               f"{' Zipf-skewed' if cfg['skew'] else ''}, fused score-route + read + fused "
                               "score-route-keys + " + WRITE_PATHS[args.write_path]
                               + (" + read backward (route, weights, bank rows)" if args.backward else "")
                               + (" on an overlay bank (shared base + touched rows)" if args.bank == "overlay" else ""),
                   "B": cfg["B"], "T": cfg["T"], "chunk": cfg["C"], "heads": cfg["H"],
                   "slots": cfg["half"] ** 2, "key_dim": cfg["dk"], "value_dim": cfg["D"], "top_k": cfg["k"],
                   "write_path": args.write_path, "backward": args.backward, "bank": args.bank,
                   "parallelism": "single GPU"},
        "roofline": roof,
        "roofline_isolated": roof_iso,
        "read_commit_hbm": {"bytes_per_step": alg_total, "seconds_per_step": rc_time,
                            "achieved_GBps": round(alg_total / rc_time / 1e9, 1),
                            "frac": round(alg_total / rc_time / HBM_PEAK, 4),
                            "op_frac": round(alg_total / (ms_step * 1e-3) / HBM_PEAK, 4),
                            "note": "frac: over the read and commit calls timed alone (serial pass); op_frac: "
                                    "over the whole step as run"},
        "scoring_mfma": {"flops_per_call": scoring_flops, "ms_per_call": round(per_call["score_route"], 5),
                         "frac": round(scoring_flops / (per_call["score_route"] * 1e-3) / MFMA_BF16_PEAK, 4),
                         "note": "fused kernel: MFMA scoring + exact top-k selection in one launch"},
        "ms_per_call": {n: round(v, 5) for n, v in per_call.items()},
        "calls_per_step": calls,
        "unique_rows_per_epoch": unique,
    }
    if args.config == 2 and args.write_path == "deltas" and not args.backward and args.bank == "dense":
        result["literal_scoring_mfma"] = literal_scoring(cfg, dev)
    copy = device_copy_rate(dev)
    result["hbm_calibration"] = {
        "device_copy_GBps": round(copy / 1e9, 1), "copy_frac_of_peak": round(copy / HBM_PEAK, 4),
        "roofline_achieved_frac_of_copy": round(roof["achieved"] * 1e9 / copy, 4),
        "read_commit_frac_of_copy": round(alg_total / rc_time / copy, 4),
        "note": "1 GiB device-to-device copy (read + write bytes / time): the streaming rate this MI355X "
                "sustains; the fractions above are of the 8 TB/s nominal peak"}
    headline = args.config == 2 and args.write_path == "deltas" and not args.backward and args.bank == "dense"
    if headline and not args.no_full_stack:
        result["full_stack"] = full_stack_rate(dev)
    if headline and not args.no_decode:
        del pipe
        torch.cuda.empty_cache()
        result["decode"] = decode_record(dev)
    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_calibration_bytes"] = src.numel()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_budget)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
