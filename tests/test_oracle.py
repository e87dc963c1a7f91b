"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is independent of the oracle's own formulation: literal known
answers from the reference tests, brute force over every slot, a lexicographic
sort with explicit key tuples, the dense one-hot equations, float64 closed
forms, and invariants.  The two restatements (torch ops and scalar C) must
also agree bit for bit on indices and commits.
"""
import itertools
import math

import pytest
import torch

from oracle import c_oracle, torch_oracle
from _util import known_answers, route_scores, gen

ROUTES = [("torch", torch_oracle.route), ("c", c_oracle.route)]


@pytest.mark.parametrize("name,route", ROUTES)
def test_route_known_answers(name, route):
    ka = known_answers()
    for case in ("route_highest_zero_scores", "route_lowest_zero_scores"):
        c = ka[case]
        idx, w = route(torch.full(c["scores_shape"], c["scores_fill"]), c["width"], c["tie"])
        assert (idx == torch.tensor(c["expect_index_row"])).all(), case
        assert torch.equal(w, torch.full_like(w, c["expect_weight"])), case


@pytest.mark.parametrize("name,route", ROUTES)
@pytest.mark.parametrize("half,count", [(4, 2), (3, 5), (8, 64), (64, 8)])
def test_route_lowest_signed_zero_known_answer(name, route, half, count):
    s = torch.randn(3, 2, 2 * half, generator=gen(13))
    s[0].zero_()
    s[0, :, 0] = -0.0
    idx, w = route(s, count, "lowest")
    assert idx[0, 0].tolist() == list(range(count))
    assert (idx[..., 1:] > idx[..., :-1]).all()


def _lexicographic_route(row, width, tie):
    """Route one row by explicit tuple keys: (score, index) with the tie rule."""
    half = len(row) // 2
    sign = 1 if tie == "highest" else -1

    def top(values, k):
        order = sorted(range(len(values)), key=lambda i: (values[i], sign * i), reverse=True)
        return order[:k]

    k = min(width, half)
    f0, f1 = row[:half], row[half:]
    p0, p1 = top(f0, k), top(f1, k)
    cands = [(torch.tensor(f0[i], dtype=torch.float32) + torch.tensor(f1[j], dtype=torch.float32)).item()
             for i in p0 for j in p1]
    slots = [i * half + j for i in p0 for j in p1]
    order = sorted(range(len(slots)), key=lambda c: (cands[c], sign * slots[c]), reverse=True)[:width]
    return sorted(slots[c] for c in order)


def _clean(row):
    # tuple sorting sees -0.0 == 0.0 like torch; keep values as python floats
    return [float(x) for x in row]


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("kind", ["randn", "floor", "zeros", "signed_zero", "bf16"])
@pytest.mark.parametrize("half,width", [(4, 4), (3, 5), (8, 3), (6, 8), (16, 16)])
def test_route_matches_lexicographic_keys(tie, kind, half, width):
    s = route_scores(kind, (6, 2 * half), seed=half * 31 + width)
    for name, route in ROUTES:
        idx, _ = route(s, width, tie)
        for r in range(s.shape[0]):
            assert idx[r].tolist() == _lexicographic_route(_clean(s[r]), width, tie), (name, r)


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("half,width", [(5, 3), (8, 8), (12, 16), (3, 9)])
def test_route_brute_force_over_all_slots(tie, half, width):
    """On tie-free inputs the kk x kk grid holds the dense top-width of all half**2 slots."""
    s = route_scores("randn", (20, 2 * half), seed=7 + half)
    for name, route in ROUTES:
        idx, w = route(s, width, tie)
        for r in range(s.shape[0]):
            row = s[r].double()
            dense = [(float(row[i] + row[half + j]), i * half + j) for i in range(half) for j in range(half)]
            best = sorted(dense, reverse=True)[:width]
            assert idx[r].tolist() == sorted(a for _, a in best), (name, r)
            z = torch.tensor([float(s[r, a // half]) + float(s[r, half + a % half]) for a in idx[r].tolist()],
                             dtype=torch.float64)
            torch.testing.assert_close(w[r].double(), torch.softmax(z, 0), atol=2e-7, rtol=2e-6)


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("kind", ["randn", "bf16", "mixed", "floor"])
@pytest.mark.parametrize("half,width", [(64, 8), (256, 16), (32, 32), (10, 64), (128, 1)])
def test_torch_and_c_oracles_agree(tie, kind, half, width):
    if width > half * half:
        pytest.skip("width above slots")
    s = route_scores(kind, (3, 17, 2, 2 * half), seed=half + width)
    a_idx, a_w = torch_oracle.route(s, width, tie)
    b_idx, b_w = c_oracle.route(s, width, tie)
    assert torch.equal(a_idx, b_idx)
    torch.testing.assert_close(a_w, b_w, atol=2e-7, rtol=2e-6, equal_nan=True)
    assert (a_idx[..., 1:] > a_idx[..., :-1]).all()
    finite = torch.isfinite(a_w).all(-1)
    torch.testing.assert_close(a_w[finite].sum(-1), torch.ones_like(a_w[finite].sum(-1)), atol=1e-6, rtol=0)


def test_read_closed_form_and_dense():
    g = gen(3)
    B, H, S, D, T, k = 2, 2, 16, 37, 5, 3
    mem = torch.randn(B, H, S, D, generator=g)
    idx = torch.stack([torch.randperm(S, generator=g)[:k].sort().values for _ in range(B * T * H)]).view(B, T, H, k)
    w = torch.randn(B, T, H, k, generator=g).softmax(-1)
    a = torch_oracle.read(mem, idx, w)
    b = torch_oracle.read(mem, idx, w, dense=True)
    c = c_oracle.read(mem, idx, w)
    exact = torch.einsum("bthk,bthkd->bthd", w.double(),
                         mem.double()[torch.arange(B)[:, None, None, None], torch.arange(H)[None, None, :, None], idx])
    for x in (a, b, c):
        torch.testing.assert_close(x.double(), exact, atol=1e-6, rtol=1e-5)


def test_commit_known_answers():
    ka = known_answers()
    c = ka["commit_stable_collisions"]
    flat = torch.zeros(c["rows"], 1)
    addr, delta = torch.tensor(c["addresses"]), torch.tensor(c["deltas"])[:, None]
    assert torch_oracle.commit(flat, addr, delta).flatten().tolist() == c["expect"]
    assert c_oracle.commit(flat, addr, delta)[0].flatten().tolist() == c["expect"]
    c = ka["commit_keyed_arrival_order"]
    addr, delta, keys = (torch.tensor(c[k]) for k in ("addresses", "deltas", "keys"))
    perm = torch.tensor(c["permutation"])
    flat = torch.zeros(c["rows"], 1)
    for fn in (torch_oracle.commit, lambda *a: c_oracle.commit(*a)[0]):
        x = fn(flat, addr, delta[:, None], keys)
        y = fn(flat, addr[perm], delta[perm][:, None], keys[perm])
        assert torch.equal(x, y) and x[3, 0].item() == c["expect_row3"]
    c = ka["commit_unrelated_addresses"]
    flat = torch.zeros(c["rows"], 1)
    addr, delta = torch.tensor(c["addresses"]), torch.tensor(c["deltas"])[:, None]
    assert torch_oracle.commit(flat, addr, delta)[3, 0].item() == c["expect_row3"]
    assert c_oracle.commit(flat, addr, delta)[0][3, 0].item() == c["expect_row3"]


@pytest.mark.parametrize("keyed", [False, True])
def test_commit_matches_dense_and_c(keyed):
    g = gen(5)
    rows, D, E = 50, 7, 400
    flat = torch.randn(rows, D, generator=g)
    addr = torch.randint(0, rows, (E,), generator=g)
    delta = torch.randn(E, D, generator=g)
    keys = addr * 1000 + torch.randperm(E, generator=g) if keyed else None
    a = torch_oracle.commit(flat, addr, delta, keys)
    b, unique = c_oracle.commit(flat, addr, delta, keys)
    assert torch.equal(a, b)
    assert unique == addr.unique().numel()
    torch.testing.assert_close(a, torch_oracle.commit_dense(flat, addr, delta), atol=1e-5, rtol=1e-5)
    untouched = torch.ones(rows, dtype=torch.bool)
    untouched[addr] = False
    assert torch.equal(a[untouched], flat[untouched])


def test_commit_bf16_rounds_once():
    g = gen(9)
    flat = torch.randn(20, 8, generator=g).bfloat16()
    addr = torch.randint(0, 20, (64,), generator=g)
    delta = torch.randn(64, 8, generator=g) * 0.02
    out = torch_oracle.commit_bf16(flat, addr, delta)
    ref = torch_oracle.commit(flat.float(), addr, delta)
    assert out.dtype == torch.bfloat16 and torch.equal(out, ref.bfloat16())


def test_planted_mistakes_are_caught():
    """A plausible slip in the oracle (wrong tie direction, tree-order commit) fails the pins."""
    ka = known_answers()["route_highest_zero_scores"]
    wrong, _ = torch_oracle.route(torch.zeros(ka["scores_shape"]), ka["width"], "lowest")
    assert wrong[0, 0].tolist() != ka["expect_index_row"]
    c = known_answers()["commit_stable_collisions"]
    d = torch.tensor(c["deltas"])
    pairwise = (d[0] + (d[2] + d[3])).item()   # a tree reduction of address 0
    assert pairwise != c["expect"][0]


def _proposal_operands(seed, lead=(2, 3), H=2, k=4, D=5):
    g = gen(seed)
    rows = torch.randn(*lead, H, k, D, generator=g)
    w = torch.randn(*lead, H, k, generator=g).softmax(-1)
    pred = torch.randn(*lead, H, D, generator=g)
    tgt = torch.randn(*lead, H, D, generator=g)
    beta = torch.rand(*lead, H, 1, generator=g)
    ld = -torch.rand(*lead, H, 1, generator=g)
    mass = torch.rand(*lead, generator=g)
    return rows, w, pred, tgt, beta, ld, mass


def test_proposal_delta_closed_form():
    rows, w, pred, tgt, beta, ld, mass = _proposal_operands(4)
    out = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, mass)
    gd = ld.double().exp()
    ref = mass.double()[..., None, None, None] * ((gd[..., None] - 1) * rows.double()
          + w.double()[..., None] * (beta.double() * (tgt.double() - gd * pred.double()))[..., None, :])
    torch.testing.assert_close(out.double(), ref, atol=1e-6, rtol=1e-5)


def test_proposal_delta_elementwise_rounding():
    """Each element is the fp32 result of the reference's five roundings in order
    (scalar numpy float32 arithmetic, one rounding per operation, no FMA)."""
    np = pytest.importorskip("numpy")
    rows, w, pred, tgt, beta, ld, mass = _proposal_operands(5, lead=(3,), H=2, k=3, D=4)
    g = ld.exp()
    out = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, mass, decay=g)
    f = np.float32
    for b in range(3):
        for h in range(2):
            gg = f(g[b, h, 0].item())
            for j in range(3):
                for d in range(4):
                    err = f(beta[b, h, 0].item()) * (f(tgt[b, h, d].item()) - gg * f(pred[b, h, d].item()))
                    x = f(mass[b].item()) * ((gg - f(1)) * f(rows[b, h, j, d].item()) + f(w[b, h, j].item()) * err)
                    assert np.float32(out[b, h, j, d].item()) == x


def test_proposal_delta_rule_invariants():
    """The delta rule's fixed points: a single full-weight write with beta = 1
    whose prediction is the written row moves the row to the target; beta = 0
    only decays it (row + delta = decay * row); mass 0 writes nothing."""
    rows, w, pred, tgt, beta, ld, mass = _proposal_operands(6, k=1)
    w = torch.ones_like(w)
    one = torch.ones_like(beta)
    new = rows + torch_oracle.proposal_delta(rows, w, rows[..., 0, :], tgt, one, ld, torch.ones_like(mass))
    torch.testing.assert_close(new[..., 0, :], tgt, atol=1e-6, rtol=1e-5)
    new = rows + torch_oracle.proposal_delta(rows, w, pred, tgt, torch.zeros_like(beta), ld, torch.ones_like(mass))
    torch.testing.assert_close(new, ld.exp()[..., None] * rows, atol=1e-6, rtol=1e-5)
    zero = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, torch.zeros_like(mass))
    assert zero.abs().max().item() == 0.0


# ---------------------------------------------------------------- scoring

def _score_operands(seed, B=2, T=5, H=3, L=12, dk=64):
    g = gen(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1).bfloat16().float()
    k = torch.nn.functional.normalize(torch.randn(H, L, dk, generator=g), dim=-1).bfloat16().float()
    return q, k


def _score_f64(q, k):
    return torch.einsum("bthe,hce->bthc", q.double(), k.double())


def test_score_float64_closed_form_and_restatements_agree():
    """oracle_score (C) and torch_oracle.score: bitwise equal to each other
    (scalar C loop vs a sequence of torch fp32 ops), within fp32 rounding of the
    float64 contraction, and every element equal to a numpy float32 scalar loop
    (one rounding per product and per add, e ascending)."""
    np = pytest.importorskip("numpy")
    q, k = _score_operands(21)
    a = c_oracle.score(q, k)
    b = torch_oracle.score(q, k)
    assert torch.equal(a, b)
    torch.testing.assert_close(a.double(), _score_f64(q, k), atol=1e-5, rtol=1e-5)
    f = np.float32
    qn, kn = q.numpy(), k.numpy()
    for (bb, t, h, c) in [(0, 0, 0, 0), (1, 4, 2, 11), (0, 3, 1, 7), (1, 2, 0, 5)]:
        s = f(0)
        for e in range(q.shape[-1]):
            s = f(s + f(qn[bb, t, h, e] * kn[h, c, e]))
        assert np.float32(a[bb, t, h, c].item()) == s


def test_score_planted_mistakes_fail_the_pin():
    """Plausible slips -- another head's sub-keys, a transposed (factor, dim)
    operand, a dropped term -- each fail the float64 closed-form check."""
    q, k = _score_operands(22, L=64, dk=64)
    exact = _score_f64(q, k)

    def close(x):
        return torch.allclose(x.double(), exact, atol=1e-5, rtol=1e-5)

    assert close(c_oracle.score(q, k))
    assert not close(c_oracle.score(q, k.roll(1, 0)))                  # wrong head
    assert not close(c_oracle.score(q, k.transpose(1, 2).contiguous()))  # transposed operand
    dropped = q.clone()
    dropped[..., -1] = 0
    assert not close(c_oracle.score(dropped, k))                        # dropped term


# ---------------------------------------------------------------- token clock

def _token_operands(seed, B=3, H=2, S=67, D=37, K=3, A=2):
    g = gen(seed)
    values = torch.randn(B, H, S, D, generator=g)
    requests = torch.tensor([2, 0])[:A]                     # ACT subset, noncanonical order
    idx = torch.stack([torch.randperm(S, generator=g)[:K] for _ in range(A * H)]).view(A, H, K)
    w = torch.randn(A, H, K, generator=g).softmax(-1)
    tgt = torch.randn(A, H, D, generator=g)
    beta = torch.rand(A, H, 1, generator=g)
    ld = -torch.rand(A, H, 1, generator=g)
    mass = torch.rand(A, generator=g)
    return values, requests, idx, w, tgt, beta, ld, mass


def test_token_addresses_closed_form():
    values, requests, idx, *_ = _token_operands(30)
    B, H, S, _ = values.shape
    addr = torch_oracle.token_addresses(values, requests, idx)
    for a in range(idx.shape[0]):
        for h in range(H):
            for j in range(idx.shape[2]):
                assert addr[a, h, j].item() == (requests[a].item() * H + h) * S + idx[a, h, j].item()


def test_token_read_closed_form_and_dense():
    values, requests, idx, w, *_ = _token_operands(31)
    a = torch_oracle.token_read(values, requests, idx, w)
    b = torch_oracle.token_read(values, requests, idx, w, dense=True)
    rows = values.double()[requests[:, None, None], torch.arange(values.shape[1])[None, :, None], idx]
    exact = (rows * w.double()[..., None]).sum(-2)
    for x in (a, b):
        torch.testing.assert_close(x.double(), exact, atol=5e-7, rtol=2e-6)


def test_token_propose_closed_form():
    values, requests, idx, w, tgt, beta, ld, mass = _token_operands(32)
    addr, delta = torch_oracle.token_propose(values, requests, idx, w, tgt, beta, ld, mass)
    rows = values.double()[requests[:, None, None], torch.arange(values.shape[1])[None, :, None], idx]
    g = ld.double().exp()[..., None]
    pred = (rows * g * w.double()[..., None]).sum(-2)
    err = beta.double() * (tgt.double() - pred)
    exact = mass.double()[:, None, None, None] * (g * rows - rows + w.double()[..., None] * err[..., None, :])
    torch.testing.assert_close(delta.double(), exact.flatten(0, 2), atol=5e-7, rtol=2e-6)
    assert torch.equal(addr, torch_oracle.token_addresses(values, requests, idx).flatten())
    _, dense = torch_oracle.token_propose(values, requests, idx, w, tgt, beta, ld, mass, dense=True)
    torch.testing.assert_close(dense, delta, atol=5e-7, rtol=2e-6)


def test_token_propose_elementwise_rounding():
    """With two routes per head the prediction's sum is one fp32 add, so every
    delta element is the reference's sequence of fp32 roundings exactly."""
    np = pytest.importorskip("numpy")
    values, requests, idx, w, tgt, beta, ld, mass = _token_operands(33, D=4, K=2)
    _, delta = torch_oracle.token_propose(values, requests, idx, w, tgt, beta, ld, mass)
    delta = delta.view(2, 2, 2, 4)
    f = np.float32
    H = values.shape[1]
    for a in range(2):
        for h in range(H):
            gg = f(ld[a, h, 0].exp().item())
            rows = [[f(values[requests[a], h, idx[a, h, j], d].item()) for d in range(4)] for j in range(2)]
            ww = [f(w[a, h, j].item()) for j in range(2)]
            dec = [[f(r * gg) for r in row] for row in rows]
            for d in range(4):
                pred = f(f(dec[0][d] * ww[0]) + f(dec[1][d] * ww[1]))
                err = f(f(beta[a, h, 0].item()) * f(f(tgt[a, h, d].item()) - pred))
                for j in range(2):
                    x = f(f(f(dec[j][d] - rows[j][d]) + f(ww[j] * err)) * f(mass[a].item()))
                    assert np.float32(delta[a, h, j, d].item()) == x


def test_token_propose_rule_invariants_and_stack_form():
    """Fixed points of the token-clock delta rule -- one full-weight write with
    beta = 1 moves the row to the target whatever the decay; beta = 0 only
    decays it; mass 0 writes nothing -- and agreement (within rounding) with
    the stack's proposal_delta given the same prediction."""
    values, requests, idx, w, tgt, beta, ld, mass = _token_operands(34, K=1)
    one_w = torch.ones_like(w)
    rows = values[requests[:, None, None], torch.arange(values.shape[1])[None, :, None], idx]
    _, d = torch_oracle.token_propose(values, requests, idx, one_w, tgt, torch.ones_like(beta), ld,
                                      torch.ones_like(mass))
    torch.testing.assert_close(rows[..., 0, :] + d.view_as(rows)[..., 0, :], tgt, atol=1e-6, rtol=1e-5)
    _, d = torch_oracle.token_propose(values, requests, idx, w, tgt, torch.zeros_like(beta), ld,
                                      torch.ones_like(mass))
    torch.testing.assert_close(rows + d.view_as(rows), ld.exp()[..., None] * rows, atol=1e-6, rtol=1e-5)
    _, d = torch_oracle.token_propose(values, requests, idx, w, tgt, beta, ld, torch.zeros_like(mass))
    assert d.abs().max().item() == 0.0
    values, requests, idx, w, tgt, beta, ld, mass = _token_operands(35, K=4)
    rows = values[requests[:, None, None], torch.arange(values.shape[1])[None, :, None], idx]
    _, d = torch_oracle.token_propose(values, requests, idx, w, tgt, beta, ld, mass)
    pred = torch_oracle.token_read(values, requests, idx, w)
    stack = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, mass)
    torch.testing.assert_close(d.view_as(stack), stack, atol=1e-6, rtol=1e-5)
