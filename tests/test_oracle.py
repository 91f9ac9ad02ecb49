"""CPU checks that pin the oracle (oracle/) before it is trusted as the parity
reference.  Each oracle function is fixed by a check that does not retype its
formula:

=====================================  ==============================================
oracle function                        pinned by
=====================================  ==============================================
label_counts                           brute force on tiny label maps; sum_g n = s^2
elementwise (p, cp, cn, w, focal)      scipy.special expit / log_expit / entr
pairwise_mask_costs (bce, dice)        naive high-resolution evaluation on nearest-
                                       upsampled logits (scipy routines, no counts);
                                       closed form at z == 0; inf iff empty GT
pairwise_{sigmoid,softmax}_label_cost  scipy logsumexp / log_expit; closed forms
assign (C restatement, all strategies) brute-force optimum over permutations;
                                       scipy linear_sum_assignment on random
                                       matrices; hand-traced known answers (all-
                                       equal matrix, ties, greedy, round,
                                       pseudo-greedy, pred_round ranking)
denominators                           enumerated flag combinations (hand values)
matching_forward_losses                gather by numpy fancy indexing; closed forms
                                       of the unmatched penalties at z == 0
matching_backward                      central finite differences of the naive
                                       high-resolution loss with frozen weights
=====================================  ==============================================

The reference ships no golden vectors, fixtures or known-answer tests for this
path (its only harness, benchmarks.py, compares CUDA against Python at run
time); tests/golden/ holds vectors written by this oracle (tests/golden/make_golden.py),
checked against the oracle on the CPU and against the HIP path on the GPU
(tests/test_golden.py).
"""
import itertools
import math

import numpy as np
import pytest
from scipy import special
from scipy.optimize import linear_sum_assignment

from oracle import assign as A
from oracle import mask_oracle as O


# ---------------------------------------------------------------------------
# independent naive formulation (high resolution, no count trick)
# ---------------------------------------------------------------------------
def naive_terms(z, ug, ugm, gamma):
    p = special.expit(z)
    cp = -special.log_expit(z)
    cn = -special.log_expit(-z)
    ent = (special.entr(p) + special.entr(1.0 - p)) / math.log(2.0)
    w = np.power(ent, ug) if ug != 0 else np.ones_like(z)
    w = np.clip(w, ugm, 1.0)
    mp = (1 - p) ** gamma if gamma > 0 else np.ones_like(z)
    mn = p ** gamma if gamma > 0 else np.ones_like(z)
    return p, cp, cn, w, mp, mn


def naive_costs(z, tgt, GT_total, bg_index, smooth=1.0, ss=1.0, ds=1.0, ug=1.0, ugm=0.05,
                gamma=0.0, alpha=-1.0, normalize=True):
    L, B, Q, H, W = z.shape
    Ht, Wt = tgt.shape[1:]
    s = Ht // H
    zu = np.repeat(np.repeat(z, s, axis=3), s, axis=4).reshape(L, B, Q, Ht * Wt)
    p, cp, cn, w, mp, mn = naive_terms(zu, ug, ugm, gamma)
    ap, an = (alpha, 1 - alpha) if alpha >= 0 else (1.0, 1.0)
    skip = 0 <= bg_index < GT_total
    bg = bg_index if bg_index >= 0 else GT_total
    GT_out = GT_total - int(skip)
    S = w.sum(-1) if normalize else np.full(w.shape[:-1], float(Ht * Wt))
    S = np.maximum(S, 1e-12)
    bce = np.zeros((L, B, Q, GT_out))
    dice = np.zeros((L, B, Q, GT_out))
    for k in range(GT_out):
        a = k + (k >= bg)
        y = (tgt.reshape(B, -1) == a).astype(np.float64)[None, :, None, :]
        num = (w * (ap * mp * cp * y + an * mn * cn * (1 - y))).sum(-1)
        I = (w * p * y).sum(-1)
        T = (w * y).sum(-1)
        P = (w * p).sum(-1)
        bk = num / S * ss
        dk = (1 - (2 * I + smooth) / (P + T + smooth)) * ds
        empty = y.sum(-1)[0, :, 0] == 0
        bk[:, empty, :] = np.inf
        dk[:, empty, :] = np.inf
        bce[..., k] = bk
        dice[..., k] = dk
    return bce, dice


def rand_case(rng, L=1, B=2, Q=5, H=6, W=5, s=1, GT_total=4, sigma=2.0):
    z = rng.normal(0, sigma, size=(L, B, Q, H, W))
    tgt = rng.integers(-1, GT_total + 1, size=(B, H * s, W * s))
    return z, tgt


# ---------------------------------------------------------------------------
# counts
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("s", [1, 2, 3])
def test_label_counts_brute(s):
    rng = np.random.default_rng(s)
    B, H, W, G = 2, 3, 4, 5
    tgt = rng.integers(-2, G + 2, size=(B, H * s, W * s))
    n = O.label_counts(tgt, H, W, G)
    for b in range(B):
        for i in range(H):
            for j in range(W):
                block = tgt[b, i * s:(i + 1) * s, j * s:(j + 1) * s].ravel()
                for g in range(G):
                    assert n[b, g, i * W + j] == sum(int(v == g) for v in block)
                in_range = sum(int(0 <= v < G) for v in block)
                assert n[b, :, i * W + j].sum() == in_range
    full = np.zeros_like(tgt)
    assert (O.label_counts(full, H, W, G).sum(1) == s * s).all()


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("ug,gamma", [(1.0, 0.0), (0.0, 0.0), (2.5, 0.0), (1.0, 2.0), (0.5, 1.5)])
def test_elementwise_vs_scipy(ug, gamma):
    z = np.linspace(-20, 20, 2001)
    e = O.elementwise(z, gamma, ug, 0.05)
    p, cp, cn, w, mp, mn = naive_terms(z, ug, 0.05, gamma)
    np.testing.assert_allclose(e.p, p, rtol=1e-13, atol=0)
    np.testing.assert_allclose(e.cp, cp, rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(e.cn, cn, rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(e.w, w, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(e.mp, mp, rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(e.mn, mn, rtol=1e-12, atol=1e-300)


def test_elementwise_zero_closed_form():
    e = O.elementwise(np.zeros(3), 0.0, 1.0, 0.05)
    assert np.allclose(e.p, 0.5) and np.allclose(e.cp, math.log(2)) and np.allclose(e.cn, math.log(2))
    assert np.allclose(e.w, 1.0)


# ---------------------------------------------------------------------------
# pairwise mask costs
# ---------------------------------------------------------------------------
CASES = [
    dict(s=1, bg=0, normalize=True, ug=1.0, gamma=0.0, alpha=-1.0),
    dict(s=1, bg=-1, normalize=False, ug=0.0, gamma=0.0, alpha=-1.0),
    dict(s=2, bg=2, normalize=True, ug=2.0, gamma=2.0, alpha=0.25),
    dict(s=3, bg=7, normalize=True, ug=0.5, gamma=1.0, alpha=0.75),
    dict(s=1, bg=1, normalize=True, ug=1.0, gamma=1.5, alpha=-1.0),
]


@pytest.mark.parametrize("case", CASES)
def test_pairwise_costs_vs_naive(case):
    rng = np.random.default_rng(7)
    z, tgt = rand_case(rng, s=case["s"])
    G = 4
    b_o, d_o = O.pairwise_mask_costs(z, tgt, G, case["bg"], smooth=1.0, sigmoid_scale=1.5,
                                     dice_scale=0.7, ug=case["ug"], ug_min=0.05,
                                     mask_gamma=case["gamma"], mask_alpha=case["alpha"],
                                     normalize=case["normalize"])
    b_n, d_n = naive_costs(z, tgt, G, case["bg"], 1.0, 1.5, 0.7, case["ug"], 0.05, case["gamma"],
                           case["alpha"], case["normalize"])
    assert np.array_equal(np.isinf(b_o), np.isinf(b_n))
    fin = np.isfinite(b_n)
    np.testing.assert_allclose(b_o[fin], b_n[fin], rtol=1e-10)
    np.testing.assert_allclose(d_o[fin], d_n[fin], rtol=1e-10)


def test_pairwise_costs_zero_logits_closed_form():
    H = W = 8
    tgt = np.zeros((1, H, W), dtype=np.int64)
    tgt[0, :3, :5] = 1   # area 15
    tgt[0, 5:, 5:] = 2   # area 9
    z = np.zeros((1, 1, 3, H, W))
    bce, dice = O.pairwise_mask_costs(z, tgt, 4, 0, smooth=1.0)
    # z == 0: p = 1/2, cp = cn = ln 2, H = 1 bit -> w = 1
    assert np.allclose(bce[..., :2], math.log(2))
    for k, area in [(0, 15.0), (1, 9.0)]:
        expect = 1 - (2 * 0.5 * area + 1) / (0.5 * H * W + area + 1)
        assert np.allclose(dice[..., k], expect)
    assert np.isinf(bce[..., 2]).all() and np.isinf(dice[..., 2]).all()  # label 3 absent


def test_pairwise_costs_invariants():
    rng = np.random.default_rng(3)
    z, tgt = rand_case(rng, Q=9, H=7, W=7, GT_total=5)
    bce, dice = O.pairwise_mask_costs(z, tgt, 5, 0)
    fin = np.isfinite(bce)
    assert (bce[fin] >= 0).all()
    assert (dice[fin] >= 0).all() and (dice[fin] < 1).all()


# ---------------------------------------------------------------------------
# label costs
# ---------------------------------------------------------------------------
def test_softmax_label_cost_vs_scipy():
    rng = np.random.default_rng(1)
    z = rng.normal(0, 3, size=(2, 2, 4, 11))
    tg = np.array([[-1, 3, 10, 0, 11], [2, -1, 5, -1, 7]])
    out = O.pairwise_softmax_label_cost(z, tg, 0, scale=2.0)
    lse = special.logsumexp(z, axis=-1)
    for b in range(2):
        for k in range(4):
            y = tg[b, k + 1]
            if 0 <= y < 11:
                np.testing.assert_allclose(out[:, b, :, k], 2.0 * (lse[:, b] - z[:, b, :, y]), rtol=1e-12)
            else:
                assert np.isinf(out[:, b, :, k]).all()
    eq = O.pairwise_softmax_label_cost(np.zeros((1, 1, 2, 7)), np.array([[1, 2]]), -1)
    assert np.allclose(eq, math.log(7))


def test_sigmoid_label_cost_vs_scipy_and_zero():
    rng = np.random.default_rng(2)
    z = rng.normal(0, 2, size=(1, 2, 3, 6))
    tg = np.array([[4, 0, -1], [5, 2, 9]])
    for gamma, alpha in [(0.0, -1.0), (2.0, 0.25)]:
        out = O.pairwise_sigmoid_label_cost(z, tg, -1, scale=1.3, gamma=gamma, alpha=alpha)
        ap, an = (alpha, 1 - alpha) if alpha >= 0 else (1.0, 1.0)
        p = special.expit(z)
        neg = an * (p ** gamma if gamma else 1) * -special.log_expit(-z)
        pos = ap * ((1 - p) ** gamma if gamma else 1) * -special.log_expit(z)
        for b in range(2):
            for k in range(3):
                y = tg[b, k]
                if 0 <= y < 6:
                    onehot = np.zeros(6)
                    onehot[y] = 1
                    expect = (pos * onehot + neg * (1 - onehot)).sum(-1)[:, b] / 6 * 1.3
                    np.testing.assert_allclose(out[:, b, :, k], expect, rtol=1e-12)
                else:
                    assert np.isinf(out[:, b, :, k]).all()
    zero = O.pairwise_sigmoid_label_cost(np.zeros((1, 1, 1, 5)), np.array([[3]]), -1)
    assert np.allclose(zero, math.log(2))


# ---------------------------------------------------------------------------
# assignment
# ---------------------------------------------------------------------------
def brute_min(cost_rows_preds):
    M, n = cost_rows_preds.shape
    best = np.inf
    for perm in itertools.permutations(range(n), M):
        best = min(best, sum(cost_rows_preds[i, perm[i]] for i in range(M)))
    return best


def run(cost, **kw):
    p2g, pr = A.assign_batch(cost[None], **kw)
    return p2g[0], pr[0]


@pytest.mark.parametrize("seed", range(30))
def test_global_vs_brute_force(seed):
    rng = np.random.default_rng(seed)
    Q, G = int(rng.integers(1, 8)), int(rng.integers(1, 5))
    cost = rng.uniform(0, 10, size=(Q, G))
    if seed % 3 == 0:
        cost = np.round(cost)  # many ties
    p2g, pr = run(cost)
    M = min(G, Q)
    rows = list(range(G))[:M]
    got = sum(cost[q, g] for q, g in enumerate(p2g) if g >= 0)
    assert (p2g >= 0).sum() == M
    assert len(set(int(g) for g in p2g if g >= 0)) == M
    assert abs(got - brute_min(cost[:, rows].T)) < 1e-9
    assert ((pr == 0) == (p2g >= 0)).all()


@pytest.mark.parametrize("seed", range(10))
def test_global_vs_scipy_lsa(seed):
    rng = np.random.default_rng(100 + seed)
    Q, G = 60, int(rng.integers(5, 40))
    cost = rng.normal(size=(Q, G))
    p2g, _ = run(cost)
    r, c = linear_sum_assignment(cost.T)  # rows = GTs
    expect = np.full(Q, -1)
    expect[c] = r
    assert (p2g == expect).all()


def test_all_equal_known_answer():
    p2g, pr = run(np.full((6, 4), 3.0))
    assert list(p2g) == [0, 1, 2, 3, -1, -1]
    assert list(pr) == [0, 0, 0, 0, -1, -1]


def test_tie_lowest_index():
    cost = np.array([[1.0], [1.0], [5.0]])
    assert list(run(cost)[0]) == [0, -1, -1]
    cost = np.array([[2.0, 1.0], [1.0, 2.0], [1.0, 1.0]])
    # optimum 2 is reached by {q1->0, q0->1}, {q1->0, q2->1}, {q2->0, q0->1}; e-maxx picks
    # row 0 -> q1 (first minimum at j=2), then row 1 -> q0 (first minimum)
    assert list(run(cost)[0]) == [1, 0, -1]


def test_invalid_entries_and_columns():
    inf = np.inf
    cost = np.array([[inf, 2.0, 1e31], [inf, 1.0, 3.0], [inf, 5.0, inf]])
    p2g, pr = run(cost, inf_thresh=1e30)
    # column 0 invalid everywhere; column 2 valid only through q1 (3.0)
    assert list(p2g) == [1, 2, -1]
    assert list(pr) == [0, 0, -1]


def test_global_topk2_and_rounds():
    cost = np.array([[1.0, 9.0], [2.0, 9.0], [3.0, 0.5], [9.0, 9.0]])
    p2g, pr = run(cost, topk=2)
    # two slots per GT: GT0 takes q0 (1.0) and q1 (2.0), GT1 takes q2 (0.5) and q3 (9.0)
    assert list(p2g) == [0, 0, 1, 1]
    assert list(pr) == [0, 1, 0, 1]


def test_round_strategy_known_answer():
    cost = np.array([[1.0, 4.0], [2.0, 3.0], [5.0, 1.5], [6.0, 6.0]])
    # round 1: Hungarian -> q0:GT0, q2:GT1; round 2 on q1,q3 -> q1:GT0 (2.0)? q1:GT0=2,q3:GT1=6 -> 8
    # vs q1:GT1=3, q3:GT0=6 -> 9; so q1->GT0, q3->GT1
    p2g, pr = run(cost, topk=2, strategy=1)
    assert list(p2g) == [0, 0, 1, 1]
    assert list(pr) == [0, 1, 0, 1]


def test_greedy_strategy_known_answer():
    cost = np.array([[1.0, 0.5], [0.2, 0.3], [0.1, 0.9]])
    # q0 picks GT1 (0.5), q1 picks GT0 (0.2), q2: both capacities exhausted (K=1)
    p2g, pr = run(cost, topk=1, strategy=2)
    assert list(p2g) == [1, 0, -1]
    p2g, pr = run(cost, topk=2, strategy=2)
    # K=2: q0->GT1, q1->GT0, q2->GT0 (0.1); ranks: GT0 {q2:0.1, q1:0.2}
    assert list(p2g) == [1, 0, 0]
    assert list(pr) == [0, 1, 0]


def test_pseudo_greedy_known_answer():
    cost = np.array([[1.0, 0.5], [0.2, 0.3], [0.1, 0.9], [0.4, 0.35]])
    # Hungarian round: best 1:1 is q2->GT0 (0.1) + q1->GT1 (0.3) = 0.4
    # greedy tail with K=2: q0 -> GT1 (0.5 < 1.0), q3 -> GT0 (0.4 vs 0.35 but GT1 full)
    p2g, pr = run(cost, topk=2, strategy=3)
    assert list(p2g) == [1, 1, 0, 0]
    assert list(pr) == [1, 0, 0, 1]


def test_topk_zero_and_empty():
    cost = np.ones((3, 2))
    assert (run(cost, topk=0)[0] == -1).all()
    assert (A.assign_batch(np.ones((1, 3, 0)))[0] == -1).all()


# ---------------------------------------------------------------------------
# loss forward
# ---------------------------------------------------------------------------
def test_denominators_enumerated():
    p2g = np.array([[[0, -1, 1], [-1, -1, 2]]])  # L=1,B=2,Q=3: 3 matched
    md, cd = O.denominators(p2g, 2, 3, -1.0, False, False, False)
    assert md[0] == 3 and cd[0] == 3
    md, cd = O.denominators(p2g, 2, 3, 10.0, False, False, False)
    assert md[0] == 10 and cd[0] == 10
    md, cd = O.denominators(p2g, 2, 3, 10.0, True, False, False)
    assert md[0] == 6 and cd[0] == 10
    md, cd = O.denominators(p2g, 2, 3, -1.0, False, True, False)
    assert md[0] == 3 and cd[0] == 6
    md, cd = O.denominators(p2g, 2, 3, -1.0, False, False, True)
    assert md[0] == 3 and cd[0] == 6
    md, cd = O.denominators(np.full((1, 2, 3), -1), 2, 3, -1.0, False, False, False)
    assert md[0] == 1 and cd[0] == 1


def test_forward_losses_gather_and_zero_penalties():
    rng = np.random.default_rng(0)
    L, B, Q, H, W, G, C = 1, 2, 4, 4, 4, 3, 5
    sep = rng.uniform(0, 2, size=(3, L, B, Q, G))
    p2g = np.array([[[0, -1, 2, -1], [-1, 1, -1, -1]]])
    z = np.zeros((L, B, Q, H, W))
    zc = np.zeros((L, B, Q, C))
    m, d, c = O.matching_forward_losses(sep, p2g, z, zc, (B, H, W), force_masks=True,
                                        force_cls=True, void_class_index=C - 1, use_softmax=True)
    idx = np.argwhere(p2g >= 0)
    g = np.array([sep[:, l, b, q, p2g[l, b, q]] for l, b, q in idx]).sum(0)
    n_un = (p2g < 0).sum()
    P = 0.5 * H * W
    expect_m = (g[0] + n_un * math.log(2)) / (B * Q)
    expect_d = (g[1] + n_un * P / (P + 1.0)) / (B * Q)
    expect_c = (g[2] + n_un * math.log(C)) / (B * Q)
    np.testing.assert_allclose([m[0], d[0], c[0]], [expect_m, expect_d, expect_c], rtol=1e-12)
    # sigmoid label loss, force to background with a void channel: ln2 per unmatched query
    m2, d2, c2 = O.matching_forward_losses(sep, p2g, z, zc, (B, H, W), force_cls=True,
                                           void_class_index=C - 1, use_softmax=False)
    np.testing.assert_allclose(c2[0], (g[2] + n_un * math.log(2)) / (B * Q), rtol=1e-12)
    np.testing.assert_allclose(m2[0], g[0] / 3, rtol=1e-12)


# ---------------------------------------------------------------------------
# backward: finite differences with frozen weights
# ---------------------------------------------------------------------------
def frozen_loss(z, zc, tgt, cls_t, p2g, w_frozen, S_frozen, gm, gd, gc, md, cd, bg, *, smooth,
                ss, ds, gamma, alpha, force_masks, force_cls, void, use_softmax, cls_gamma,
                cls_alpha):
    L, B, Q, H, W = z.shape
    Ht, Wt = tgt.shape[1:]
    s = Ht // H
    GT_total = cls_t.shape[1]
    ap, an = (alpha, 1 - alpha) if alpha >= 0 else (1.0, 1.0)
    tot = 0.0
    for l in range(L):
        for b in range(B):
            for q in range(Q):
                out = p2g[l, b, q]
                act = out + (out >= bg) if out >= 0 else -1
                matched = out >= 0 and act < GT_total
                if matched or force_masks:
                    zu = np.repeat(np.repeat(z[l, b, q], s, 0), s, 1).ravel()
                    p, cp, cn, _, mp, mn = naive_terms(zu, 0.0, 0.0, gamma)
                    w = w_frozen[l, b, q]
                    y = (tgt[b].ravel() == act).astype(float) if matched else np.zeros_like(zu)
                    bce = (w * (ap * mp * cp * y + an * mn * cn * (1 - y))).sum() / S_frozen[l, b, q] * ss
                    I = (w * p * y).sum()
                    dice = (1 - (2 * I + smooth) / ((w * p).sum() + (w * y).sum() + smooth)) * ds
                    tot += gm[l] / md[l] * bce + gd[l] / md[l] * dice
                zz = zc[l, b, q]
                C = zz.shape[0]
                if matched:
                    y = cls_t[b, act]
                    if not (0 <= y < C):
                        continue
                    if use_softmax:
                        tot += gc[l] / cd[l] * (special.logsumexp(zz) - zz[y])
                    else:
                        cap, can = (cls_alpha, 1 - cls_alpha) if cls_alpha >= 0 else (1.0, 1.0)
                        pc = special.expit(zz)
                        onehot = np.zeros(C)
                        onehot[y] = 1
                        pos = cap * ((1 - pc) ** cls_gamma if cls_gamma else 1) * -special.log_expit(zz)
                        neg = can * (pc ** cls_gamma if cls_gamma else 1) * -special.log_expit(-zz)
                        tot += gc[l] / cd[l] * (pos * onehot + neg * (1 - onehot)).sum() / C
                elif force_cls or void >= 0:
                    if use_softmax and force_cls:
                        tot += gc[l] / cd[l] * (special.logsumexp(zz) - zz[void])
                    elif use_softmax:
                        tot += gc[l] / cd[l] * -special.log_expit(zz[void])
                    else:
                        pc = special.expit(zz)
                        cap, can = (cls_alpha, 1 - cls_alpha) if cls_alpha >= 0 else (1.0, 1.0)
                        pos = cap * ((1 - pc) ** cls_gamma if cls_gamma else 1) * -special.log_expit(zz)
                        neg = can * (pc ** cls_gamma if cls_gamma else 1) * -special.log_expit(-zz)
                        if force_cls:
                            onehot = np.zeros(C)
                            if void >= 0:
                                onehot[void] = 1
                            tot += gc[l] / cd[l] * (pos * onehot + neg * (1 - onehot)).sum() / C
                        else:
                            tot += gc[l] / cd[l] * pos[void]
    return tot


BWD_CASES = [
    dict(s=1, softmax=True, force_masks=False, force_cls=True, void=True, gamma=0.0, alpha=-1.0, normalize=True),
    dict(s=2, softmax=False, force_masks=True, force_cls=False, void=True, gamma=2.0, alpha=0.25, normalize=True),
    dict(s=1, softmax=False, force_masks=False, force_cls=True, void=False, gamma=1.0, alpha=-1.0, normalize=False),
    dict(s=1, softmax=True, force_masks=True, force_cls=False, void=True, gamma=0.0, alpha=0.6, normalize=True),
]


@pytest.mark.parametrize("case", BWD_CASES)
def test_backward_finite_differences(case):
    rng = np.random.default_rng(11)
    L, B, Q, H, W, C, GT_total = 1, 2, 4, 3, 3, 5, 4
    s = case["s"]
    z = rng.normal(0, 1.5, size=(L, B, Q, H, W))
    zc = rng.normal(0, 1.0, size=(L, B, Q, C))
    tgt = rng.integers(0, GT_total, size=(B, H * s, W * s))
    cls_t = np.array([[-1, 1, 3, 0], [-1, 2, -1, 4]])
    void = C - 1 if case["void"] else -1
    if void >= 0:
        cls_t[cls_t == void] = 0
    p2g = np.array([[[0, -1, 2, 1], [-1, 0, -1, 2]]])
    kw = dict(smooth=1.0, sigmoid_scale=1.3, dice_scale=0.8, cls_scale=1.1, background_index=0,
              ug=1.0, ug_min=0.05, num_masks=-1.0, force_cls=case["force_cls"],
              force_masks=case["force_masks"], mask_gamma=case["gamma"], mask_alpha=case["alpha"],
              cls_gamma=case["gamma"], cls_alpha=case["alpha"], void_class_index=void,
              use_softmax=case["softmax"], normalize=case["normalize"])
    gm, gd, gc = np.array([0.7]), np.array([1.2]), np.array([0.9])
    gz, gzc = O.matching_backward(gm, gd, gc, z, tgt, zc, cls_t, p2g, **kw)
    # frozen weights and normaliser at z
    zu = np.repeat(np.repeat(z, s, 3), s, 4).reshape(L, B, Q, -1)
    _, _, _, w0, _, _ = naive_terms(zu, 1.0, 0.05, 0.0)
    S0 = w0.sum(-1) if case["normalize"] else np.full(w0.shape[:-1], float(H * W * s * s))
    md, cd = O.denominators(p2g, B, Q, -1.0, case["force_masks"], case["force_cls"], void >= 0)
    fl = dict(smooth=1.0, ss=1.3, ds=0.8, gamma=case["gamma"], alpha=case["alpha"],
              force_masks=case["force_masks"], force_cls=case["force_cls"], void=void,
              use_softmax=case["softmax"], cls_gamma=case["gamma"], cls_alpha=case["alpha"])

    def F(zz, zzc):
        # cls_scale applies to the label terms
        return frozen_loss(zz, zzc, tgt, cls_t, p2g, w0, S0, gm, gd, gc * 1.1, md, cd, 0, **fl)

    h = 1e-6
    for idx in [(0, 0, 0, 1, 2), (0, 1, 1, 0, 0), (0, 0, 2, 2, 1), (0, 1, 3, 1, 1), (0, 0, 1, 0, 2)]:
        zp, zm = z.copy(), z.copy()
        zp[idx] += h
        zm[idx] -= h
        fd = (F(zp, zc) - F(zm, zc)) / (2 * h)
        assert abs(fd - gz[idx]) <= 1e-6 * max(1.0, abs(fd)), (idx, fd, gz[idx])
    for idx in [(0, 0, 0, 1), (0, 0, 1, 4), (0, 1, 1, 2), (0, 1, 2, 4), (0, 1, 3, 0)]:
        zp, zm = zc.copy(), zc.copy()
        zp[idx] += h
        zm[idx] -= h
        fd = (F(z, zp) - F(z, zm)) / (2 * h)
        assert abs(fd - gzc[idx]) <= 1e-6 * max(1.0, abs(fd)), (idx, fd, gzc[idx])
