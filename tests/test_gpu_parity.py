"""GPU parity: the HIP path (through the `mask_loss` extension and its C ABI)
against the float64 oracle on the same seeded inputs.

Tolerances (north star): float32 logits rel 1e-5, bfloat16 logits rel 2e-2.
A value r is matched by g when |g - r| <= rtol * (|r| + floor), with floor =
1e-2 for costs and losses (dice costs approach 0 for good matches, where a
purely relative bound is ill-posed) and floor = 1e-2 * max|r| for gradients.
Assignment indices are compared bit for bit against the C restatement of the
reference solver run on the GPU's own float32 cost matrix (the reference
solver's input), and against the oracle's float64 costs where the optimal
assignment's cost gap exceeds the tolerance.
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import assign as OA  # noqa: E402
from oracle import mask_oracle as O  # noqa: E402
from assign_rule import check_f64_assignment_total  # noqa: E402

pytestmark = pytest.mark.gpu

RTOL = {"float32": 1e-5, "bfloat16": 2e-2, "float16": 2e-3}
TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


@pytest.fixture(scope="module")
def ml():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mask_loss_amd
    return mask_loss_amd.mask_loss


def close(g, r, rtol, floor):
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.array_equal(np.isinf(g), np.isinf(r)), "inf pattern differs"
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    bound = rtol * (np.abs(r[f]) + floor)
    bad = err > bound
    assert not bad.any(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"


def rounded(z, dtype):
    t = torch.from_numpy(np.ascontiguousarray(z, dtype=np.float32)).to(TDT[dtype])
    return t, t.float().numpy().astype(np.float64)


def make_case(seed, L=1, B=2, Q=20, H=16, W=16, s=1, G=6, C=9, dtype="float32", sigma=2.0,
              empty_image=False, extreme=False, grid=False, grid_sizes=None):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, sigma, size=(L, B, Q, H, W)).astype(np.float32)
    if extreme:  # |z| >= 64 in a few rows: outside the bf16 table, formulas redo those waves
        vals = np.array([64.0, -64.0, 80.0, -100.0, 300.0, -1000.0, 65.5, -8192.0], np.float32)
        for l, b, q in [(0, 0, 1), (0, 0, 2), (0, 1, Q - 1)]:
            cells = rng.choice(H * W, size=12, replace=False)
            z[l, b, q].reshape(-1)[cells] = rng.choice(vals, size=12)
        z[0, 1, 0] = 70.0  # a whole row beyond the table
    tgt = np.zeros((B, H * s, W * s), dtype=np.int64)
    for b in range(B):
        if empty_image and b == 0:
            continue
        if grid:  # Gb disjoint blocks, labels shuffled: exactly Gb non-empty GTs
            Gb = G if grid_sizes is None else grid_sizes[b]
            r = int(math.ceil(math.sqrt(Gb)))
            c = int(math.ceil(Gb / r))
            hb, wb = (H * s) // r, (W * s) // c
            assert hb > 0 and wb > 0, "grid case: blocks need a cell each"
            perm = rng.permutation(G)[:Gb] + 1
            for i in range(Gb):
                y0, x0 = (i // c) * hb, (i % c) * wb
                tgt[b, y0:y0 + hb, x0:x0 + wb] = perm[i]
            continue
        for g in range(1, G + 1):
            cy, cx = rng.uniform(0, H * s), rng.uniform(0, W * s)
            ry, rx = rng.uniform(1, H * s / 3), rng.uniform(1, W * s / 3)
            yy, xx = np.mgrid[0:H * s, 0:W * s]
            tgt[b][((yy - cy) / ry) ** 2 + ((xx - cx) / rx) ** 2 <= 1] = g
    cls_t = np.full((B, G + 2), -1, dtype=np.int64)  # slot 0 = background, last = padding
    cls_t[:, 1:G + 1] = rng.integers(0, C - 1, size=(B, G))
    zc = rng.normal(0, 1, size=(L, B, Q, C)).astype(np.float32)
    zt, z64 = rounded(z, dtype)
    return dict(z=zt.cuda(), z64=z64, tgt=torch.from_numpy(tgt).cuda(), tgt_np=tgt,
                zc=torch.from_numpy(zc).cuda(), zc64=zc.astype(np.float64),
                ct=torch.from_numpy(cls_t).cuda(), ct_np=cls_t, C=C, dtype=dtype)


COST_CASES = [
    dict(name="f32_default", kw={}, p={}),
    dict(name="bf16_default", kw=dict(dtype="bfloat16", sigma=3.0), p={}),
    dict(name="f16_default", kw=dict(dtype="float16"), p={}),
    dict(name="f32_counts_s2", kw=dict(s=2, H=12, W=12), p={}),
    dict(name="f32_counts_s4", kw=dict(s=4, H=8, W=8), p={}),
    # 16-bit counts: s = 16 (n and N2 - n up to 256) and s = 17 (289: the
    # one-hot operands split into high and low bf16 terms)
    dict(name="f32_counts_s16", kw=dict(s=16, H=4, W=4), p={}),
    dict(name="f32_counts_s17", kw=dict(s=17, H=3, W=5, Q=24), p=dict(mask_gamma=2.0, mask_alpha=0.25)),
    dict(name="bf16_counts_s17", kw=dict(s=17, H=4, W=3, dtype="bfloat16", sigma=3.0), p={}),
    dict(name="f32_focal", kw={}, p=dict(mask_gamma=2.0, mask_alpha=0.25, cls_gamma=2.0, cls_alpha=0.25)),
    dict(name="f32_focal_g1", kw={}, p=dict(mask_gamma=1.0, mask_alpha=0.6, cls_gamma=1.5)),
    dict(name="f32_ug0_nonorm", kw={}, p=dict(ug=0.0, normalize=False)),
    dict(name="f32_ug2", kw={}, p=dict(ug=2.0, ug_min=0.1)),
    dict(name="f32_nobg", kw={}, p=dict(bg=-1)),
    dict(name="f32_bg_mid", kw={}, p=dict(bg=3)),
    dict(name="f32_softmax", kw={}, p=dict(use_softmax=True)),
    dict(name="f32_odd_shapes", kw=dict(Q=37, H=7, W=5, B=3), p={}),
    dict(name="f32_tail32", kw=dict(Q=17, H=10, W=10), p={}),
    dict(name="f32_many_gt", kw=dict(G=40, Q=50, H=32, W=32), p={}),
    dict(name="bf16_many_gt", kw=dict(G=120, Q=64, H=32, W=32, dtype="bfloat16"), p={}),
    dict(name="bf16_extreme", kw=dict(Q=40, H=32, W=32, dtype="bfloat16", sigma=3.0, extreme=True), p={}),
    dict(name="bf16_extreme_many_gt",
         kw=dict(G=70, Q=40, H=32, W=32, dtype="bfloat16", sigma=3.0, extreme=True), p={}),
    # the wide classes: slot sums with a 2-term split (f16), a background
    # label inside the GT range (the label -> slot table), focal terms in the
    # 16-tile class, and count operands (grouped K-splits, complement form)
    # (grid: exactly G non-empty GTs, 40 in the 7-tile class, 120 in the
    # 16-tile one)
    dict(name="f32_grid40", kw=dict(G=40, Q=50, H=32, W=32, grid=True), p={}),
    dict(name="f32_grid120_focal", kw=dict(G=120, Q=40, H=32, W=32, grid=True),
         p=dict(mask_gamma=2.0, mask_alpha=0.25, ug=2.0, ug_min=0.1)),
    dict(name="f16_grid40", kw=dict(G=40, Q=50, H=32, W=32, dtype="float16", grid=True), p={}),
    dict(name="f16_grid120", kw=dict(G=120, Q=40, H=32, W=32, dtype="float16", grid=True), p={}),
    dict(name="bf16_grid40", kw=dict(G=40, Q=64, H=32, W=32, dtype="bfloat16", sigma=3.0, grid=True), p={}),
    dict(name="bf16_grid120", kw=dict(G=120, Q=40, H=32, W=32, dtype="bfloat16", sigma=3.0, grid=True), p={}),
    dict(name="f32_grid40_bg_mid", kw=dict(G=40, Q=50, H=32, W=32, grid=True), p=dict(bg=3)),
    dict(name="f32_counts_s2_grid40", kw=dict(s=2, G=40, Q=40, H=32, W=32, grid=True), p={}),
    dict(name="f32_empty_image", kw=dict(empty_image=True), p={}),
    dict(name="f32_L2", kw=dict(L=2), p=dict(scales=(1.3, 0.7, 2.0), smooth=0.5)),
]


def params(p):
    d = dict(smooth=1.0, scales=(1.0, 1.0, 1.0), bg=0, ug=1.0, ug_min=0.05, mask_gamma=0.0,
             mask_alpha=-1.0, cls_gamma=0.0, cls_alpha=-1.0, use_softmax=False, normalize=True)
    d.update(p)
    return d


def gpu_costs(ml, x, P):
    ss, ds, cs = P["scales"]
    return ml.pairwise_mask_loss_forward(
        x["z"], x["tgt"], x["zc"], x["ct"], P["smooth"], ss, ds, cs, P["bg"], P["ug"],
        P["ug_min"], P["mask_gamma"], P["mask_alpha"], P["cls_gamma"], P["cls_alpha"],
        P["use_softmax"], P["normalize"])


def oracle_costs(x, P):
    ss, ds, cs = P["scales"]
    return O.pairwise_mask_loss_forward(
        x["z64"], x["tgt_np"], x["zc64"], x["ct_np"], P["smooth"], ss, ds, cs, P["bg"], P["ug"],
        P["ug_min"], P["mask_gamma"], P["mask_alpha"], P["cls_gamma"], P["cls_alpha"],
        P["use_softmax"], P["normalize"])


@pytest.mark.parametrize("case", COST_CASES, ids=lambda c: c["name"])
def test_pairwise_costs(ml, case):
    x = make_case(5, **case["kw"])
    P = params(case["p"])
    got = gpu_costs(ml, x, P).cpu().numpy()
    ref = oracle_costs(x, P)
    rt = RTOL[x["dtype"]]
    close(got[0], ref[0], rt, 1e-2)
    close(got[1], ref[1], rt, 1e-2)
    close(got[2], ref[2], 1e-5, 1e-2)  # label costs are float32 in every case


@pytest.mark.parametrize("softmax", [False, True])
def test_label_cost_ops(ml, softmax):
    x = make_case(9)
    if softmax:
        got = ml.forward_pw_softmax_label_loss(x["zc"], x["ct"], 0, 1.7).cpu().numpy()
        ref = O.pairwise_softmax_label_cost(x["zc64"], x["ct_np"], 0, 1.7)
    else:
        got = ml.forward_pw_sigmoid_label_loss(x["zc"], x["ct"], -1, 1.7, 2.0, 0.25).cpu().numpy()
        ref = O.pairwise_sigmoid_label_cost(x["zc64"], x["ct_np"], -1, 1.7, 2.0, 0.25)
    close(got, ref, 1e-5, 1e-2)


def matching_call(ml, x, P, M, prefill=None, check_void=False):
    ss, ds, cs = P["scales"]
    return ml.mask_matching_fused(
        x["z"], x["tgt"], x["zc"], x["ct"], P["smooth"], ss, ds, cs, P["bg"], P["ug"], P["ug_min"],
        M["inf_thresh"], M["num_masks"], M["force_cls"], M["force_masks"], M["K"], M["strategy"],
        P["mask_gamma"], P["mask_alpha"], P["cls_gamma"], P["cls_alpha"], M["void"],
        P["use_softmax"], P["normalize"], prefill, check_void)


MATCH_CASES = [
    dict(name="global_softmax_forcebg", kw={}, p=dict(use_softmax=True),
         m=dict(force_cls=True, void=8)),
    dict(name="global_sigmoid", kw={}, p={}, m={}),
    dict(name="global_sigmoid_void_forcemasks", kw={}, p={}, m=dict(void=8, force_masks=True)),
    dict(name="global_K2", kw=dict(Q=30), p={}, m=dict(K=2)),
    dict(name="round_K2", kw=dict(Q=30), p={}, m=dict(K=2, strategy=1)),
    dict(name="greedy_K2", kw=dict(Q=30), p={}, m=dict(K=2, strategy=2)),
    dict(name="pseudo_greedy_K3", kw=dict(Q=30), p={}, m=dict(K=3, strategy=3)),
    dict(name="more_gts_than_queries", kw=dict(Q=5, G=9), p={}, m={}),
    dict(name="bf16_headline_like", kw=dict(dtype="bfloat16", sigma=3.0, Q=70, G=30, H=32, W=32),
         p=dict(use_softmax=True), m=dict(force_cls=True, void=8)),
    dict(name="num_masks", kw={}, p={}, m=dict(num_masks=7.0)),
    dict(name="inf_thresh_low", kw={}, p={}, m=dict(inf_thresh=2.0)),
    dict(name="counts_s2_force", kw=dict(s=2, H=12, W=12), p=dict(mask_gamma=2.0, mask_alpha=0.25),
         m=dict(force_masks=True, force_cls=True)),
    dict(name="counts_s17_force", kw=dict(s=17, H=4, W=4), p={}, m=dict(force_masks=True, force_cls=True)),
    # wider column classes with unweighted row sums: K-splits added in the
    # cost workgroup (8 per partial at 41 columns, 4 at 121)
    dict(name="wide7_force", kw=dict(G=40, Q=50, H=32, W=32, grid=True), p={},
         m=dict(force_masks=True, force_cls=True)),
    dict(name="wide16_force", kw=dict(G=120, Q=40, H=32, W=32, grid=True), p={}, m=dict(force_masks=True)),
    dict(name="wide16", kw=dict(G=120, Q=130, H=32, W=32, grid=True), p={}, m={}),
    # images in all three column-tile classes (10, 60, 120 GTs), two layers:
    # the widest class's finalize and assignment run on the side stream
    dict(name="mixed_classes_l2", kw=dict(L=2, B=3, G=120, Q=130, H=32, W=32, grid=True,
                                          grid_sizes=(10, 60, 120)), p={}, m={}),
    # only wide images (115-130 GTs), one and two layers
    dict(name="wide_parts", kw=dict(B=4, G=130, Q=140, H=32, W=32, grid=True,
                                    grid_sizes=(115, 130, 120, 125)), p={}, m={}),
    dict(name="bf16_wide_parts_l2", kw=dict(L=2, B=4, G=130, Q=140, H=32, W=32, dtype="bfloat16", sigma=3.0,
                                            grid=True, grid_sizes=(125, 40, 130, 118)), p={},
         m=dict(force_cls=True, void=8)),
    dict(name="mixed_classes_round_K2", kw=dict(B=3, G=120, Q=130, H=32, W=32, grid=True,
                                                grid_sizes=(120, 25, 70)), p=dict(use_softmax=True),
         m=dict(K=2, strategy=1, force_cls=True, void=8)),
    # bf16 with forced-empty masks runs without the table: slot sums in bf16
    dict(name="bf16_wide7_force", kw=dict(G=40, Q=50, H=32, W=32, dtype="bfloat16", sigma=3.0, grid=True),
         p={}, m=dict(force_masks=True, force_cls=True)),
    dict(name="empty_image", kw=dict(empty_image=True), p={}, m=dict(force_cls=True, void=8)),
    dict(name="q_tail_1024", kw=dict(Q=130, H=8, W=8, G=20), p={}, m={}),
    # cost matrices too large for LDS (300 x 250 floats): every row read in
    # place from the total-cost plane
    dict(name="global_rows", kw=dict(Q=300, H=8, W=8, G=250), p={}, m={}),
    dict(name="global_rows_round_K2", kw=dict(Q=300, H=8, W=8, G=160), p={}, m=dict(K=2, strategy=1)),
    dict(name="global_rows_pseudo_greedy_K2", kw=dict(Q=300, H=8, W=8, G=200), p={},
         m=dict(K=2, strategy=3)),
    # finalize's wide form: more than 192 classes held in registers (20 per lane)
    dict(name="softmax_C700", kw=dict(C=700, Q=24), p=dict(use_softmax=True),
         m=dict(force_cls=True, void=699)),
    dict(name="sigmoid_C1280", kw=dict(C=1280, Q=24), p={}, m=dict(force_cls=True, void=1279)),
]


def mparams(m):
    d = dict(inf_thresh=1e30, num_masks=-1.0, force_cls=False, force_masks=False, K=1,
             strategy=0, void=-1)
    d.update(m)
    return d


@pytest.mark.parametrize("case", MATCH_CASES, ids=lambda c: c["name"])
def test_matching_forward(ml, case):
    x = make_case(21, **case["kw"])
    P, M = params(case["p"]), mparams(case["m"])
    p2g, pr, m, d, c, saved = [t.cpu() for t in matching_call(ml, x, P, M)]
    # 1. solver bit-exactness on the GPU's own float32 cost matrix
    sep = gpu_costs(ml, x, P)
    total = ((sep[0] + sep[1]) + sep[2]).double().cpu().numpy()
    L, B, Q, G = total.shape
    rp2g, rpr = OA.assign_batch(total.reshape(L * B, Q, G), M["inf_thresh"], M["K"], M["strategy"])
    assert np.array_equal(p2g.numpy().reshape(L * B, Q), rp2g), "assignment differs from reference solver"
    assert np.array_equal(pr.numpy().reshape(L * B, Q), rpr), "pred_round differs"
    # 2. losses against the oracle evaluated at the same assignment
    ss, ds, cs = P["scales"]
    ref_sep = oracle_costs(x, P)
    rm, rd, rc = O.matching_forward_losses(
        ref_sep, p2g.numpy(), x["z64"], x["zc64"], x["tgt_np"].shape, P["smooth"], ss, ds, cs,
        P["mask_gamma"], P["mask_alpha"], P["cls_gamma"], P["cls_alpha"], M["num_masks"],
        M["force_masks"], M["force_cls"], M["void"], P["use_softmax"])
    rt = RTOL[x["dtype"]]
    close(m.numpy(), rm, rt, 1e-2)
    close(d.numpy(), rd, rt, 1e-2)
    close(c.numpy(), rc, 1e-5, 1e-2)
    # 3. the oracle's own float64 assignment agrees wherever it is not a near-tie
    check_f64_assignment(ref_sep, p2g.numpy(), rt, M)


def check_f64_assignment(ref_sep, p2g, rt, M, exact=False):
    """The north-star rule for indices (tests/assign_rule.py) on the float64
    oracle's separate costs ref_sep (3, L, B, Q, G): the total is
    (bce + dice) + label, the reference's sum (src/cpu/matching.cpp:665-704)."""
    rt64 = (ref_sep[0] + ref_sep[1]) + ref_sep[2]
    L, B, Q, G = rt64.shape
    op2g, _ = check_f64_assignment_total(rt64.reshape(L * B, Q, G), p2g, rt, M["inf_thresh"],
                                         M["K"], M["strategy"], exact=exact)
    return op2g


def separated_case(seed, Q=48, G=10, H=32, W=32, dtype="bfloat16", ties=False):
    """bf16 inputs whose float64 optimum is separated from every other
    assignment: query 3k+1 carries GT k's mask as +/-6 logits (a strong
    match), the others are N(0, 3) noise.  ties: query 3k+2 repeats query
    3k+1 exactly (mask and class logits), so two queries tie exactly for
    GT k in both float32 and float64 and the solver's tie rule (lowest index)
    decides."""
    x = make_case(seed, B=2, Q=Q, G=G, H=H, W=W, dtype="float32", sigma=3.0)
    z = x["z64"].astype(np.float32).copy()
    zc = x["zc64"].astype(np.float32).copy()
    for b in range(2):
        for k in range(G):
            if 3 * k + 1 >= Q:
                break
            m = x["tgt_np"][b] == k + 1
            if not m.any():
                continue
            z[0, b, 3 * k + 1] = np.where(m, 6.0, -6.0)
            zc[0, b, 3 * k + 1, int(x["ct_np"][b, k + 1])] = 4.0
            if ties and 3 * k + 2 < Q:
                z[0, b, 3 * k + 2] = z[0, b, 3 * k + 1]
                zc[0, b, 3 * k + 2] = zc[0, b, 3 * k + 1]
    zt, z64 = rounded(z, dtype)
    return dict(x, z=zt.cuda(), z64=z64, zc=torch.from_numpy(zc).cuda(),
                zc64=zc.astype(np.float64), dtype=dtype)


@pytest.mark.parametrize("ties", [False, True], ids=["clear_gap", "exact_ties"])
def test_assignment_bf16_separated(ml, ties):
    """bf16 logits (costs from the bf16 table): with a clear gap, and with
    exact ties decided by the tie rule, the indices equal the float64
    optimum's bit for bit."""
    x = separated_case(61, ties=ties)
    P, M = params(dict(use_softmax=True)), mparams(dict(force_cls=True, void=8))
    p2g = matching_call(ml, x, P, M)[0].cpu().numpy()
    ref_sep = oracle_costs(x, P)
    op2g = check_f64_assignment(ref_sep, p2g, RTOL["bfloat16"], M, exact=True)
    G = ref_sep.shape[-1]
    for b in range(2):  # the strong matches (or, with ties, their twins) are the ones taken
        for k in range(G):
            if 3 * k + 2 < x["z64"].shape[2] and (x["tgt_np"][b] == k + 1).any():
                took = [q for q in (3 * k + 1, 3 * k + 2) if op2g[b][q] == k]
                assert took == [3 * k + 1] or (ties and len(took) == 1), (b, k, took)


def test_assignment_bf16_near_tie(ml):
    """Two queries one bf16 step apart in a single cell: their costs differ by
    far less than the tolerance, so either may take the GT; the GPU's choice
    must then cost no more than rt * sum|costs| above the float64 optimum."""
    x = separated_case(62, ties=True)
    z = x["z"].clone()
    z.view(torch.int16)[0, 0, 2, 0, 0] += 1  # one bf16 step in one cell of query 2
    x = dict(x, z=z, z64=z.float().cpu().numpy().astype(np.float64))
    P, M = params(dict(use_softmax=True)), mparams(dict(force_cls=True, void=8))
    p2g = matching_call(ml, x, P, M)[0].cpu().numpy()
    check_f64_assignment(oracle_costs(x, P), p2g, RTOL["bfloat16"], M)


BWD_CASES = [
    dict(name="f32_softmax_forcebg", kw={}, p=dict(use_softmax=True), m=dict(force_cls=True, void=8)),
    dict(name="f32_sigmoid_focal_forcemasks", kw={}, p=dict(mask_gamma=2.0, mask_alpha=0.25,
         cls_gamma=2.0, cls_alpha=0.25), m=dict(force_masks=True, void=8)),
    dict(name="f32_counts_s2", kw=dict(s=2, H=12, W=12), p={}, m=dict(force_cls=True)),
    dict(name="f32_counts_s17", kw=dict(s=17, H=4, W=3), p={}, m=dict(force_cls=True)),
    dict(name="bf16_counts_s16", kw=dict(s=16, H=4, W=4, dtype="bfloat16", sigma=3.0), p={},
         m=dict(force_cls=True)),
    dict(name="f32_nonorm_ug0", kw={}, p=dict(ug=0.0, normalize=False), m={}),
    dict(name="bf16_softmax", kw=dict(dtype="bfloat16", sigma=3.0), p=dict(use_softmax=True),
         m=dict(force_cls=True, void=8)),
    dict(name="f32_odd", kw=dict(Q=37, H=7, W=5, B=3), p={}, m=dict(void=8)),
    # class rows longer than 256 logits: held 8 or 16 logits per lane by the
    # f32 masks' kernels (the matched-row kernel, which also writes the class
    # gradients in the prefilled mode, and the class launch of the other
    # modes), streamed by the bf16 table kernel
    dict(name="f32_softmax_C300", kw=dict(C=300, Q=24), p=dict(use_softmax=True),
         m=dict(force_cls=True, void=299)),
    # every query matched (more GTs than queries): the matched-row items fill
    # the whole grid, so every workgroup takes class rows after its mask items
    dict(name="f32_all_matched_C300", kw=dict(C=300, Q=12, G=20), p=dict(use_softmax=True),
         m=dict(force_cls=True, void=299)),
    dict(name="f32_softmax_C700", kw=dict(C=700, Q=24), p=dict(use_softmax=True),
         m=dict(force_cls=True, void=699)),
    dict(name="bf16_softmax_C700", kw=dict(C=700, Q=24, dtype="bfloat16", sigma=3.0),
         p=dict(use_softmax=True), m=dict(force_cls=True, void=699)),
    # the wide classes' statistics (slot sums for f32, the table for bf16)
    dict(name="f32_grid40", kw=dict(G=40, Q=50, H=32, W=32, grid=True), p={}, m=dict(force_cls=True, void=8)),
    dict(name="bf16_grid120", kw=dict(G=120, Q=130, H=32, W=32, dtype="bfloat16", sigma=3.0, grid=True),
         p={}, m=dict(force_cls=True, void=8)),
    # the widest class's images assigned on the side stream, the gradient
    # fill with the other images' launches (the mixed cases); only wide images
    dict(name="f32_mixed_classes_l2", kw=dict(L=2, B=3, G=120, Q=130, H=32, W=32, grid=True,
                                              grid_sizes=(10, 60, 120)), p={}, m=dict(force_cls=True, void=8)),
    dict(name="bf16_mixed_classes", kw=dict(B=3, G=120, Q=130, H=32, W=32, dtype="bfloat16", sigma=3.0,
                                            grid=True, grid_sizes=(120, 8, 120)), p={}, m={}),
    dict(name="f32_wide_parts", kw=dict(B=4, G=130, Q=140, H=32, W=32, grid=True,
                                        grid_sizes=(115, 130, 120, 125)), p={}, m=dict(force_cls=True, void=8)),
    dict(name="f32_grid120_forcemasks", kw=dict(G=120, Q=40, H=32, W=32, grid=True), p={},
         m=dict(force_masks=True)),
]


@pytest.mark.parametrize("mode", ["saved", "prefilled", "two_pass"])
@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: c["name"])
def test_matching_backward(ml, case, mode):
    x = make_case(33, **case["kw"])
    P, M = params(case["p"]), mparams(case["m"])
    prefill = None
    if mode == "prefilled":
        if M["force_masks"]:
            pytest.skip("no prefill when unmatched masks are forced to empty")
        # garbage in the buffer: the forward's side-stream fill must clear it
        prefill = torch.full_like(x["z"], 7.0)
    outs = matching_call(ml, x, P, M, prefill)
    p2g, saved = outs[0], outs[5]
    L = x["z"].shape[0]
    gm = torch.tensor([0.7] * L, device="cuda")
    gd = torch.tensor([1.3] * L, device="cuda")
    gc = torch.tensor([0.9] * L, device="cuda")
    ss, ds, cs = P["scales"]
    args = (gm, gd, gc, x["z"], x["tgt"], x["zc"], x["ct"], p2g, P["smooth"], ss, ds, cs, P["bg"],
            P["ug"], P["ug_min"], M["num_masks"], M["force_cls"], M["force_masks"], P["mask_gamma"],
            P["mask_alpha"], P["cls_gamma"], P["cls_alpha"], M["void"], P["use_softmax"],
            P["normalize"])
    if mode == "saved":
        gz, gzc = ml.mask_matching_backward_fused(*args, saved)
    elif mode == "prefilled":
        gz, gzc = ml.mask_matching_backward_fused(*args, saved, prefill)
        assert gz.data_ptr() == prefill.data_ptr()
    else:
        gz, gzc = ml.mask_matching_backward(*args)
    assert gz.dtype == x["z"].dtype and gzc.dtype == x["zc"].dtype
    rz, rzc = O.matching_backward(
        gm.cpu().numpy(), gd.cpu().numpy(), gc.cpu().numpy(), x["z64"], x["tgt_np"], x["zc64"],
        x["ct_np"], p2g.cpu().numpy(), P["smooth"], ss, ds, cs, P["bg"], P["ug"], P["ug_min"],
        M["num_masks"], M["force_cls"], M["force_masks"], P["mask_gamma"], P["mask_alpha"],
        P["cls_gamma"], P["cls_alpha"], M["void"], P["use_softmax"], P["normalize"])
    rt = RTOL[x["dtype"]]
    gzn = gz.float().cpu().numpy()
    close(gzn, rz, rt, 1e-2 * np.abs(rz).max())
    close(gzc.cpu().numpy(), rzc, 1e-5, 1e-2 * np.abs(rzc).max())
    unmatched = p2g.cpu().numpy() < 0
    if not M["force_masks"]:
        assert (gzn[unmatched] == 0).all()


@pytest.mark.parametrize("G,class1_empty", [(31, True), (40, False)])
def test_prefilled_fill_shares(ml, G, class1_empty):
    """The prefilled gradient's zero fill is shared by three launches (the
    column pass, finalize and the assignment). With a 7.0 sentinel in the
    buffer, the prefilled backward must equal the saved-state backward (which
    writes every row itself) bit for bit, at a size where every share is used
    (105 MB of gradient) and with GT_out + 1 > 32 columns, so the NT = 7
    column-tile class is launched: empty (every image has at most 31
    non-empty GTs) or not."""
    x = make_case(47, B=4, Q=200, H=256, W=256, G=G, dtype="bfloat16", sigma=3.0)
    present = [int((np.unique(x["tgt_np"][b]) > 0).sum()) for b in range(4)]
    assert (max(present) <= 31) == class1_empty, present  # the case's premise
    P, M = params(dict(use_softmax=True)), mparams(dict(force_cls=True, void=8))
    prefill = torch.full_like(x["z"], 7.0)
    outs = matching_call(ml, x, P, M, prefill)
    p2g, saved = outs[0], outs[5]
    gm = torch.tensor([0.7], device="cuda")
    gd = torch.tensor([1.3], device="cuda")
    gc = torch.tensor([0.9], device="cuda")
    ss, ds, cs = P["scales"]
    args = (gm, gd, gc, x["z"], x["tgt"], x["zc"], x["ct"], p2g, P["smooth"], ss, ds, cs, P["bg"],
            P["ug"], P["ug_min"], M["num_masks"], M["force_cls"], M["force_masks"], P["mask_gamma"],
            P["mask_alpha"], P["cls_gamma"], P["cls_alpha"], M["void"], P["use_softmax"],
            P["normalize"])
    gz_pre, _ = ml.mask_matching_backward_fused(*args, saved, prefill)
    gz_all, _ = ml.mask_matching_backward_fused(*args, saved)
    torch.cuda.synchronize()
    assert gz_pre.data_ptr() == prefill.data_ptr()
    assert not (gz_pre == 7.0).any()
    unmatched = (p2g < 0).reshape(-1)
    assert (gz_pre.reshape(-1, 256 * 256)[unmatched] == 0).all()
    assert torch.equal(gz_pre, gz_all)


def test_function_autograd_bf16(ml):
    from mask_loss_amd.functions import MaskMatchingFunction
    x = make_case(44, dtype="bfloat16", sigma=3.0, Q=40, G=12)
    z = x["z"].clone().requires_grad_(True)
    zc = x["zc"].clone().requires_grad_(True)
    p2g, pr, m, d, c = MaskMatchingFunction.apply(
        z, x["tgt"], zc, x["ct"], 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, True, 1e30, -1.0, True, False,
        1, "global", 0.0, None, 0.0, None, 8, "softmax")
    (m.sum() + d.sum() + c.sum()).backward()
    assert z.grad.dtype == torch.bfloat16 and z.grad.shape == z.shape
    rz, rzc = O.matching_backward(
        np.ones(1), np.ones(1), np.ones(1), x["z64"], x["tgt_np"], x["zc64"], x["ct_np"],
        p2g.cpu().numpy(), 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, -1.0, True, False, 0.0, -1.0, 0.0,
        -1.0, 8, True, True)
    close(z.grad.float().cpu().numpy(), rz, 2e-2, 1e-2 * np.abs(rz).max())
    close(zc.grad.cpu().numpy(), rzc, 1e-5, 1e-2 * np.abs(rzc).max())


def test_function_double_backward_fresh_buffer(ml):
    """The prefilled gradient buffer serves the first backward only; a second
    backward through the retained graph allocates anew, so the first result
    (held as .grad) is not overwritten."""
    from mask_loss_amd.functions import MaskMatchingFunction
    x = make_case(45, dtype="bfloat16", sigma=3.0, Q=40, G=12)
    z = x["z"].clone().requires_grad_(True)
    zc = x["zc"].clone().requires_grad_(True)
    outs = MaskMatchingFunction.apply(
        z, x["tgt"], zc, x["ct"], 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, True, 1e30, -1.0, True, False,
        1, "global", 0.0, None, 0.0, None, 8, "softmax")
    m, d, c = outs[2:]
    g1 = torch.autograd.grad(m.sum() + d.sum() + c.sum(), [z], retain_graph=True)[0]
    first = g1.clone()
    g2 = torch.autograd.grad(2.0 * (m.sum() + d.sum() + c.sum()), [z])[0]
    assert g1.data_ptr() != g2.data_ptr()
    assert torch.equal(g1, first)
    close(g2.float().cpu().numpy(), 2.0 * first.float().cpu().numpy(), 1e-2,
          1e-2 * first.float().abs().max().item())


@pytest.mark.parametrize("where", ["absent", "first_image", "last_image_padding"])
def test_void_class_check(ml, where):
    """The reference raises ValueError when cls_targets holds the void index
    (functions/mask/matching.py:184-185).  Here the forward's preparation
    kernels make that check and the fused binding returns it as a seventh
    output; MaskMatchingFunction raises on it.  The forward's results do not
    depend on the check."""
    from mask_loss_amd.functions import MaskMatchingFunction
    x = make_case(46, B=3, Q=24, G=5)  # classes drawn from [0, 8): void 8 absent
    ct = x["ct"].clone()
    if where == "first_image":
        ct[0, 1] = 8
    elif where == "last_image_padding":
        ct[2, -1] = 8
    x = dict(x, ct=ct)
    P, M = params(dict(use_softmax=True)), mparams(dict(force_cls=True, void=8))
    outs = matching_call(ml, x, P, M, check_void=True)
    assert len(outs) == 7 and outs[6].device.type == "cpu"
    assert outs[6].tolist() == [0 if where == "absent" else 1]
    plain = matching_call(ml, x, P, M)
    assert len(plain) == 6
    for u, v in zip(outs[:5], plain[:5]):
        assert torch.equal(u, v)
    # no valid void index: the check reports 0
    none = matching_call(ml, x, params({}), mparams(dict(void=-1)), check_void=True)
    assert none[6].tolist() == [0]
    args = (x["z"], x["tgt"], x["zc"], ct, 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, True, 1e30, -1.0,
            True, False, 1, "global", 0.0, None, 0.0, None, 8, "softmax")
    if where == "absent":
        MaskMatchingFunction.apply(*args)
    else:
        with pytest.raises(ValueError, match="void class index"):
            MaskMatchingFunction.apply(*args)


def test_reference_wrapper_argument_order(ml):
    """The reference's MaskMatchingFunction calls mask_matching with 25
    positional arguments (normalize_uncertainty twice); both orders work."""
    x = make_case(3)
    a24 = ml.mask_matching(x["z"], x["tgt"], x["zc"], x["ct"], 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05,
                           1e30, -1.0, False, False, 1, 0, 0.0, -1.0, 0.0, -1.0, -1, False, True)
    a25 = ml.mask_matching(x["z"], x["tgt"], x["zc"], x["ct"], 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05,
                           True, 1e30, -1.0, False, False, 1, 0, 0.0, -1.0, 0.0, -1.0, -1, False,
                           True)
    for u, v in zip(a24, a25):
        assert torch.equal(u, v)


def test_deterministic(ml):
    x = make_case(8, dtype="bfloat16", Q=64, G=20, H=32, W=32)
    P, M = params(dict(use_softmax=True)), mparams(dict(force_cls=True, void=8))
    a = [t.clone() for t in matching_call(ml, x, P, M)]
    b = [t.clone() for t in matching_call(ml, x, P, M)]
    L, B, Q = a[0].shape
    head = (L * B * Q * 4 + L * 2) * 4  # float head of the saved state: stats + layer block
    a[5], b[5] = a[5][:head], b[5][:head]
    for u, v in zip(a, b):
        assert torch.equal(u, v)
