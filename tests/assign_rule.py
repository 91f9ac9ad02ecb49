"""The north-star rule for assignment indices, shared by the GPU parity tests.

On each (layer, image) slice the GPU's assignment must equal the one the
reference solver (src/cpu/matching.cpp:95-186, :476-571, restated in
oracle/assign.c) finds on the float64 oracle costs, unless the two choices are
not separated by more than the cost tolerance: the GPU's assignment may then
cost at most rt * sum |matched oracle costs| more than the float64 optimum,
evaluated on the float64 costs.  Test infrastructure only.
"""
import numpy as np

from oracle import assign as OA


def assignment_cost(c64, a):
    """Total float64 cost of assignment a (query -> column or -1) on one slice."""
    return float(sum(c64[q, g] for q, g in enumerate(a) if g >= 0))


def check_f64_assignment_total(total64, p2g, rt, inf_thresh=1e30, topk=1, strategy=0,
                               exact=False, nthreads=1):
    """total64: (L*B, Q, G) float64 oracle total costs; p2g: the GPU's
    pred_to_gt, any shape that flattens to (L*B, Q).  `exact`: the case is
    constructed with a clear gap (or exact ties), so the indices must be
    equal.  Returns the float64 optimum's pred_to_gt and the number of slices
    whose indices differ from it (each within the tolerance)."""
    c = np.ascontiguousarray(total64, dtype=np.float64)
    N, Q, G = c.shape
    op2g, _ = OA.assign_batch(c, inf_thresh, topk, strategy, nthreads=nthreads)
    got = np.asarray(p2g).reshape(N, Q)
    differ = 0
    for s_ in range(N):
        if np.array_equal(op2g[s_], got[s_]):
            continue
        differ += 1
        assert not exact, f"slice {s_}: assignment differs from the float64 optimum"
        gap = assignment_cost(c[s_], got[s_]) - assignment_cost(c[s_], op2g[s_])
        tol = rt * sum(abs(c[s_, q, g]) for q, g in enumerate(op2g[s_]) if g >= 0)
        assert abs(gap) <= tol, f"slice {s_}: float64 cost gap {gap:.3e} > {tol:.3e}"
    return op2g, differ
