"""Write the committed golden fixtures (tests/golden/*.npz) from the float64
oracle on small seeded inputs.

The reference ships no golden vectors for this path, so these fixtures are
produced by the oracle (itself pinned by tests/test_oracle.py) and serve two
purposes: the CPU suite re-derives them to detect any drift of the oracle, and
the GPU suite checks the HIP path against the stored outputs without running
the oracle.  Run from the repository root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import mask_oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, seed, shape and options); inputs as float32 (the GPU path's input)
CASES = [
    dict(name="small_sigmoid", seed=11, L=1, B=2, Q=12, H=12, W=12, s=1, G=4, C=6,
         kw=dict(background_index=0, use_softmax=False, force_cls=True, void_class_index=5)),
    dict(name="small_softmax_s2", seed=12, L=2, B=2, Q=10, H=8, W=8, s=2, G=3, C=5,
         kw=dict(background_index=0, use_softmax=True, force_cls=True, void_class_index=4,
                 mask_gamma=2.0, mask_alpha=0.25)),
    dict(name="small_nobg_forced", seed=13, L=1, B=3, Q=9, H=10, W=6, s=1, G=3, C=4,
         kw=dict(background_index=-1, use_softmax=False, force_masks=True, ug=0.0)),
]


def make_inputs(c):
    rng = np.random.default_rng(c["seed"])
    L, B, Q, H, W, s, G, C = (c[k] for k in ("L", "B", "Q", "H", "W", "s", "G", "C"))
    z = rng.normal(0, 2, size=(L, B, Q, H, W)).astype(np.float32)
    tgt = np.zeros((B, H * s, W * s), dtype=np.int64)
    yy, xx = np.mgrid[0:H * s, 0:W * s]
    for b in range(B):
        for g in range(1, G + 1):
            cy, cx = rng.uniform(0, H * s), rng.uniform(0, W * s)
            ry, rx = rng.uniform(1.5, H * s / 2.5), rng.uniform(1.5, W * s / 2.5)
            tgt[b][((yy - cy) / ry) ** 2 + ((xx - cx) / rx) ** 2 <= 1] = g
    cls_t = np.full((B, G + 1), -1, dtype=np.int64)
    void = c["kw"].get("void_class_index", -1)
    ncls = C - 1 if void >= 0 else C
    cls_t[:, 1:] = rng.integers(0, ncls, size=(B, G))
    zc = rng.normal(0, 1, size=(L, B, Q, C)).astype(np.float32)
    return z, tgt, zc, cls_t


def outputs(c, z, tgt, zc, cls_t):
    kw = dict(c["kw"])
    z64, zc64 = z.astype(np.float64), zc.astype(np.float64)
    cost_kw = {k: kw[k] for k in ("background_index", "use_softmax", "mask_gamma", "mask_alpha", "ug")
               if k in kw}
    sep = O.pairwise_mask_loss_forward(z64, tgt, zc64, cls_t, **cost_kw)
    p2g, prd, mm, dm, cm, _ = O.mask_matching(z64, tgt, zc64, cls_t, **kw)
    L = z.shape[0]
    bwd_kw = {k: v for k, v in kw.items() if k not in ("topk", "strategy", "inf_thresh")}
    gz, gzc = O.matching_backward(np.ones(L), np.ones(L), np.ones(L), z64, tgt, zc64, cls_t, p2g,
                                  **bwd_kw)
    return dict(sep=sep, pred_to_gt=p2g, pred_round=prd, mask_mean=mm, dice_mean=dm,
                cls_mean=cm, grad_mask=gz, grad_cls=gzc)


def main():
    for c in CASES:
        z, tgt, zc, cls_t = make_inputs(c)
        out = outputs(c, z, tgt, zc, cls_t)
        np.savez_compressed(os.path.join(HERE, c["name"] + ".npz"), z=z, tgt=tgt, zc=zc, cls_t=cls_t,
                            **out)
        print(c["name"], {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
