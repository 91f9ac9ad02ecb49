"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the float64 oracle).

CPU: the oracle, re-run on the stored inputs, still reproduces the stored
outputs (guards against oracle drift).  GPU: the HIP path on the stored inputs
matches the stored outputs -- costs, losses and gradients within the float32
tolerance (relative 1e-5 with a 1e-2 floor; gradients with a floor of
1e-2 * max|g|), assignments and rounds exactly.
"""
import importlib.util
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
MG = importlib.util.module_from_spec(spec)
spec.loader.exec_module(MG)

CASES = {c["name"]: c for c in MG.CASES}


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    d = load(name)
    out = MG.outputs(CASES[name], d["z"], d["tgt"], d["zc"], d["cls_t"])
    for k, v in out.items():
        if v.dtype.kind in "iu":
            assert np.array_equal(v, d[k]), k
        else:
            assert np.array_equal(np.isinf(v), np.isinf(d[k])), k
            f = np.isfinite(v)
            assert np.allclose(v[f], d[k][f], rtol=1e-12, atol=1e-14), k


def close(g, r, rtol, floor):
    g = np.asarray(g, np.float64)
    r = np.asarray(r, np.float64)
    assert g.shape == r.shape
    assert np.array_equal(np.isinf(g), np.isinf(r))
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    assert (err <= rtol * (np.abs(r[f]) + floor)).all(), err.max()


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_gpu_matches_fixture(name):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mask_loss_amd
    ml = mask_loss_amd.mask_loss
    d = load(name)
    kw = dict(CASES[name]["kw"])
    dev = torch.device("cuda:0")
    z = torch.from_numpy(d["z"]).to(dev)
    tgt = torch.from_numpy(d["tgt"]).to(dev)
    zc = torch.from_numpy(d["zc"]).to(dev)
    ct = torch.from_numpy(d["cls_t"]).to(dev)
    bg = kw.get("background_index", -1)
    ug = kw.get("ug", 1.0)
    mg, ma = kw.get("mask_gamma", 0.0), kw.get("mask_alpha", -1.0)
    sm = kw.get("use_softmax", False)
    fc, fm = kw.get("force_cls", False), kw.get("force_masks", False)
    void = kw.get("void_class_index", -1)
    sep = ml.pairwise_mask_loss_forward(z, tgt, zc, ct, 1.0, 1.0, 1.0, 1.0, bg, ug, 0.05, mg, ma,
                                        0.0, -1.0, sm, True).cpu().numpy()
    close(sep, d["sep"], 1e-5, 1e-2)
    p2g, prd, mm, dm, cm = ml.mask_matching(z, tgt, zc, ct, 1.0, 1.0, 1.0, 1.0, bg, ug, 0.05, 1e30,
                                            -1.0, fc, fm, 1, 0, mg, ma, 0.0, -1.0, void, sm, True)
    assert np.array_equal(p2g.cpu().numpy(), d["pred_to_gt"])
    assert np.array_equal(prd.cpu().numpy(), d["pred_round"])
    for got, key in ((mm, "mask_mean"), (dm, "dice_mean"), (cm, "cls_mean")):
        close(got.float().cpu().numpy(), d[key], 1e-5, 1e-2)
    L = z.shape[0]
    ones = torch.ones(L, device=dev)
    gz, gzc = ml.mask_matching_backward(ones, ones, ones, z, tgt, zc, ct, p2g, 1.0, 1.0, 1.0, 1.0, bg,
                                        ug, 0.05, -1.0, fc, fm, mg, ma, 0.0, -1.0, void, sm, True)
    for got, key in ((gz, "grad_mask"), (gzc, "grad_cls")):
        r = d[key]
        close(got.float().cpu().numpy(), r, 1e-5, 1e-2 * max(np.abs(r).max(), 1e-30))
