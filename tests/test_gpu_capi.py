"""The matching forward through the C ABI alone: ml_mask_matching_forward
(include/mask_loss_hip.h; reference src/cpu/matching.cpp:592-752) called with
ctypes on device buffers that torch only allocates, with no use of the
`mask_loss` extension module.  Checked against the test oracle: the
assignment and pred_round bit for bit against the C restatement of the
reference solver on the call's own float32 cost matrix, the cost planes and
the layer means against the float64 oracle (float32
rel 1e-5, bfloat16 2e-2, as |g - r| <= rtol (|r| + 1e-2)), and the void-class
flag against a direct check of the class targets."""
import ctypes
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import assign as OA  # noqa: E402
from oracle import mask_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "mask_loss_amd", "libmask_loss_hip.so")
ML_F32, ML_BF16 = 0, 1
RTOL = {ML_F32: 1e-5, ML_BF16: 2e-2}


class Shape(ctypes.Structure):
    _fields_ = [(k, ctypes.c_int64) for k in ["L", "B", "Q", "H", "W", "Ht", "Wt", "C", "GT_total"]]


class Params(ctypes.Structure):
    _fields_ = [("smooth", ctypes.c_float), ("sigmoid_scale", ctypes.c_float),
                ("dice_scale", ctypes.c_float), ("cls_scale", ctypes.c_float),
                ("background_index", ctypes.c_int64), ("uncertainty_gamma", ctypes.c_float),
                ("uncertainty_gamma_min", ctypes.c_float), ("inf_thresh", ctypes.c_double),
                ("num_masks", ctypes.c_double), ("force_cls", ctypes.c_int32),
                ("force_masks", ctypes.c_int32), ("topk", ctypes.c_int64),
                ("strategy", ctypes.c_int64), ("mask_gamma", ctypes.c_float),
                ("mask_alpha", ctypes.c_float), ("cls_gamma", ctypes.c_float),
                ("cls_alpha", ctypes.c_float), ("void", ctypes.c_int64),
                ("softmax", ctypes.c_int32), ("normalize", ctypes.c_int32)]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.zeros(1, device="cuda")  # the HIP runtime is up before the library's first call
    lib = ctypes.CDLL(LIB)
    P = ctypes.c_void_p
    lib.ml_mask_matching_forward.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params), ctypes.c_int,
                                             P, P, ctypes.c_int, P, P, P, P, P, P, P, P, P, P, P,
                                             ctypes.c_size_t, P]
    lib.ml_mask_matching_workspace_size.restype = ctypes.c_size_t
    lib.ml_mask_matching_workspace_size.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params),
                                                    ctypes.c_int]
    lib.ml_saved_bytes.restype = ctypes.c_size_t
    lib.ml_saved_bytes.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params), ctypes.c_int]
    lib.ml_last_error.restype = ctypes.c_char_p
    return lib


def make(seed, B, Q, H, W, G, C, dtype, void_in_targets=False):
    rng = np.random.default_rng(seed)
    z = torch.from_numpy(rng.normal(0, 3 if dtype == ML_BF16 else 2, size=(1, B, Q, H, W)).astype(np.float32))
    z = z.to(torch.bfloat16 if dtype == ML_BF16 else torch.float32)
    tgt = np.zeros((B, H, W), np.int64)
    yy, xx = np.mgrid[0:H, 0:W]
    for b in range(B):
        for g in range(1, G + 1):
            cy, cx, r = rng.uniform(0, H), rng.uniform(0, W), rng.uniform(1, H / 3)
            tgt[b][(yy - cy) ** 2 + (xx - cx) ** 2 <= r * r] = g
    ct = np.full((B, G + 1), -1, np.int64)
    ct[:, 1:] = rng.integers(0, C - 1, size=(B, G))
    if void_in_targets:
        ct[B - 1, 1] = C - 1
    zc = rng.normal(0, 1, size=(1, B, Q, C)).astype(np.float32)
    return dict(z=z.cuda(), z64=z.float().numpy().astype(np.float64), tgt=torch.from_numpy(tgt).cuda(),
                tgt_np=tgt, zc=torch.from_numpy(zc).cuda(), zc64=zc.astype(np.float64),
                ct=torch.from_numpy(ct).cuda(), ct_np=ct, dtype=dtype,
                shape=Shape(1, B, Q, H, W, H, W, C, G + 1))


def forward(lib, x, p):
    s = x["shape"]
    L, B, Q, G = s.L, s.B, s.Q, s.GT_total - 1
    dev = "cuda"
    out = dict(p2g=torch.full((L, B, Q), -7, dtype=torch.int64, device=dev),
               pr=torch.full((L, B, Q), -7, dtype=torch.int64, device=dev),
               means=torch.full((3, L), float("nan"), device=dev),
               sep=torch.full((3, L, B, Q, G), float("nan"), device=dev),
               saved=torch.zeros(lib.ml_saved_bytes(s, p, x["dtype"]), dtype=torch.uint8, device=dev),
               void=torch.full((1,), -1, dtype=torch.int32, device=dev))
    wsb = lib.ml_mask_matching_workspace_size(s, p, x["dtype"])
    assert wsb > 0, lib.ml_last_error()
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.ml_mask_matching_forward(ctypes.byref(s), ctypes.byref(p), x["dtype"], ptr(x["z"]),
                                      ptr(x["tgt"]), ML_F32, ptr(x["zc"]), ptr(x["ct"]), ptr(out["p2g"]),
                                      ptr(out["pr"]), ptr(out["means"]), ptr(out["sep"]),
                                      ptr(out["saved"]), None, ptr(out["void"]), None, ptr(ws), wsb,
                                      stream)
    assert rc == 0, lib.ml_last_error().decode()
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in out.items()}


def close(g, r, rtol):
    g = np.asarray(g, np.float64)
    r = np.asarray(r, np.float64)
    assert np.array_equal(np.isinf(g), np.isinf(r)), "inf pattern differs"
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    assert (err <= rtol * (np.abs(r[f]) + 1e-2)).all(), f"max err {err.max():.3e}"


CASES = [
    # the benchmark's arguments: softmax label cost, unmatched queries to no-object
    dict(name="bf16_softmax_force_cls", mk=dict(B=3, Q=48, H=32, W=32, G=14, C=9, dtype=ML_BF16),
         p=dict(force_cls=1, softmax=1, void=8)),
    dict(name="f32_sigmoid_K2_round", mk=dict(B=2, Q=30, H=16, W=16, G=6, C=7, dtype=ML_F32),
         p=dict(topk=2, strategy=1)),
    dict(name="f32_void_flag", mk=dict(B=2, Q=20, H=16, W=16, G=5, C=7, dtype=ML_F32, void_in_targets=True),
         p=dict(void=6)),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c["name"])
def test_capi_matching_forward(lib, case):
    x = make(31, **case["mk"])
    d = dict(force_cls=0, force_masks=0, topk=1, strategy=0, void=-1, softmax=0)
    d.update(case["p"])
    p = Params(1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, 1e30, -1.0, d["force_cls"], d["force_masks"], d["topk"],
               d["strategy"], 0.0, -1.0, 0.0, -1.0, d["void"], d["softmax"], 1)
    out = forward(lib, x, p)
    sep = out["sep"].numpy()
    L, B, Q, G = sep.shape[1:]
    # 1. the solver, bit for bit, on the call's own float32 costs
    total = ((out["sep"][0] + out["sep"][1]) + out["sep"][2]).double().numpy().reshape(L * B, Q, G)
    rp2g, rpr = OA.assign_batch(total, 1e30, d["topk"], d["strategy"])
    assert np.array_equal(out["p2g"].numpy().reshape(L * B, Q), rp2g)
    assert np.array_equal(out["pr"].numpy().reshape(L * B, Q), rpr)
    assert (rp2g >= 0).any()
    # 2. costs and means against the float64 oracle
    ref = O.pairwise_mask_loss_forward(x["z64"], x["tgt_np"], x["zc64"], x["ct_np"], 1.0, 1.0, 1.0, 1.0,
                                       0, 1.0, 0.05, 0.0, -1.0, 0.0, -1.0, bool(d["softmax"]), True)
    rt = RTOL[x["dtype"]]
    close(sep[0], ref[0], rt)
    close(sep[1], ref[1], rt)
    close(sep[2], ref[2], 1e-5)
    rm, rd, rc = O.matching_forward_losses(
        ref, out["p2g"].numpy(), x["z64"], x["zc64"], x["tgt_np"].shape, 1.0, 1.0, 1.0, 1.0, 0.0, -1.0,
        0.0, -1.0, -1.0, bool(d["force_masks"]), bool(d["force_cls"]), d["void"], bool(d["softmax"]))
    means = out["means"].numpy()
    close(means[0], rm, rt)
    close(means[1], rd, rt)
    close(means[2], rc, 1e-5)
    # 3. the void-class flag (reference functions/mask/matching.py:184-185)
    want_void = int(d["void"] >= 0 and (x["ct_np"] == d["void"]).any())
    assert int(out["void"].item()) == want_void


# ---- the forward that launches only the column-tile classes with images ----
def hip_runtime():
    """The HIP runtime the process has loaded (torch's), for pinned memory."""
    for line in open("/proc/self/maps"):
        path = line.split()[-1]
        if "libamdhip64.so" in path:
            rt = ctypes.CDLL(path)
            rt.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
            rt.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                                   ctypes.c_uint]
            rt.hipHostFree.argtypes = [ctypes.c_void_p]
            return rt
    pytest.skip("HIP runtime not found in the process")


def polled_forward(lib, x, p, words, prefill=False):
    """ml_mask_matching_forward_polled with the host/device words `words`
    (with prefill: a gradient-sized buffer of nonzero bytes to zero-fill,
    returned as "prefill")."""
    s = x["shape"]
    L, B, Q, G = s.L, s.B, s.Q, s.GT_total - 1
    dev = "cuda"
    out = dict(p2g=torch.full((L, B, Q), -7, dtype=torch.int64, device=dev),
               pr=torch.full((L, B, Q), -7, dtype=torch.int64, device=dev),
               means=torch.full((3, L), float("nan"), device=dev),
               sep=torch.full((3, L, B, Q, G), float("nan"), device=dev),
               saved=torch.zeros(lib.ml_saved_bytes(s, p, x["dtype"]), dtype=torch.uint8, device=dev),
               void=torch.full((1,), -1, dtype=torch.int32, device=dev))
    if prefill:
        out["prefill"] = torch.full((x["z"].numel() * x["z"].element_size(),), 0x5A, dtype=torch.uint8,
                                    device=dev)
    wsb = lib.ml_mask_matching_workspace_size(s, p, x["dtype"])
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    hdev, hhost = words
    rc = lib.ml_mask_matching_forward_polled(
        ctypes.byref(s), ctypes.byref(p), x["dtype"], ptr(x["z"]), ptr(x["tgt"]), ML_F32, ptr(x["zc"]),
        ptr(x["ct"]), ptr(out["p2g"]), ptr(out["pr"]), ptr(out["means"]), ptr(out["sep"]),
        ptr(out["saved"]), ptr(out["prefill"]) if prefill else None, ptr(out["void"]), None, ptr(ws), wsb,
        stream, hdev, hhost)
    assert rc == 0, lib.ml_last_error().decode()
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in out.items()}


def class_of(g):
    """Column-tile class of an image with g non-empty GTs (g + 1 slots in
    tiles of 16: at most 2 tiles, at most 7, more)."""
    need = (g + 1 + 15) // 16
    return 0 if need <= 2 else 1 if need <= 7 else 2


def two_size_case(seed, dtype, big_gts):
    """Images 0, 1 with at most 12 and 20 GTs and image 2 with exactly
    `big_gts` non-empty GTs (disjoint 3 x 3 squares), so that image 2 is in
    column-tile class class_of(big_gts) and images 0, 1 in class 0; GT_total
    is 41 (64 x 64 cells and GT_total 121 for big_gts > 40)."""
    wide = big_gts > 40
    G = 120 if wide else 40
    x = make(seed, B=3, Q=40, H=64 if wide else 32, W=64 if wide else 32, G=G, C=9, dtype=dtype)
    per = 16 if wide else 8
    tgt = x["tgt_np"].copy()
    tgt[0][tgt[0] > 12] = 0
    tgt[1][tgt[1] > 20] = 0
    tgt[2] = 0
    for g in range(1, big_gts + 1):
        y0, x0 = ((g - 1) // per) * 6, ((g - 1) % per) * 4
        tgt[2, y0:y0 + 3, x0:x0 + 3] = g
    x["tgt_np"] = tgt
    x["tgt"] = torch.from_numpy(tgt).cuda()
    return x


@pytest.mark.parametrize("dtype", [ML_F32, ML_BF16])
@pytest.mark.parametrize("big_gts", [20, 40, 120])
def test_capi_polled_forward_same_results(lib, dtype, big_gts):
    """The polled forward skips the empty wider classes (big_gts = 20: only
    class 0 has images) or launches them (40: class 1, 120: class 2), and
    returns exactly what ml_mask_matching_forward returns, with the gradient
    buffer zero-filled.  With two non-empty classes the first class's
    finalize and assignment run on the side stream (class 0 first for 40,
    the widest class first for 120).  Its words hold the classes' task
    counts."""
    rt = hip_runtime()
    P = ctypes.c_void_p
    lib.ml_mask_matching_forward_polled.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params), ctypes.c_int,
                                                    P, P, ctypes.c_int, P, P, P, P, P, P, P, P, P, P, P,
                                                    ctypes.c_size_t, P, P, P]
    h = ctypes.c_void_p()
    assert rt.hipHostMalloc(ctypes.byref(h), 64, 0x2 | 0x40000000) == 0  # mapped | coherent
    try:
        d = ctypes.c_void_p()
        assert rt.hipHostGetDevicePointer(ctypes.byref(d), h, 0) == 0
        words = (ctypes.c_int32 * 16).from_address(h.value)
        x = two_size_case(77, dtype, big_gts)
        p = Params(1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, 1e30, -1.0, 1, 0, 1, 0, 0.0, -1.0, 0.0, -1.0, 8, 1, 1)
        want = forward(lib, x, p)
        for _ in range(2):  # twice: the words are re-armed by each call
            got = polled_forward(lib, x, p, (d, h), prefill=True)
            for k in ("p2g", "pr", "means", "sep", "saved", "void"):
                assert torch.equal(got[k], want[k]), k
            assert not got["prefill"].any()
            rtiles = (x["shape"].Q + 15) // 16
            present = [len(np.setdiff1d(np.unique(x["tgt_np"][b]), [0])) for b in range(3)]
            assert present[2] == big_gts
            cls = [class_of(g) for g in present]
            n = [words[i] for i in range(3)]
            assert n == [cls.count(c) * rtiles for c in range(3)], (n, present)
            assert n[class_of(big_gts)] >= rtiles
    finally:
        rt.hipHostFree(h)
