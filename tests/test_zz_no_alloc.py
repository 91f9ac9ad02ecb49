"""The matching forward that allocates nothing (ml_mask_matching_forward_noalloc,
scratch in a static device array) against ml_mask_matching_forward with a
caller workspace, both called through the C ABI with ctypes (the `mask_loss`
extension module is not involved; torch only provides device memory and the
stream).  Two calls in a row, the second on a smaller input, so the second
runs on scratch the first left behind.  Indices and pred_round bit-exact;
costs, means and the saved statistics within the north-star tolerance (float32
1e-5, bfloat16 2e-2; the two paths share kernels and K-splits, so they agree
bit for bit in practice)."""
import ctypes
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

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
    common = [ctypes.POINTER(Shape), ctypes.POINTER(Params), ctypes.c_int, P, P, ctypes.c_int, P, P,
              P, P, P, P, P, P, P, P]
    lib.ml_mask_matching_forward.argtypes = common + [P, ctypes.c_size_t, P]
    lib.ml_mask_matching_forward_noalloc.argtypes = common + [P]
    lib.ml_mask_matching_workspace_size.restype = ctypes.c_size_t
    lib.ml_mask_matching_workspace_size.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params), ctypes.c_int]
    lib.ml_saved_bytes.restype = ctypes.c_size_t
    lib.ml_saved_bytes.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params), ctypes.c_int]
    lib.ml_mask_matching_forward_noalloc_bytes.restype = ctypes.c_size_t
    lib.ml_mask_matching_forward_noalloc_bytes.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Params),
                                                          ctypes.c_int]
    lib.ml_last_error.restype = ctypes.c_char_p
    return lib


def make_inputs(seed, B, Q, H, W, G, C, dtype):
    rng = np.random.default_rng(seed)
    z = torch.from_numpy(rng.normal(0, 3, size=(1, B, Q, H, W)).astype(np.float32))
    z = z.to(torch.bfloat16 if dtype == ML_BF16 else torch.float32)
    tgt = np.zeros((B, H, W), np.int64)
    yy, xx = np.mgrid[0:H, 0:W]
    for b in range(B):
        for g in range(1, G + 1):
            cy, cx = rng.uniform(0, H), rng.uniform(0, W)
            r = rng.uniform(1, H / 3)
            tgt[b][(yy - cy) ** 2 + (xx - cx) ** 2 <= r * r] = g
    ct = np.full((B, G + 1), -1, np.int64)
    ct[:, 1:] = rng.integers(0, C - 1, size=(B, G))
    zc = rng.normal(0, 1, size=(1, B, Q, C)).astype(np.float32)
    return dict(z=z.cuda(), tgt=torch.from_numpy(tgt).cuda(), zc=torch.from_numpy(zc).cuda(),
                ct=torch.from_numpy(ct).cuda(), dtype=dtype,
                shape=Shape(1, B, Q, H, W, H, W, C, G + 1))


def params(C):
    # the benchmark's arguments: softmax label cost, unmatched queries forced to no-object
    return Params(1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, 1e30, -1.0, 1, 0, 1, 0, 0.0, -1.0, 0.0, -1.0,
                  C - 1, 1, 1)


def forward(lib, x, noalloc):
    s, p = x["shape"], params(x["shape"].C)
    L, B, Q, G = s.L, s.B, s.Q, s.GT_total - 1
    dev = "cuda"
    out = dict(p2g=torch.full((L, B, Q), -7, dtype=torch.int64, device=dev),
               pr=torch.full((L, B, Q), -7, dtype=torch.int64, device=dev),
               means=torch.full((3, L), float("nan"), device=dev),
               sep=torch.full((3, L, B, Q, G), float("nan"), device=dev),
               saved=torch.zeros(lib.ml_saved_bytes(s, p, x["dtype"]), dtype=torch.uint8, device=dev),
               void=torch.full((1,), -1, dtype=torch.int32, device=dev))
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    args = [ctypes.byref(s), ctypes.byref(p), x["dtype"], ptr(x["z"]), ptr(x["tgt"]), ML_F32,
            ptr(x["zc"]), ptr(x["ct"]), ptr(out["p2g"]), ptr(out["pr"]), ptr(out["means"]),
            ptr(out["sep"]), ptr(out["saved"]), None, ptr(out["void"]), None]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = lib.ml_mask_matching_forward_noalloc(*args, stream)
    else:
        wsb = lib.ml_mask_matching_workspace_size(s, p, x["dtype"])
        assert wsb > 0, lib.ml_last_error()
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        rc = lib.ml_mask_matching_forward(*args, ptr(ws), wsb, stream)
        out["ws"] = ws
    assert rc == 0, lib.ml_last_error().decode()
    torch.cuda.synchronize()
    return out


def close(g, r, rtol, what):
    g = g.double().cpu().numpy()
    r = r.double().cpu().numpy()
    assert np.array_equal(np.isinf(g), np.isinf(r)), f"{what}: inf pattern differs"
    f = np.isfinite(r)
    assert np.isfinite(g[f]).all(), f"{what}: non-finite values"
    err = np.abs(g[f] - r[f])
    assert (err <= rtol * (np.abs(r[f]) + 1e-2)).all(), f"{what}: max err {err.max():.3e}"


def test_noalloc_forward_matches_workspace_forward(lib):
    cases = [make_inputs(1, B=3, Q=48, H=32, W=32, G=14, C=9, dtype=ML_BF16),
             make_inputs(2, B=2, Q=20, H=16, W=16, G=6, C=7, dtype=ML_F32)]  # smaller second call
    for i, x in enumerate(cases):
        got = forward(lib, x, noalloc=True)
        ref = forward(lib, x, noalloc=False)
        rt = RTOL[x["dtype"]]
        assert torch.equal(got["p2g"], ref["p2g"]), f"call {i}: pred_to_gt differs"
        assert torch.equal(got["pr"], ref["pr"]), f"call {i}: pred_round differs"
        assert torch.equal(got["void"], ref["void"]) and got["void"].item() == 0
        assert (got["p2g"] >= 0).any(), f"call {i}: nothing matched"
        close(got["means"], ref["means"], rt, f"call {i} means")
        close(got["sep"], ref["sep"], rt, f"call {i} costs")
        s = x["shape"]
        nstat = s.L * s.B * s.Q * 4 + s.L * 2  # float head: per-query statistics, layer block
        close(got["saved"][:4 * nstat].view(torch.float32), ref["saved"][:4 * nstat].view(torch.float32),
              rt, f"call {i} saved statistics")


SCRATCH_BYTES = 128 << 20  # ML_NOALLOC_SCRATCH_BYTES (include/mask_loss_hip.h)


def test_noalloc_rejects_shapes_beyond_its_scratch(lib):
    # 128 label maps of 1024 x 1024: the forward's compact label map alone
    # ([B][H W] 16-bit labels, the cost contraction's column operand) is
    # twice the scratch array, checked here on the host before the call.
    # Null device pointers: the call must fail before any launch (and the
    # forward rejects null pointers itself if a shape ever passes the size check).
    s = Shape(1, 128, 100, 1024, 1024, 1024, 1024, 9, 250)
    assert s.B * s.Ht * s.Wt * 2 >= 2 * SCRATCH_BYTES
    p = params(9)
    assert lib.ml_mask_matching_forward_noalloc_bytes(ctypes.byref(s), ctypes.byref(p), ML_BF16) > SCRATCH_BYTES
    dummy = ctypes.c_void_p(0)
    rc = lib.ml_mask_matching_forward_noalloc(ctypes.byref(s), ctypes.byref(p), ML_BF16, dummy, dummy,
                                              ML_F32, dummy, dummy, dummy, dummy, dummy, None, None,
                                              None, None, None, None)
    assert rc == 4, rc  # ML_EUNSUPPORTED, before anything is launched
    assert b"scratch" in lib.ml_last_error()


def test_noalloc_unsupported_shape_codes_match(lib):
    """A shape the assignment does not take (Q = 1025) gives ML_EUNSUPPORTED
    from both forwards, before any launch (null pointers throughout)."""
    s = Shape(1, 2, 1025, 16, 16, 16, 16, 9, 7)
    p = params(9)
    dummy = ctypes.c_void_p(0)
    rc_na = lib.ml_mask_matching_forward_noalloc(ctypes.byref(s), ctypes.byref(p), ML_F32, dummy,
                                                 dummy, ML_F32, dummy, dummy, dummy, dummy, dummy,
                                                 None, None, None, None, None, None)
    err_na = lib.ml_last_error()
    rc_ws = lib.ml_mask_matching_forward(ctypes.byref(s), ctypes.byref(p), ML_F32, dummy, dummy,
                                         ML_F32, dummy, dummy, dummy, dummy, dummy, None, None, None,
                                         None, None, dummy, 1 << 20, None)
    err_ws = lib.ml_last_error()
    assert rc_na == rc_ws == 4, (rc_na, rc_ws)
    assert err_na == err_ws and b"1024 queries" in err_na


def test_noalloc_scratch_query(lib):
    """ml_mask_matching_forward_noalloc_bytes: the headline shape (B=16,
    Q=200, 256 x 256 bf16, 100 GT columns) fits the scratch array, a shape the
    assignment does not take reports 0, and the size grows with the batch."""
    p = params(133)
    q = lambda s, dt: lib.ml_mask_matching_forward_noalloc_bytes(ctypes.byref(s), ctypes.byref(p), dt)
    head = q(Shape(1, 16, 200, 256, 256, 256, 256, 134, 101), ML_BF16)
    assert 0 < head <= SCRATCH_BYTES, head
    assert q(Shape(1, 32, 200, 256, 256, 256, 256, 134, 101), ML_BF16) > head
    assert q(Shape(1, 2, 1025, 16, 16, 16, 16, 134, 7), ML_F32) == 0
    assert b"1024 queries" in lib.ml_last_error()


def test_noalloc_fitted_plan_large_shape(lib):
    """A cfg5-sized shape (8 images x 300 queries, 128 x 128 float32 logits,
    250 GT columns, 1,204 classes): with the device's full cost plan it needs
    more than the scratch array (146 MiB on MI355X), so the allocation-free
    forward sizes its plan for fewer resident slots (a smaller K-split).  Its
    costs agree with the workspace forward's to the float32 tolerance, and its
    assignment is the reference solver's on its own costs."""
    from oracle import assign as OA

    x = make_inputs(5, B=8, Q=300, H=128, W=128, G=250, C=1204, dtype=ML_F32)
    s, p = x["shape"], params(x["shape"].C)
    need = lib.ml_mask_matching_forward_noalloc_bytes(ctypes.byref(s), ctypes.byref(p), ML_F32)
    assert 0 < need <= SCRATCH_BYTES, need
    got = forward(lib, x, noalloc=True)
    ref = forward(lib, x, noalloc=False)
    close(got["sep"], ref["sep"], RTOL[ML_F32], "costs")
    close(got["means"], ref["means"], RTOL[ML_F32], "means")
    total = ((got["sep"][0] + got["sep"][1]) + got["sep"][2]).double().cpu().numpy().reshape(8, 300, 250)
    rp2g, rpr = OA.assign_batch(total, 1e30, 1, 0)
    assert np.array_equal(got["p2g"].cpu().numpy().reshape(8, 300), rp2g)
    assert np.array_equal(got["pr"].cpu().numpy().reshape(8, 300), rpr)
    assert (rp2g >= 0).any()
