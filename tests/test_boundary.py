"""CPU checks of the drop-in boundary: the C-ABI library exports every symbol
declared in include/mask_loss_hip.h, the `mask_loss` module exposes the
reference's operator names, and host tensors are rejected (there is no CPU
implementation behind the boundary)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mask_loss_hip.h")
LIB = os.path.join(ROOT, "mask_loss_amd", "libmask_loss_hip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ml_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ["ml_mask_matching_forward", "ml_mask_matching_backward",
              "ml_pairwise_mask_loss_forward", "ml_pairwise_label_loss_forward",
              "ml_last_error", "ml_mask_matching_workspace_size"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (shares one HIP runtime with the library)
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    lib = ctypes.CDLL(LIB)
    for n in declared_functions():
        assert hasattr(lib, n), f"{n} not exported"
    lib.ml_version.restype = ctypes.c_int
    assert lib.ml_version() >= 1


def test_workspace_query_rejects_bad_shapes():
    import torch  # noqa: F401
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    lib = ctypes.CDLL(LIB)

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

    lib.ml_mask_matching_workspace_size.restype = ctypes.c_size_t
    p = Params(1, 1, 1, 1, 0, 1, 0.05, 1e30, -1, 1, 0, 1, 0, 0, -1, 0, -1, 133, 1, 1)
    good = Shape(1, 16, 200, 256, 256, 256, 256, 134, 101)
    assert lib.ml_mask_matching_workspace_size(ctypes.byref(good), ctypes.byref(p), 1) > 0
    bad = Shape(1, 16, 200, 256, 256, 300, 256, 134, 101)  # not an integer multiple
    assert lib.ml_mask_matching_workspace_size(ctypes.byref(bad), ctypes.byref(p), 1) == 0


def test_extension_surface_and_host_tensors_rejected():
    import torch
    import mask_loss_amd
    ml = mask_loss_amd.mask_loss
    # the reference module's 11 operators (src/bindings.cpp:157-169)
    for n in ["forward_sigmoid_ce_loss", "backward_sigmoid_ce_loss", "forward_pw_sigmoid_ce_loss",
              "forward_dice_loss", "backward_dice_loss", "forward_pw_dice_loss",
              "pairwise_mask_loss_forward", "mask_matching", "mask_matching_backward",
              "forward_pw_sigmoid_label_loss", "forward_pw_softmax_label_loss"]:
        assert hasattr(ml, n)
    z = torch.zeros(1, 1, 2, 4, 4)
    t = torch.zeros(1, 4, 4, dtype=torch.long)
    zc = torch.zeros(1, 1, 2, 3)
    ct = torch.zeros(1, 2, dtype=torch.long)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.mask_matching(z, t, zc, ct, 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, 1e30, -1.0, False,
                         False, 1, 0, 0.0, -1.0, 0.0, -1.0, -1, False, True)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.pairwise_mask_loss_forward(z, t, zc, ct, 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, 0.0, -1.0,
                                      0.0, -1.0, False, True)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.forward_sigmoid_ce_loss(z, t, 1.0, 1.0, 0.0, -1.0)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.forward_dice_loss(z, t, 1.0, 1.0, 1.0)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.forward_pw_dice_loss(z, t, 1.0, -1, 1.0, 1.0, 0.05)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.forward_pw_sigmoid_ce_loss(z, t, -1, 1.0, 0.0, -1.0, 1.0, 0.05, True)


def test_dense_workspace_query():
    import torch  # noqa: F401
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    lib = ctypes.CDLL(LIB)

    class DShape(ctypes.Structure):
        _fields_ = [(k, ctypes.c_int64) for k in ["L", "B", "C", "H", "W", "Ht", "Wt"]]

    lib.ml_dense_loss_workspace_size.restype = ctypes.c_size_t
    good = DShape(1, 2, 133, 64, 64, 256, 256)
    for dice in (0, 1):
        for bwd in (0, 1):
            assert lib.ml_dense_loss_workspace_size(ctypes.byref(good), 1, dice, bwd) > 0
    assert lib.ml_dense_loss_workspace_size(ctypes.byref(DShape(1, 2, 4, 64, 64, 256, 250)), 1, 0, 0) == 0
    # s = 16 and s = 17 take 16-bit counts (twice the bytes of s = 15's 8-bit ones);
    # s = 256 does not fit them
    w15 = lib.ml_dense_loss_workspace_size(ctypes.byref(DShape(1, 2, 4, 4, 4, 60, 60)), 1, 0, 1)
    w16 = lib.ml_dense_loss_workspace_size(ctypes.byref(DShape(1, 2, 4, 4, 4, 64, 64)), 1, 0, 1)
    assert w15 > 0 and w16 == 2 * w15
    assert lib.ml_dense_loss_workspace_size(ctypes.byref(DShape(1, 2, 4, 4, 4, 68, 68)), 1, 0, 0) > 0
    assert lib.ml_dense_loss_workspace_size(ctypes.byref(DShape(1, 2, 4, 1, 1, 256, 256)), 1, 0, 0) == 0


def test_point_sampling_queries_and_host_tensors_rejected():
    """The front end's size queries accept only the (L,B,C,1,P) sampled shape
    and valid planes; its operators reject host tensors (no CPU path)."""
    import torch
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    lib = ctypes.CDLL(LIB)

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

    q = lib.ml_pairwise_points_workspace_size
    q.restype = ctypes.c_size_t
    q.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    p = Params(1, 1, 1, 1, 0, 0, 0, 1e30, -1, 0, 0, 1, 0, 0, -1, 0, -1, -1, 0, 0)
    good = Shape(1, 8, 100, 1, 12544, 1, 12544, 0, 51)
    assert q(ctypes.byref(good), ctypes.byref(p), 0, 512, 512) > 0
    assert q(ctypes.byref(Shape(1, 8, 100, 2, 12544, 2, 12544, 0, 51)), ctypes.byref(p), 0, 512, 512) == 0
    assert q(ctypes.byref(good), ctypes.byref(p), 0, 0, 512) == 0
    b = lib.ml_point_sample_backward_workspace_size
    b.restype = ctypes.c_size_t
    b.argtypes = [ctypes.c_int] + [ctypes.c_int64] * 6
    # grouped form ((H+1)(W+1) <= 16,900 buckets, <= 16,384 points, >= 8
    # planes per coordinate set): per set, the bucket offsets, then P point
    # indices and P float4 corner weights (each region 256-byte aligned)
    a256 = lambda x: (x + 255) // 256 * 256
    assert b(0, 8, 100, 128, 128, 12544, 8) == (a256(8 * (129 * 129 + 1) * 4) + a256(8 * 12544 * 4)
                                                + 8 * 12544 * 16)
    assert b(0, 2, 3, 16, 16, 100, 2) == 0                     # < 8 planes: LDS atomics
    assert b(0, 2, 8, 128, 128, 17000, 2) == 0                 # > 16,384 points: LDS atomics
    assert b(0, 2, 3, 130, 140, 100, 2) == 2 * 3 * 130 * 140 * 4  # float workspace
    assert b(7, 2, 3, 130, 140, 100, 2) == 0                   # unknown dtype
    assert b(0, 2, 3, 130, 140, 100, 0) == 0                   # no coordinate set
    import mask_loss_amd
    ml = mask_loss_amd.mask_loss
    x = torch.zeros(2, 3, 4, 4)
    c = torch.zeros(2, 5, 2)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.point_sample(x, c, False)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.point_labels(torch.zeros(2, 4, 4, dtype=torch.long), c)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ml.forward_pw_dice_loss_sampling(torch.zeros(1, 2, 3, 4, 4), torch.zeros(2, 8, 8, dtype=torch.long),
                                         c, 1.0, -1, 1.0, False)


def test_function_validation_errors():
    import torch
    from mask_loss_amd.functions import MaskMatchingFunction
    z = torch.zeros(1, 1, 2, 4, 4)
    t = torch.zeros(1, 4, 4, dtype=torch.long)
    zc = torch.zeros(1, 1, 2, 3)
    ct = torch.zeros(1, 2, dtype=torch.long)
    base = [z, t, zc, ct, 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, True, 1e30, -1.0, False, False, 1,
            "global", 0.0, None, 0.0, None, None, "sigmoid"]

    def call(**over):
        names = ["mask_logits", "mask_targets", "cls_logits", "cls_targets", "smooth",
                 "sigmoid_scale", "dice_scale", "cls_scale", "background_index",
                 "uncertainty_gamma", "uncertainty_gamma_min", "normalize_uncertainty",
                 "inf_thresh", "num_masks", "force_bg", "force_empty", "K", "strategy",
                 "mask_gamma", "mask_alpha", "cls_gamma", "cls_alpha", "void", "label_loss"]
        args = list(base)
        for k, v in over.items():
            args[names.index(k)] = v
        return MaskMatchingFunction.apply(*args)

    with pytest.raises(ValueError, match="assignment_strategy"):
        call(strategy="hungarian")
    with pytest.raises(ValueError, match="K must be"):
        call(K=-1)
    with pytest.raises(ValueError, match="uncertainty_gamma_min"):
        call(uncertainty_gamma_min=1.5)
    with pytest.raises(ValueError, match="void index"):
        call(void=7)
    with pytest.raises(ValueError, match="void_class_index must be provided"):
        call(label_loss="softmax", force_bg=True)
    with pytest.raises(ValueError, match="label_loss"):
        call(label_loss="hinge")
    with pytest.raises(ValueError, match="focal_alpha"):
        call(mask_alpha=2.0)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        call()


def test_losses_dispatcher_argument_errors():
    """functions/losses.py:8-67: the branches whose operators the reference's
    sources lack, and malformed arguments, raise before any GPU work; every
    implementation value but "python" goes to the GPU operator."""
    import torch
    from mask_loss_amd.functions import losses
    z = torch.zeros(2, 3, 4, 4)
    t = torch.zeros(2, 8, 8, dtype=torch.long)
    for fn in (losses.sigmoid_cross_entropy_loss, losses.dice_loss):
        with pytest.raises(NotImplementedError, match="multi-class"):
            fn(z, t, class_mapping=torch.arange(256))
        with pytest.raises(NotImplementedError, match="pure-PyTorch"):
            fn(z, t, implementation="python")
        # any other value selects the GPU operator, as in the reference, so
        # host tensors are rejected by it
        with pytest.raises(RuntimeError, match="CUDA tensor"):
            fn(z, t, implementation="triton")
        with pytest.raises(ValueError, match="logits must be"):
            fn(z[0], t)
