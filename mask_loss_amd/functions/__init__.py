"""Autograd front-ends with the reference's names and signatures
(functions/__init__.py of AndyBarcia/mask_loss), backed by the HIP extension.

Only the Function classes of the fused mask-cost -> matching -> loss path are
provided; every one of them runs on the GPU through ``mask_loss``."""
from .mask.matching import MaskMatchingFunction
from .mask.pw_mask import PairwiseMaskLossFunction
from .label.pw_sigmoid_label_loss import PairwiseSigmoidLabelLossFunction
from .label.pw_softmax_label_loss import PairwiseSoftmaxLabelLossFunction, pairwise_softmax_label_loss

__all__ = [
    "MaskMatchingFunction",
    "PairwiseMaskLossFunction",
    "PairwiseSigmoidLabelLossFunction",
    "PairwiseSoftmaxLabelLossFunction",
    "pairwise_softmax_label_loss",
]
