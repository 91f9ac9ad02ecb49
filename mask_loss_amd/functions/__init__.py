"""Autograd front-ends with the reference's names and signatures
(functions/__init__.py of AndyBarcia/mask_loss), backed by the HIP extension.

The Function classes of the reference's compiled operators are provided; each
runs on the GPU through ``mask_loss``.  The reference's pure-PyTorch ``*_py``
restatements are not part of this package (their float64 counterparts live in
the test oracle)."""
from .sigmoid.sigmoid_ce import SigmoidCELossFunction
from .dice.dice_loss import DiceLossFunction
from .sigmoid.pw_sigmoid_ce import PairwiseSigmoidCELossFunction
from .dice.pw_dice_loss import PairwiseDiceLossFunction
from .label.pw_sigmoid_label_loss import PairwiseSigmoidLabelLossFunction
from .label.pw_softmax_label_loss import PairwiseSoftmaxLabelLossFunction, pairwise_softmax_label_loss
from .mask.pw_mask import PairwiseMaskLossFunction
from .mask.matching import MaskMatchingFunction

__all__ = [
    "SigmoidCELossFunction",
    "DiceLossFunction",
    "PairwiseSigmoidCELossFunction",
    "PairwiseDiceLossFunction",
    "PairwiseSigmoidLabelLossFunction",
    "PairwiseSoftmaxLabelLossFunction",
    "pairwise_softmax_label_loss",
    "PairwiseMaskLossFunction",
    "MaskMatchingFunction",
]
