"""Autograd front-ends with the reference's names and signatures
(functions/__init__.py of AndyBarcia/mask_loss), backed by the HIP extension.

The Function classes of the reference's compiled operators are provided; each
runs on the GPU through ``mask_loss``.  The reference's pure-PyTorch ``*_py``
restatements are not part of this package (their float64 counterparts live in
the test oracle), except the point-sampled pairwise costs, which the reference
exports under their ``*_sampling_py`` names and which run here on the HIP
point gather.  The loss dispatchers of functions/losses.py
(``sigmoid_cross_entropy_loss``, ``dice_loss``) call the count-based Functions."""
from .sigmoid.sigmoid_ce import SigmoidCELossFunction
from .dice.dice_loss import DiceLossFunction
from .sigmoid.pw_sigmoid_ce import (PairwiseSigmoidCELossFunction,
                                    pairwise_sigmoid_cross_entropy_loss_sampling_py)
from .dice.pw_dice_loss import PairwiseDiceLossFunction, pairwise_dice_loss_sampling_py
from .utils import (calculate_uncertainty, get_uncertain_point_coords_with_randomness,
                    point_sample)
from .label.pw_sigmoid_label_loss import PairwiseSigmoidLabelLossFunction
from .label.pw_softmax_label_loss import PairwiseSoftmaxLabelLossFunction, pairwise_softmax_label_loss
from .mask.pw_mask import PairwiseMaskLossFunction
from .mask.matching import MaskMatchingFunction
from .losses import sigmoid_cross_entropy_loss, dice_loss

__all__ = [
    "sigmoid_cross_entropy_loss",
    "dice_loss",
    "SigmoidCELossFunction",
    "DiceLossFunction",
    "PairwiseSigmoidCELossFunction",
    "PairwiseDiceLossFunction",
    "PairwiseSigmoidLabelLossFunction",
    "PairwiseSoftmaxLabelLossFunction",
    "pairwise_softmax_label_loss",
    "PairwiseMaskLossFunction",
    "MaskMatchingFunction",
    "pairwise_sigmoid_cross_entropy_loss_sampling_py",
    "pairwise_dice_loss_sampling_py",
    "point_sample",
    "calculate_uncertainty",
    "get_uncertain_point_coords_with_randomness",
]
