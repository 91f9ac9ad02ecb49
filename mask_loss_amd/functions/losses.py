"""Loss dispatchers with the reference's names and signatures
(functions/losses.py:8-67 of AndyBarcia/mask_loss).

Each runs the count-based operator on the GPU through ``mask_loss``
(SigmoidCELossFunction, DiceLossFunction).  The reference's dispatchers also
name multi-class operators (``class_mapping``) and pure-PyTorch restatements
(``implementation="python"``) from modules its sources do not contain
(functions/losses.py:1-5 imports ``.sigmoid_ce``, ``.mc_sigmoid_ce``,
``.dice.dice_loss``'s ``dice_loss_efficient_py`` and ``.mc_dice``, none of
which exist there), so those branches raise NotImplementedError here instead
of an ImportError at import time.

Logits may be (B, C, h, w), as the reference's docstrings state, giving a
scalar, or (L, B, C, h, w), as its Function classes take, giving one loss per
layer."""
from .sigmoid.sigmoid_ce import SigmoidCELossFunction
from .dice.dice_loss import DiceLossFunction


def _check(implementation, class_mapping, who):
    # as the reference's dispatchers (functions/losses.py:24-33, 57-67): every
    # value other than "python" selects the GPU operator
    if class_mapping is not None:
        raise NotImplementedError(
            f"{who}: class_mapping selects the reference's multi-class operators, which are not part of "
            "its sources")
    if implementation == "python":
        raise NotImplementedError(
            f"{who}: the reference's pure-PyTorch restatement is not part of its sources; "
            "implementation='cuda' runs the operator on the GPU")


def _layers(logits):
    if logits.dim() == 4:
        return logits.unsqueeze(0), True
    if logits.dim() == 5:
        return logits, False
    raise ValueError(f"logits must be (B, C, h, w) or (L, B, C, h, w), got {tuple(logits.shape)}")


def sigmoid_cross_entropy_loss(logits, targets, class_mapping=None, num_masks=None,
                               implementation="cuda", scale=1.0):
    """Count-based BCE-with-logits of nearest-upsampled logits against every
    class's binary mask (functions/losses.py:8-33).  targets: (B, H, W)
    integer labels.  num_masks defaults to the number of (layer, image,
    class) masks; the loss sums over cells, divided by num_masks * H * W,
    times scale."""
    _check(implementation, class_mapping, "sigmoid_cross_entropy_loss")
    x, single = _layers(logits)
    out = SigmoidCELossFunction.apply(x, targets, num_masks, scale, None, None)
    return out[0] if single else out


def dice_loss(logits, targets, smooth=1e-6, class_mapping=None, num_masks=None,
              implementation="cuda", scale=1.0):
    """Count-based Dice loss of nearest-upsampled logits against every class's
    binary mask (functions/losses.py:36-67): H and W are integer multiples of
    h and w, so each s x s block shares one logit.  Returns the sum over
    masks of (1 - dice), divided by num_masks, times scale."""
    _check(implementation, class_mapping, "dice_loss")
    x, single = _layers(logits)
    out = DiceLossFunction.apply(x, targets, smooth, num_masks, scale)
    return out[0] if single else out
