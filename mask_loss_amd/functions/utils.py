"""Point-sampling helpers with the reference's names and signatures
(functions/utils.py:6-54 of AndyBarcia/mask_loss), on the HIP point gather.

* ``point_sample``: bilinear sampling with ``torch.nn.functional.grid_sample``
  semantics at coordinates in [0, 1] (grid = 2 * coords - 1), zero padding
  (functions/utils.py:12-20), differentiable with respect to the sampled
  input (grid_sample's input gradient; the coordinates take no gradient).
* ``calculate_uncertainty``: -|logit| (functions/utils.py:6-9).
* ``get_uncertain_point_coords_with_randomness``: oversampled random points,
  the most uncertain ``importance_sample_ratio * num_points`` of them, plus
  fresh random points (functions/utils.py:23-54); the random draws are
  ``torch.rand`` on the logits' device, as in the reference.
"""
from __future__ import annotations

import torch
from torch.autograd import Function

import mask_loss_amd  # noqa: F401  (registers the `mask_loss` extension)
import mask_loss


class PointSampleFunction(Function):
    """Bilinear point sampling with its input gradient (HIP forward and
    backward); coordinates are constants."""

    @staticmethod
    def forward(ctx, input, coords, align_corners):
        ctx.save_for_backward(coords)
        ctx.hw = (input.shape[-2], input.shape[-1])
        ctx.align = bool(align_corners)
        return mask_loss.point_sample(input, coords, ctx.align)

    @staticmethod
    def backward(ctx, grad_out):
        (coords,) = ctx.saved_tensors
        g = mask_loss.point_sample_backward(grad_out.contiguous(), coords, ctx.hw[0], ctx.hw[1],
                                            ctx.align)
        return g, None, None


def calculate_uncertainty(logits):
    assert logits.shape[1] == 1
    return -(torch.abs(logits))


def point_sample(input, point_coords, **kwargs):
    """``input`` (N, C, H, W); ``point_coords`` (N, P, 2) -> (N, C, P), or
    (N, Hg, Wg, 2) -> (N, C, Hg, Wg).  Keyword arguments as grid_sample's:
    ``align_corners`` (default False); only mode="bilinear" and
    padding_mode="zeros" (grid_sample's defaults) are provided.  The result
    carries the gradient with respect to ``input``."""
    align = bool(kwargs.pop("align_corners", False) or False)
    mode = kwargs.pop("mode", "bilinear")
    padding = kwargs.pop("padding_mode", "zeros")
    if mode != "bilinear" or padding != "zeros":
        raise NotImplementedError("point_sample: only mode='bilinear', padding_mode='zeros'")
    if kwargs:
        raise TypeError(f"point_sample: unexpected arguments {sorted(kwargs)}")
    if point_coords.requires_grad and torch.is_grad_enabled():
        raise NotImplementedError("point_sample: no gradient with respect to the coordinates")
    coords = point_coords.detach().to(dtype=torch.float32).contiguous()
    if input.requires_grad and torch.is_grad_enabled():
        return PointSampleFunction.apply(input.contiguous(), coords, align)
    return mask_loss.point_sample(input.contiguous(), coords, align)


def get_uncertain_point_coords_with_randomness(
    coarse_logits,
    uncertainty_func,
    num_points,
    oversample_ratio,
    importance_sample_ratio,
):
    assert oversample_ratio >= 1
    assert importance_sample_ratio <= 1 and importance_sample_ratio >= 0
    num_boxes = coarse_logits.shape[0]
    num_sampled = int(num_points * oversample_ratio)
    point_coords = torch.rand(num_boxes, num_sampled, 2, device=coarse_logits.device)
    point_logits = point_sample(coarse_logits, point_coords, align_corners=False)
    point_uncertainties = uncertainty_func(point_logits)
    num_uncertain_points = int(importance_sample_ratio * num_points)
    num_random_points = num_points - num_uncertain_points
    idx = torch.topk(point_uncertainties[:, 0, :], k=num_uncertain_points, dim=1)[1]
    point_coords = torch.gather(point_coords, 1, idx[:, :, None].expand(-1, -1, 2))
    if num_random_points > 0:
        point_coords = torch.cat(
            [point_coords,
             torch.rand(num_boxes, num_random_points, 2, device=coarse_logits.device)],
            dim=1)
    return point_coords


def shared_point_coords(B, num_points, device, targets=None, background_index=None):
    """One point set per image, (B, P, 2), with the reference's draws
    (functions/sigmoid/pw_sigmoid_ce.py:465-486, functions/dice/pw_dice_loss.py:206-232):
    ``torch.rand(1, P, 2)`` per image, in image order, only for the images the
    reference draws for -- none when the label maps hold no GT class
    (targets.max() + 1 <= 0, or only the background class), else every image
    with a label other than ``background_index``.  The other images' rows are
    zero; their costs are +inf whatever the points.  Without ``targets`` every
    image draws.  Deciding which images draw reads the label maps back to the
    host, as the reference's torch.unique does."""
    if B == 0:
        return torch.empty(0, num_points, 2, device=device)
    draw = [True] * B
    if targets is not None:
        t = targets.reshape(B, -1)
        gt_all = int(t.max().item()) + 1 if t.numel() else 0
        G = gt_all - (1 if background_index is not None and 0 <= background_index < gt_all else 0)
        if gt_all <= 0 or G <= 0:
            draw = [False] * B
        elif background_index is not None:
            draw = (t != background_index).any(dim=1).tolist()
    rows = [torch.rand(1, num_points, 2, device=device) if d
            else torch.zeros(1, num_points, 2, device=device) for d in draw]
    return torch.cat(rows, dim=0)
