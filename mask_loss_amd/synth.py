"""Synthetic inputs for the benchmark configurations (no datasets exist here).

Recipe (shared by tests, ``__graft_entry__.smoke`` and ``bench.py``):

* NumPy ``Generator(PCG64(seed))``; L = 1 decoder layer; targets at the logit
  grid (s = 1) unless ``scale`` is given.
* Label map with background label 0, GTs painted in order g = 1..G_b (later
  shapes overwrite earlier ones, so some GTs may vanish): ellipses (uniform
  centre, area fraction as configured, aspect U[0.5, 2], angle U[0, pi)) or
  star-shaped polygons (5-12 vertices at random radii, scaled to the area).
* ``cls_targets``: (B, G_max + 1) int64; column 0 = -1 (the background slot,
  dropped with ``background_index = 0``); columns 1..G_b ~ U{0..C-1}; -1
  padding.  Class logits have C + 1 channels, the last one being the
  no-object ("void") class.
* Mask logits ~ N(0, sigma) (sigma read as the standard deviation) drawn in
  float32 and rounded to the configured dtype (bf16 round-to-nearest-even).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import numpy as np


@dataclass(frozen=True)
class Config:
    name: str
    B: int
    Q: int
    H: int
    W: int
    G: tuple                # (G_min, G_max) per image
    C: int                  # real classes (+1 void channel added)
    dtype: str              # "float32" | "bfloat16"
    sigma: float
    area: tuple             # area fraction range per shape
    shapes: str             # "ellipse" | "polygon" | "mixed"
    cls_mean: float = 0.0
    scale: int = 1          # target / logit resolution factor
    seed: int = 0
    L: int = 1
    # operator arguments (the reference's own test_mask_matching choices,
    # benchmarks.py:560-578)
    kwargs: dict = field(default_factory=lambda: dict(
        smooth=1.0, sigmoid_scale=1.0, dice_scale=1.0, cls_scale=1.0, background_index=0,
        uncertainty_gamma=1.0, uncertainty_gamma_min=0.05, normalize_uncertainty=True,
        inf_thresh=1e30, num_masks=-1.0, force_unmatched_class_to_background=True,
        force_unmatched_masks_to_empty=False, K=1, assignment_strategy="global",
        mask_focal_gamma=0.0, mask_focal_alpha=None, cls_focal_gamma=0.0, cls_focal_alpha=None,
        label_loss="softmax"))


CONFIGS = [
    Config("cfg1_cpu_ref", B=2, Q=100, H=64, W=64, G=(8, 8), C=80, dtype="float32", sigma=2.0,
           area=(0.02, 0.30), shapes="ellipse", seed=1),
    Config("cfg2_point_sampled", B=8, Q=100, H=112, W=112, G=(1, 50), C=133, dtype="float32",
           sigma=2.0, area=(0.005, 0.30), shapes="ellipse", seed=2),
    Config("cfg3_dense_headline", B=16, Q=200, H=256, W=256, G=(5, 100), C=133,
           dtype="bfloat16", sigma=3.0, area=(0.005, 0.40), shapes="polygon", seed=3),
    Config("cfg4_high_res", B=4, Q=200, H=512, W=512, G=(100, 100), C=150, dtype="bfloat16",
           sigma=3.0, area=(0.02, 0.40), shapes="mixed", seed=4),
    Config("cfg5_large_query", B=8, Q=300, H=128, W=128, G=(50, 250), C=1203, dtype="float32",
           sigma=2.0, area=(0.0005, 0.02), shapes="mixed", cls_mean=-4.0, seed=5),
]
BY_NAME = {c.name: c for c in CONFIGS}
HEADLINE = BY_NAME["cfg3_dense_headline"]


def shrink(cfg: Config, **kw) -> Config:
    """Same recipe at another size (test cases)."""
    return replace(cfg, **kw)


def _ellipse(rng, H, W, frac):
    A = frac * H * W
    rho = rng.uniform(0.5, 2.0)
    a = math.sqrt(A * rho / math.pi)
    b = math.sqrt(A / (math.pi * rho))
    th = rng.uniform(0.0, math.pi)
    cy, cx = rng.uniform(0, H), rng.uniform(0, W)
    R = max(a, b) + 1
    y0, y1 = max(0, int(cy - R)), min(H, int(cy + R) + 1)
    x0, x1 = max(0, int(cx - R)), min(W, int(cx + R) + 1)
    if y0 >= y1 or x0 >= x1:
        return None
    yy, xx = np.mgrid[y0:y1, x0:x1]
    dy, dx = yy + 0.5 - cy, xx + 0.5 - cx
    u = dx * math.cos(th) + dy * math.sin(th)
    v = -dx * math.sin(th) + dy * math.cos(th)
    return (y0, y1, x0, x1, (u / a) ** 2 + (v / b) ** 2 <= 1.0)


def _polygon(rng, H, W, frac):
    k = int(rng.integers(5, 13))
    ang = np.sort(rng.uniform(0.0, 2 * math.pi, size=k))
    rad = rng.uniform(0.5, 1.0, size=k)
    area_unit = 0.5 * np.sum(rad * np.roll(rad, -1) * np.sin(np.roll(ang, -1) - ang + 2 * math.pi * (np.arange(k) == k - 1)))
    area_unit = max(area_unit, 1e-3)
    s = math.sqrt(frac * H * W / area_unit)
    cy, cx = rng.uniform(0, H), rng.uniform(0, W)
    py = cy + s * rad * np.sin(ang)
    px = cx + s * rad * np.cos(ang)
    y0, y1 = max(0, int(py.min())), min(H, int(py.max()) + 2)
    x0, x1 = max(0, int(px.min())), min(W, int(px.max()) + 2)
    if y0 >= y1 or x0 >= x1:
        return None
    yy, xx = np.mgrid[y0:y1, x0:x1]
    Y, X = yy + 0.5, xx + 0.5
    inside = np.zeros(Y.shape, dtype=bool)
    for i in range(k):
        ay, ax, by, bx = py[i], px[i], py[(i + 1) % k], px[(i + 1) % k]
        cond = (ay > Y) != (by > Y)
        with np.errstate(divide="ignore", invalid="ignore"):
            xint = ax + (Y - ay) * (bx - ax) / (by - ay)
        inside ^= cond & (X < xint)
    return (y0, y1, x0, x1, inside)


def make_targets(cfg: Config, rng: np.random.Generator):
    """(mask_targets (B,Ht,Wt) int64, cls_targets (B, G_max+1) int64, G per image)."""
    Ht, Wt = cfg.H * cfg.scale, cfg.W * cfg.scale
    gmin, gmax = cfg.G
    tgt = np.zeros((cfg.B, Ht, Wt), dtype=np.int64)
    cls = np.full((cfg.B, gmax + 1), -1, dtype=np.int64)
    Gs = []
    for b in range(cfg.B):
        Gb = int(rng.integers(gmin, gmax + 1))
        Gs.append(Gb)
        for g in range(1, Gb + 1):
            frac = rng.uniform(*cfg.area)
            kind = cfg.shapes
            if kind == "mixed":
                kind = "ellipse" if rng.uniform() < 0.5 else "polygon"
            shp = _ellipse(rng, Ht, Wt, frac) if kind == "ellipse" else _polygon(rng, Ht, Wt, frac)
            if shp is None:
                continue
            y0, y1, x0, x1, m = shp
            tgt[b, y0:y1, x0:x1][m] = g
        cls[b, 1:Gb + 1] = rng.integers(0, cfg.C, size=Gb)
    return tgt, cls, Gs


def make_numpy(cfg: Config):
    """All inputs as float32 / int64 NumPy arrays (mask logits already rounded
    to the configured dtype's values)."""
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    tgt, cls_t, Gs = make_targets(cfg, rng)
    z = rng.standard_normal((cfg.L, cfg.B, cfg.Q, cfg.H, cfg.W), dtype=np.float32) * np.float32(cfg.sigma)
    if cfg.dtype == "bfloat16":
        z = round_bf16(z)
    zc = (rng.standard_normal((cfg.L, cfg.B, cfg.Q, cfg.C + 1), dtype=np.float32)
          + np.float32(cfg.cls_mean))
    return dict(mask_logits=z, mask_targets=tgt, cls_logits=zc, cls_targets=cls_t, G=Gs)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 value (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def make_torch(cfg: Config, device="cuda", logits_on_device_rng=False):
    """Inputs as torch tensors on `device`.  With ``logits_on_device_rng`` the
    (large) mask logits are drawn by torch's generator on the device (seeded
    with cfg.seed) instead of NumPy -- used by the benchmark at full size."""
    import torch
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    tgt, cls_t, Gs = make_targets(cfg, rng)
    tdt = {"float32": torch.float32, "bfloat16": torch.bfloat16}[cfg.dtype]
    if logits_on_device_rng:
        g = torch.Generator(device=device)
        g.manual_seed(cfg.seed)
        z = torch.randn((cfg.L, cfg.B, cfg.Q, cfg.H, cfg.W), generator=g, device=device,
                        dtype=torch.float32).mul_(cfg.sigma).to(tdt)
        zc = (torch.randn((cfg.L, cfg.B, cfg.Q, cfg.C + 1), generator=g, device=device,
                          dtype=torch.float32) + cfg.cls_mean)
    else:
        z_np = rng.standard_normal((cfg.L, cfg.B, cfg.Q, cfg.H, cfg.W), dtype=np.float32) * np.float32(cfg.sigma)
        z = torch.from_numpy(z_np).to(device).to(tdt)
        zc = torch.from_numpy(rng.standard_normal((cfg.L, cfg.B, cfg.Q, cfg.C + 1), dtype=np.float32)
                              + np.float32(cfg.cls_mean)).to(device)
    return dict(mask_logits=z.contiguous(), mask_targets=torch.from_numpy(tgt).to(device),
                cls_logits=zc.contiguous(), cls_targets=torch.from_numpy(cls_t).to(device), G=Gs)


def call_args(cfg: Config, x: dict):
    """Positional arguments of MaskMatchingFunction.apply for inputs x."""
    k = cfg.kwargs
    void = cfg.C  # last channel
    return (x["mask_logits"], x["mask_targets"], x["cls_logits"], x["cls_targets"], k["smooth"],
            k["sigmoid_scale"], k["dice_scale"], k["cls_scale"], k["background_index"],
            k["uncertainty_gamma"], k["uncertainty_gamma_min"], k["normalize_uncertainty"],
            k["inf_thresh"], k["num_masks"], k["force_unmatched_class_to_background"],
            k["force_unmatched_masks_to_empty"], k["K"], k["assignment_strategy"],
            k["mask_focal_gamma"], k["mask_focal_alpha"], k["cls_focal_gamma"],
            k["cls_focal_alpha"], void, k["label_loss"])
