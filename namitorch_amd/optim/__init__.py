"""Optimizers of the MI355X optimizer-step path (namitorch/optim)."""

from .adam import Adam, AdamW
from .clip_grad import clip_grad_norm_, clip_grad_value_, get_grad_norm
from .lr_scheduler import (CosineAnnealingLR, ExponentialLR, LinearLR, LRScheduler, MultiStepLR, StepLR,
                           WarmupCosine)
from .optimizer import Optimizer

__all__ = ["Optimizer", "Adam", "AdamW", "clip_grad_norm_", "clip_grad_value_", "get_grad_norm", "LRScheduler",
           "StepLR", "MultiStepLR", "ExponentialLR", "CosineAnnealingLR", "LinearLR", "WarmupCosine"]
