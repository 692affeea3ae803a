"""Optimizers of the MI355X optimizer-step path (namitorch/optim)."""

from .adam import Adam, AdamW
from .clip_grad import clip_grad_norm_, clip_grad_value_, get_grad_norm
from .optimizer import Optimizer

__all__ = ["Optimizer", "Adam", "AdamW", "clip_grad_norm_", "clip_grad_value_", "get_grad_norm"]
