"""Carry the denoising timestep from a transformer's forward into its attention processors.

The reference reaches this by replacing diffusers' WanTransformerBlock /
WanTransformer3DModel forwards (svg/models/wan/custom_models.py:23-207) and the
HunyuanVideo block and model forwards (svg/models/hyvideo/custom_models.py:16-263)
with copies that pass ``timestep=`` down to ``attn(...)``.  This build does not
carry copies of diffusers' model code.  Instead, ``install`` wraps the model
class's ``forward`` so that the timestep of the running call sits in a context
variable, and the PASA processors read it when they are called without one.

Only self-attention reads it: a Wan processor called with encoder states (the
cross-attention ``attn2``) keeps the dense path, as in the reference, where
only ``attn1`` receives the timestep.
"""
from __future__ import annotations

import contextvars
import functools
from typing import Any, Optional

_TIMESTEP: contextvars.ContextVar = contextvars.ContextVar("pasa_timestep", default=None)


def current_timestep() -> Optional[Any]:
    """The timestep of the transformer forward running on this thread, or None."""
    return _TIMESTEP.get()


def wrap_forward(cls, timestep_arg: int = 1) -> bool:
    """Wrap ``cls.forward`` so its timestep argument is visible to the processors.

    ``timestep_arg`` is the position of ``timestep`` in forward's signature after
    ``self`` minus one (``forward(self, hidden_states, timestep, ...)`` -> 1); it is
    also found by keyword.  Wrapping twice is a no-op."""
    orig = cls.forward
    if getattr(orig, "_pasa_timestep_wrapped", False):
        return True

    @functools.wraps(orig)
    def forward(self, *args, **kwargs):
        ts = kwargs.get("timestep", args[timestep_arg] if len(args) > timestep_arg else None)
        token = _TIMESTEP.set(ts)
        try:
            return orig(self, *args, **kwargs)
        finally:
            _TIMESTEP.reset(token)

    forward._pasa_timestep_wrapped = True
    cls.forward = forward
    return True


def install_wan() -> bool:
    """Hook diffusers' WanTransformer3DModel; False when diffusers is not importable."""
    try:
        from diffusers.models.transformers.transformer_wan import WanTransformer3DModel
    except ImportError:
        return False
    return wrap_forward(WanTransformer3DModel)


def install_hunyuan() -> bool:
    """Hook diffusers' HunyuanVideoTransformer3DModel; False when diffusers is not importable."""
    try:
        from diffusers.models.transformers.transformer_hunyuan_video import HunyuanVideoTransformer3DModel
    except ImportError:
        return False
    return wrap_forward(HunyuanVideoTransformer3DModel)
