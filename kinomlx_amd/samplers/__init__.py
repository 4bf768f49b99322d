"""Diffusion sampler steps on MI355X (mirror of ``kinomlx/samplers``)."""

from .steps import euler_step, euler_velocity_step

__all__ = ["euler_step", "euler_velocity_step"]
