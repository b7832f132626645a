"""Observation innovation and capped parameter update."""

from .observation import compute_innovation, compute_innovation_with_indices, hrc_innovation
from .parameters import get_cap_factor, update_parameters, update_parameters_multi

__all__ = ["compute_innovation", "get_cap_factor", "update_parameters", "update_parameters_multi"]
