"""Scalar CPU oracle of the NeRF hot path (test infrastructure only)."""
