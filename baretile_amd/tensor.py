"""Placeholder until the Tensor surface lands."""
