"""Loaders with the reference signatures (src/kops/registry/<slug>.py)."""
