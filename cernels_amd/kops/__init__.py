"""Kernel ops: loaders in ``kops.registry`` mirror src/kops/registry of the reference."""
