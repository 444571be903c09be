"""Model integration: instance-level expert swaps (src/modeling of the reference)."""
