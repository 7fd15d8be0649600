"""Sparse decode reader: read plans, resident ternary sketch and the HIP operator."""
