"""Verify-step callers: the fused MoE verify layer and greedy / p-q acceptance."""
