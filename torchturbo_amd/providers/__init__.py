"""Operator providers. ``hip`` holds the MI355X (gfx950) kernels."""
