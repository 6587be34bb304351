"""Operators and engine packs backed by libsdv's gfx950 kernels."""
