"""Kernel ops. ``hip`` holds the gfx950 HIP kernels behind a C ABI (include/nanonemo_fa.h)."""
