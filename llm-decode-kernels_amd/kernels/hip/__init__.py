"""Native decode entry point (the counterpart of the reference's `kernels/cuda` package)."""
