"""End-to-end layer-swap harness (the reference's kernels/e2e): a Qwen2 runner with swappable
linear / norm / activation backends, hipGraph decode and the per-layer timing."""
