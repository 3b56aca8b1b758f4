"""momij_amd -- MI355X-native speculative-decode verify step (HIP kernels behind a C ABI)."""
