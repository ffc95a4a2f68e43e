"""HIP-backed replacements of anima-flat's src/kernels modules on the attention path."""
