"""HIP-backed replacements for the reference's kernel modules (src/sparsepr/kernels/)."""
