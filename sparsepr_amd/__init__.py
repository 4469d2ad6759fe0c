"""SparsePR sparse-attention hot path, MI355X-native (gfx950 HIP kernels behind a C ABI).

Subpackages mirror the reference's public modules:
  sparsepr_amd.flash_kmeans      <- flash_kmeans
  sparsepr_amd.kmeans_utils      <- sparsepr.kmeans_utils
  sparsepr_amd.kernels.*         <- sparsepr.kernels.triton.* and sparsepr.kernels.n8_extension
"""

__version__ = "0.1.0"
