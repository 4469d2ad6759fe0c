"""FlashKMeans estimator (reference flash_kmeans/interface.py:27-287) on the HIP kernels."""

from __future__ import annotations

from typing import Optional

import torch

from .kmeans_impl import X_SQ_BF16, euclid_assign, lloyd


class FlashKMeans:
    """Batched K-Means on the GPU.  d: features, k: clusters, niter: max
    iterations, tol: stop when the max centroid shift drops below it, seed:
    seeds the random initialisation.  CPU-resident data larger than
    chunk_size_data_cpu (the reference's multi-GPU streaming path) is not
    supported here and raises."""

    def __init__(self, d: int, k: int, niter: int = 25, tol: float = 1e-8, use_triton: bool = True,
                 seed: int = 0, chunk_size_data: int = 32768, chunk_size_centroids: int = 1024,
                 chunk_size_data_cpu: int = 1048576, verbose: bool = False,
                 dtype: Optional[torch.dtype] = None, device: Optional[torch.device] = None):
        self.d = int(d)
        self.k = int(k)
        self.niter = int(niter)
        self.tol = float(tol)
        self.use_triton = bool(use_triton)
        self.seed = int(seed)
        self.chunk_size_data = int(chunk_size_data)
        self.chunk_size_centroids = int(chunk_size_centroids)
        self.chunk_size_data_cpu = int(chunk_size_data_cpu)
        self.verbose = bool(verbose)
        self.dtype = dtype
        self.device = device if device is not None else torch.device("cuda:0")
        self.centroids_b = None
        self.cluster_ids_b = None
        self._batch_size = None

    @staticmethod
    def _batched(data: torch.Tensor):
        if data.ndim == 2:
            return None, data.unsqueeze(0)
        if data.ndim == 3:
            return data.shape[0], data
        raise ValueError("data must be of shape (n_samples, n_features) or (batch_size, n_samples, n_features)")

    def train(self, data: torch.Tensor):
        B, x_b = self._batched(data)
        if data.device.type == "cpu" and x_b.shape[1] > self.chunk_size_data_cpu:
            raise RuntimeError("host-streamed k-means for N larger than GPU memory is not supported")
        x_b = x_b.to(device=self.device, dtype=self.dtype or x_b.dtype)
        gen = torch.Generator(device=x_b.device)
        gen.manual_seed(self.seed)
        from .kmeans_impl import random_init

        init = random_init(x_b, self.k, generator=gen)
        res = lloyd(x_b, self.k, self.niter, self.tol, init, x_sq_mode=X_SQ_BF16, verbose=self.verbose)
        self.centroids_b = res.centroids
        self.cluster_ids_b = res.labels
        self._batch_size = B
        return self

    def fit(self, data: torch.Tensor):
        self.train(data)
        return self

    def predict(self, data: torch.Tensor) -> torch.Tensor:
        if self.centroids_b is None:
            raise RuntimeError("Model not trained. Call train() or fit() first.")
        B, x_b = self._batched(data)
        if B != self._batch_size:
            raise ValueError(
                f"Model was trained with batch size B={self._batch_size}, "
                f"but predict received B={B}. Provide matching batch size."
            )
        x_b = x_b.to(device=self.device, dtype=self.dtype or x_b.dtype)
        labels = euclid_assign(x_b, self.centroids_b, None, x_sq_mode=X_SQ_BF16)
        return labels.squeeze(0) if B is None else labels

    def fit_predict(self, data: torch.Tensor) -> torch.Tensor:
        self.train(data)
        return self.cluster_ids_b.squeeze(0) if self._batch_size is None else self.cluster_ids_b
