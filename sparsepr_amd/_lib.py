"""ctypes binding of libsparsepr_hip.so (the C ABI declared in include/sparsepr_hip.h).

Every entry point takes raw device pointers, sizes and a hipStream_t, and
returns an int status; a nonzero status is raised here as RuntimeError with the
library's last error text (the reference raises RuntimeError through
TORCH_CHECK, n8_ops.cu:505-514).  Launches go on torch's current stream.
There is no CPU path: a missing library or a non-GPU tensor raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsparsepr_hip.so"

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "spr_last_error": (ctypes.c_char_p, []),
    "spr_abi_version": (ctypes.c_int, []),
    # permute.hip
    "spr_permute_rows": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "spr_inverse_permute_rows": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "spr_inverse_permute_rows_strided": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
    "spr_permute_concat_rows": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "spr_gather_rows": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
    "spr_scatter_rows": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
    # sort.hip
    "spr_argsort_labels_workspace": (_sz, [_i64, _i64, _i32]),
    "spr_argsort_labels": (ctypes.c_int, [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _sz, _vp]),
    # kmeans.hip
    "spr_centroid_sq": (ctypes.c_int, [_vp, _i32, _i64, _i32, _vp, _vp]),
    "spr_kmeans_assign_bf16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i32, _i32, _vp, _vp]),
    "spr_centroid_mean_workspace": (_sz, [_i64, _i64, _i32, _i32]),
    "spr_centroid_mean": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _sz, _vp]),
    "spr_original_centroids_workspace": (_sz, [_i64, _i64, _i32, _i32]),
    "spr_original_centroids": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp,
                                              _vp, _sz, _vp]),
    "spr_role_assign_fp32": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp]),
    "spr_kmeans_assign_tf32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp]),
    # select.hip
    "spr_topp_map": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _f32, _f32, _i32, _i32, _vp, _vp, _vp]),
    "spr_select_budget": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "spr_compact_selected": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, _vp]),
    "spr_density": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp]),
    # attention.hip
    "spr_block_sparse_attention_workspace": (_sz, [_i64, _i32, _i32]),
    "spr_block_sparse_attention_plan": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _sz, _vp]),
    "spr_block_sparse_attention_plan_schedule": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _sz,
                                                                _vp]),
    "spr_block_sparse_attention_run": (ctypes.c_int, [_vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i32, _i32, _i32,
                                                      _f32, _vp, _vp, _vp, _vp, _vp]),
    "spr_block_sparse_attention": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32,
                                                  _f32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "spr_block_sparse_attention_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32,
                                                          _i32, _f32, _vp, _vp, _vp, _vp, _vp]),
    "spr_dense_attention_workspace": (_sz, [_i64, _i64, _i32, _i32]),
    "spr_dense_attention": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _f32, _i32, _vp, _i32, _vp,
                                           _vp, _sz, _vp]),
    "spr_dense_attention_strided": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _f32, _i32, _vp,
                                                   _i32, _vp, _vp, _sz, _vp]),
    "spr_block_sparse_attention_run_ex": (ctypes.c_int, [_vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i32, _i32, _i32,
                                                         _f32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "spr_block_sparse_attention_ex": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32,
                                                     _f32, _i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "spr_dense_attention_strided_ex": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _f32, _i32,
                                                      _i32, _vp, _i32, _vp, _vp, _sz, _vp]),
    # repair.hip
    "spr_probe_distances": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp]),
    "spr_probe_select_workspace": (_sz, [_i64, _i32]),
    "spr_probe_select": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _sz,
                                        _vp]),
    "spr_repair_fit_prep": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "spr_repair_apply": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _f32, _f32, _vp, _vp]),
    "spr_repair_fit_prep_role": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _i32, _vp, _i64, _i64, _i32, _i32, _vp,
                                                _vp, _vp, _vp]),
    "spr_repair_apply_role": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _f32,
                                             _f32, _vp, _vp]),
    "spr_probe_scatter": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i64, _i32, _i32, _vp, _vp]),
    # qkv.hip
    "spr_wan_qkv_norm_rope_layout": (ctypes.c_int, [_vp] * 7 + [_i32, _i64, _i64, _i32, _i32, _f32] + [_vp] * 4),
    "spr_cosmos25_qkv_norm_rope_bshd": (ctypes.c_int, [_vp] * 6 + [_i32, _i64, _i64, _i32, _i32, _f32] + [_vp] * 4),
    # rrr.hip
    "spr_rrr_fit_workspace": (_sz, [_i64]),
    "spr_rrr_fit": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _f32, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _sz, _vp]),
    "spr_rrr_fit_ex": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _sz, _vp]),
    "spr_rrr_fit_top16": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp,
                                         _vp, _vp, _vp, _sz, _vp]),
    "spr_rrr_top16_basis": (ctypes.c_int, [_vp, _i64, _i32, _i32, _vp, _vp]),
    "spr_rrr_output_basis": (ctypes.c_int, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _sz, _vp]),
    "spr_rrr_recover": (ctypes.c_int, [_vp] * 10 + [_i64, _i32, _i32, _i32] + [_vp] * 7),
    "spr_sym_top_eig": (ctypes.c_int, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp]),
    # metric.hip
    "spr_role_metric": (ctypes.c_int, [_vp, _i32, _i64, _i64, _i32, _vp, _i32, _vp, _i32, _f32, _vp, _vp]),
    "spr_metric_factor_workspace": (_sz, [_i64, _i32]),
    "spr_metric_factor": (ctypes.c_int, [_vp, _i64, _i32, _i32, _vp, _vp, _sz, _vp]),
    "spr_warm_metric_factor": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _vp,
                                              _vp, _vp, _vp]),
    "spr_warm_metric_factor_workspace": (_sz, [_i64, _i32, _i32, _i32]),
    "spr_warm_metric_factor_ex": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _vp,
                                                 _vp, _vp, _vp, _sz, _vp]),
    "spr_project_rows": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _vp, _vp]),
    "spr_project_rows_ex": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _f32, _vp, _i32,
                                           _i32, _vp]),
    # role_proj.hip
    "spr_role_projection_rms": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp]),
    "spr_role_k_projection_workspace": (_sz, [_i64, _i64]),
    "spr_role_k_projection": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "spr_role_k_projection_ex": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _i32, _i32, _f32, _vp, _i32, _i32, _vp,
                                                _vp, _sz, _vp]),
    # svg_ear.hip
    "spr_svg_ear_scores_flops": (_sz, [_i64, _i32, _i64]),
    "spr_svg_ear_compensation": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64,
                                                _i32, _i32, _i32, _i32, _vp, _vp]),
    "spr_svg_ear_scores": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _i32, _i32, _i64, _i64,
                                          _i32, _i32, _i32, _vp, _vp]),
}

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"Could not load {LIB_PATH.name}: not built (run `python -m sparsepr_amd.build_hip` "
                "or __graft_entry__.build())."
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise RuntimeError(f"{LIB_PATH.name} does not export {name}; rebuild it")
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = lib
    return _LIB


def available() -> bool:
    try:
        load()
    except Exception:
        return False
    return torch.cuda.is_available()


def call(name: str, *args) -> int:
    """Call an entry point; raise RuntimeError on a nonzero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.spr_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {status}): {msg}")
    return status


def query(name: str, *args):
    return getattr(load(), name)(*args)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor | None, what: str = "tensor") -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{what}: SparsePR HIP kernels require GPU tensors (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors are on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError(f"{what}: no tensor given")
    return dev


DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch memory from torch's caching allocator (never a raw hipMalloc)."""
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)
