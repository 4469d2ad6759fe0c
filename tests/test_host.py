"""Host-side logic of the Python drop-ins that needs no GPU: configuration checks
and the refusals of configurations that have no HIP path."""

import pytest


def test_output_role_repair_config():
    """repair_features="output_role" (reference n8_v6.py:1246-1290) is accepted with the Q role
    ranks the role-feature apply kernel takes (16, 32, 48, 64) and refused with others."""
    from sparsepr_amd.n8_v6 import N8V6Config

    N8V6Config(repair_features="output").validate()
    N8V6Config(repair_features="output_role").validate()
    N8V6Config(repair_features="output_role", role_q_rank=32).validate()
    with pytest.raises(NotImplementedError, match="role_q_rank"):
        N8V6Config(repair_features="output_role", role_q_rank=40).validate()
    with pytest.raises(ValueError, match="repair_features must be"):
        N8V6Config(repair_features="bogus").validate()


def test_route_feature_dims_the_kernels_take():
    """The role-space k-means runs on feature dims that are multiples of 16 up to 128: other
    Q role ranks or K (+ V) feature counts are refused before any launch, naming the limit."""
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    N8V6Core(N8V6Config())._check_route_config(128)
    N8V6Core(N8V6Config(role_k_rank=32, role_v_rank=16, role_v_weight=0.5))._check_route_config(64)
    for cfg, dim in ((N8V6Config(role_q_rank=40), 128), (N8V6Config(role_k_rank=24), 128),
                     (N8V6Config(role_k_rank=64, role_v_rank=72, role_v_weight=0.5), 128),
                     (N8V6Config(), 96)):
        with pytest.raises(NotImplementedError, match="multiple of 16"):
            N8V6Core(cfg, validate=False)._check_route_config(dim)
