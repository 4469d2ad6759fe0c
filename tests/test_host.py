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
