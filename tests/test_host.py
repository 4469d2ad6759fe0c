"""Host-side logic of the Python drop-ins that needs no GPU: configuration checks
and the refusals of configurations that have no HIP path."""

import pytest


def test_output_role_repair_is_refused():
    """repair_features="output_role" (reference n8_v6.py:1246-1290) has no kernels in
    this build: the config is refused rather than silently running the output repair."""
    from sparsepr_amd.n8_v6 import N8V6Config

    N8V6Config(repair_features="output").validate()
    with pytest.raises(NotImplementedError, match="output_role"):
        N8V6Config(repair_features="output_role").validate()
    with pytest.raises(ValueError, match="repair_features must be"):
        N8V6Config(repair_features="bogus").validate()


def test_output_role_refused_by_repair_even_without_validation():
    from sparsepr_amd.n8_v6 import N8V6Config, N8V6Core

    core = N8V6Core(N8V6Config(repair_features="output_role"), validate=False)
    torch = pytest.importorskip("torch")
    x = torch.zeros((1, 1, 4, 64), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="output_role"):
        core.repair(x, x, x, x, route=None)
