"""Batch administration (finalize, filter, extend, extract, merge) of the
shipped caches against the oracle's, on CPU (kernel wrappers replaced by
conftest.cpu_kernels; tests/test_gpu_batch_admin.py runs the same
scenarios on the HIP kernels).  The scenarios (tests/admin_scenarios.py)
compare whole buffers and counters bit-exactly after every step and check
that every sequence keeps its tokens through each step."""

import pytest

from admin_scenarios import BATCH_SCENARIOS, ROTATING_SCENARIOS, batch_scenario, rotating_scenario


@pytest.mark.parametrize("name", BATCH_SCENARIOS)
def test_batch_admin(cpu_kernels, name):
    batch_scenario(name, bits=4, gs=32, dtype="f16", seed=1)


@pytest.mark.parametrize("keep", [0, 2])
@pytest.mark.parametrize("name", ROTATING_SCENARIOS)
def test_rotating_batch_admin(cpu_kernels, name, keep):
    rotating_scenario(name, max_size=8, keep=keep, bits=8, gs=64, dtype="bf16", seed=2)
