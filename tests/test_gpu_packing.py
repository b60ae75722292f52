"""The row packing policy's library-vs-oracle tests, collected again under the `gpu` marker so that
the GPU-box run (which runs `-m gpu` only) also covers the native packing code in
libaspec_amd.so. The policy itself is host code: nothing here launches a kernel."""

import pytest

from tests import test_packing as T

pytestmark = pytest.mark.gpu


def test_reference_cases_through_the_library_gpu_box(gpu):
    T.test_reference_cases_through_the_library()


def test_library_errors_match_the_reference_gpu_box(gpu):
    T.test_library_errors_match_the_reference()


def test_library_eligible_starts_match_oracle_batched_gpu_box(gpu):
    T.test_library_eligible_starts_match_oracle_batched()


@pytest.mark.parametrize("seed", range(4))
def test_library_matches_oracle_on_random_pools_gpu_box(gpu, seed):
    T.test_library_matches_oracle_on_random_pools(seed)


def test_library_density_ties_are_exact_double_quotients_gpu_box(gpu):
    T.test_library_density_ties_are_exact_double_quotients()


def test_library_large_pool_invariants_and_speed_gpu_box(gpu):
    T.test_library_large_pool_invariants_and_speed()
