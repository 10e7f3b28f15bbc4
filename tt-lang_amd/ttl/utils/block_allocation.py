"""`ttl.utils.block_allocation`: the same module as `utils.block_allocation`."""

from utils.block_allocation import *  # noqa: F401,F403
from utils.block_allocation import (  # noqa: F401
    SUBBLOCK_HW_CHOICES,
    MatmulParams,
    filter_factor_pairs_by_2d_grid,
    get_large_matmul_params,
    get_maximum_block_dim,
    get_number_of_cores,
    get_possible_products,
    get_prime_factors_with_multiplicity,
    num_cores_to_grid_ranges,
    remove_leading_ones,
    split_work_to_cores,
)
