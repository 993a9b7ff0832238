"""The bit-exact bookkeeping tests, run again on the GPU box.

The CPU suite checks the native partition bookkeeping (gr_build_subgraph,
gr_partition_boundaries, gr_csr_transpose, gr_spmm_plan, the partitioner and
the preprocessing pipeline of grinnder/data/partition.py:178-363) against the
oracle, the reference's compiled subgraph.cpp and hand-derived known
answers.  These twins run the same checks under the `gpu` marker, so the
library the GPU box loads, not only the one in the build container, is
attested bit-exact.
"""

import pytest

from tests import test_host_logic as host
from tests import test_oracle as orc

pytestmark = pytest.mark.gpu

test_box_library_exports_every_declared_symbol = host.test_library_exports_every_declared_symbol
test_box_build_subgraph_known_answers = host.test_build_subgraph_known_answers
test_box_build_subgraph_bit_exact = host.test_build_subgraph_bit_exact
test_box_partition_subgraph_and_pipeline_bit_exact = \
    host.test_partition_subgraph_and_pipeline_bit_exact
test_box_halo_order_known_answer = host.test_native_partition_subgraph_halo_order_known_answer
test_box_halo_layout_property = host.test_native_partition_subgraph_halo_layout_property
test_box_csr_transpose_is_stable_and_complete = host.test_csr_transpose_is_stable_and_complete
test_box_spmm_plan_covers_every_edge_once = host.test_spmm_plan_covers_every_edge_once
test_box_rmat_stream_independent_of_threads = host.test_rmat_stream_independent_of_threads
test_box_partitioner_is_a_balanced_permutation = host.test_partitioner_is_a_balanced_permutation
test_box_directed_rmat_pipeline_bit_exact = host.test_directed_rmat_pipeline_bit_exact
test_box_native_directed_pipeline_known_answer_and_brute_force = \
    host.test_native_directed_pipeline_known_answer_and_brute_force
test_box_whole_adjacency_orientation = \
    host.test_whole_adjacency_is_the_full_graph_in_partition_order
test_box_directed_pipeline_known_answer = orc.test_directed_pipeline_known_answer
test_box_gcn_norm_triangle_known_answer = orc.test_gcn_norm_triangle_known_answer
test_box_gcn_norm_matches_brute_force_degrees = orc.test_gcn_norm_matches_brute_force_degrees
test_box_csr_rows_and_permutation = orc.test_csr_rows_and_permutation
test_box_build_subgraph_matches_compiled_reference = \
    orc.test_build_subgraph_matches_compiled_reference


def test_box_compiled_reference_is_present():
    """oracle/_ref (the reference's subgraph.cpp, built in the build
    container) travels with the tree, so the comparisons above run here
    instead of skipping."""
    import oracle

    assert oracle.ref_build_subgraph() is not None
