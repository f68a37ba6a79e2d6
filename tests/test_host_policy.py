"""Host-side choice of the plain forward's segment length (pure Python, no device)."""
from pragnosia_amd.ops import COMPUTE_UNITS, seg_chunks


def test_full_machine_keeps_one_workgroup_per_head():
    # 192 heads of 8 chunks already cover most compute units; so do 256 or more heads at any length
    assert seg_chunks(192, 8, range(1, 9)) == 8
    for heads in (256, 512, 4096):
        for NC in (1, 8, 64):
            assert seg_chunks(heads, NC, range(1, NC + 1)) == NC


def test_few_heads_over_many_chunks_split():
    # 24 heads of 128 chunks; one round of segments over the compute units, each walking 13 chunks
    P = seg_chunks(24, 128, range(1, 129))
    nseg = -(-128 // P)
    assert P == 13 and 24 * nseg <= COMPUTE_UNITS < 24 * (nseg + 1)
    # windowed carrying: only divisors of the window's chunk count are offered; the largest that fits is taken
    assert seg_chunks(24, 128, [1, 2, 4, 8]) == 8
    # never below two chunks, never when the walk saved is smaller than the sums' overhead
    assert seg_chunks(2, 64, range(1, 65)) == 2
    assert seg_chunks(96, 16, range(1, 17)) == 16


def test_single_chunk_and_single_candidate():
    assert seg_chunks(1, 1, [1]) == 1
    assert seg_chunks(4, 3, []) == 3


def test_backward_splits_sooner():
    # the backward's chunk step is heavier, so 96 heads of 16 chunks split for it (measured 41.8 -> 36.8 us) but
    # not for the forward (22.6 us sequential vs 26 segmented); 128 heads of 8 chunks split for neither
    assert seg_chunks(96, 16, range(1, 17), "bwd") == 8
    assert seg_chunks(96, 16, range(1, 17), "fwd") == 16
    assert seg_chunks(128, 8, range(1, 9), "bwd") == 8
    assert seg_chunks(192, 8, range(1, 9), "bwd") == 8
