"""Read-hint planning (the host policy of src/l2_prefetch_plan.rs, restated in gfr_moe) against the reference's own
unit-test vectors (l2_prefetch_plan.rs tests: retained_policy_is_bounded_and_skips_prefill,
aligned_read_hints_never_exceed_tensor_or_site, canonical_fp8_reads_scales_before_words,
routed_gate_up_heads_keep_shared_expert_outside_the_weight_extent), plus the C ABI's argument checks, which run on
the host before any device call (no GPU needed)."""
import ctypes

import pytest


@pytest.fixture(scope="module")
def g():
    import gfr_moe
    return gfr_moe


def test_policy_is_bounded_and_skips_prefill(g):
    assert g.pf_budget(24 << 20) == g.PF_BUDGET
    assert g.pf_budget(0) == g.PF_BUDGET
    assert g.pf_budget(8 << 20) == 4 << 20
    for rows in (1, 2, 8, 16, 64):
        assert g.pf_rows_enabled(rows)
    for rows in (0, 65, 512, 8192):
        assert not g.pf_rows_enabled(rows)
    assert g.pf_grid(g.PF_BUDGET, 48) == 2
    assert g.pf_grid(16, 48) == 1
    with pytest.raises(ValueError):
        g.pf_grid(g.PF_BUDGET + 1, 48)
    with pytest.raises(ValueError):
        g.pf_grid(16, 0)


def test_line_grid_covers_the_bytes(g):
    """This library's grid: one thread a PF_LINE_CHUNK of lines, 128 threads a workgroup, at most one a CU."""
    assert g.pf_grid(g.PF_BUDGET, 256, g.PF_LINE_CHUNK) == 32
    for n in (16, 2048, 2064, 262144, 262160, 1 << 20):
        grid = g.pf_grid(n, 1024, g.PF_LINE_CHUNK)
        assert grid * g.PF_THREADS * g.PF_LINE_CHUNK >= n
        assert (grid - 1) * g.PF_THREADS * g.PF_LINE_CHUNK < n
    assert g.pf_grid(g.PF_BUDGET, 4, g.PF_LINE_CHUNK) == 4


def test_aligned_read_hints_never_exceed_tensor_or_site(g):
    T = g.PfTensor
    out = g.pf_take([T(0x1003, 61), T(0x2000, 64)], 80)
    assert out == [g.PfSpan(0x1010, 48), g.PfSpan(0x2000, 32)]
    with pytest.raises(ValueError):
        g.pf_take([T(2 ** 64 - 32, 64)], 64)
    with pytest.raises(ValueError):
        g.pf_take([T(0, 64)], 64)
    assert g.pf_take([T(0x1000, 64, contiguous=False)], 64) == []
    with pytest.raises(ValueError):
        g.pf_take([T(0x1000, 64)], 0)


def test_scaled_weights_read_scales_before_words(g):
    T = g.PfTensor
    out = g.pf_take([(T(0x1000, 4096), T(0x10000, 16 << 20))], g.PF_BUDGET)
    assert out == [g.PfSpan(0x1000, 4096), g.PfSpan(0x10000, g.PF_BUDGET - 4096)]


def test_routed_gate_up_heads_stay_inside_the_weight_extent(g):
    T = g.PfTensor
    plan = g.pf_experts(T(0x10000, 288 * 131072), T(0x5000000, 288 * 131072), 288)
    assert plan == g.ExpertPlan((0x10000, 0x5000000), 131072, 65536, 288)
    assert g.pf_experts(T(0x10001, 288 * 131072), T(0x5000000, 288 * 131072), 288) is None
    assert g.pf_experts(T(0x10000, 32), T(0x5000000, 16), 1) is None
    assert g.pf_experts(T(0x10000, 32), T(0x5000000, 32), 1).bytes == 32
    assert g.pf_expert_grid(1, 288, 289, 48) == (9, 9)
    assert g.pf_expert_grid(4, 288, 289, 48) == (33, 33)
    assert g.pf_expert_grid(16, 288, 289, 48) == (129, 48)
    assert g.pf_expert_grid(64, 288, 289, 48) == (289, 48)
    with pytest.raises(ValueError):
        g.pf_expert_grid(4, 288, 9, 48)
    # every hinted byte lies inside its expert: bytes <= stride, and the last expert's range ends at the extent
    for count, per in ((288, 131072), (65, 3145728), (161, 16), (7, 48)):
        p = g.pf_experts(T(0x10000, count * per), T(0x5000000, count * per), count)
        assert p.bytes <= p.stride and p.bytes % 16 == 0 and p.bytes == min(65536, per)
        assert p.bases[0] + (count - 1) * p.stride + p.bytes <= 0x10000 + count * per


def test_abi_version(g):
    assert g.lib().gfr_prefetch_abi() == 1


@pytest.mark.parametrize("args", [
    # ids, count, maxu, bases, stride, bytes, experts, grid, stream
    (0, 16, 9, 16, 131072, 65536, 288, 9, 16),            # null ids
    (16, 0, 9, 16, 131072, 65536, 288, 9, 16),            # null count
    (16, 16, 9, 0, 131072, 65536, 288, 9, 16),            # null bases
    (16, 16, 0, 16, 131072, 65536, 288, 9, 16),           # maxu 0
    (16, 16, 9, 16, 131072, 65536, 0, 9, 16),             # no experts
    (16, 16, 9, 16, 131072, 65552, 288, 9, 16),           # above 64 KiB
    (16, 16, 9, 16, 32, 48, 288, 9, 16),                  # above the stride
    (16, 16, 9, 16, 131072, 65528, 288, 9, 16),           # bytes not a multiple of 16
    (16, 16, 9, 16, 131080, 65536, 288, 9, 16),           # stride not a multiple of 16
    (16, 16, 9, 16, 131072, 0, 288, 9, 16),               # empty
    (16, 16, 9, 16, 131072, 65536, 288, 0, 16),           # grid 0
    (16, 16, 9, 16, 131072, 65536, 288, 9, 0),            # null stream
])
def test_experts_entry_rejects(g, args):
    ids, count, maxu, bases, stride, nbytes, experts, grid, stream = args
    rc = g.lib().gfr_prefetch_experts(ids, count, maxu, bases, stride, nbytes, experts, grid, stream)
    assert rc == g.GFR_EINVAL and "prefetch experts" in g.lib().gfr_last_error().decode()


@pytest.mark.parametrize("args", [(0, 4, 2, 16), (16, 0, 2, 16), (16, 4, 0, 16), (16, 4, 2, 0)])
def test_segments_entry_rejects(g, args):
    rc = g.lib().gfr_prefetch_segments(*args)
    assert rc == g.GFR_EINVAL and "prefetch segments" in g.lib().gfr_last_error().decode()


def test_properties_and_capturing_reject_null_outputs(g):
    assert g.lib().gfr_prefetch_properties(None, None) == g.GFR_EINVAL
    assert g.lib().gfr_prefetch_capturing(None, ctypes.byref(ctypes.c_int())) == g.GFR_EINVAL
    assert g.lib().gfr_prefetch_capturing(16, None) == g.GFR_EINVAL
