"""Read hints on the GPU (csrc/prefetch.hip, gfr_moe.Prefetch; the reference's native/l2-prefetch and
l2_prefetch.rs Owner): the kernels read weight memory and write nothing, so a layer run behind them is byte-identical
to the same layer without them, eagerly and over replays of a captured graph; expert ids outside the plan's experts
and table entries that are not 16-byte aligned are skipped."""
import pytest
import torch

pytestmark = pytest.mark.gpu

E, D, N, BITS, TOPK = 64, 2048, 1536, 4, 4
SLOTS = TOPK + 1


def _setup(gfr, rows, seed):
    import synth
    w = synth.experts(E + 1, D, N, BITS, seed=seed)
    x = synth.activations(rows, D, seed + 1)
    lg = synth.logits(rows, E, seed + 2)
    picks, _ = gfr.route(lg, TOPK)
    torch.cuda.synchronize()
    return w, x, picks


def _expert_plan(gfr, w):
    """The routed experts' gate / up heads (the shared expert, id E, lies past the routed extent and is skipped)."""
    stride = w.gt[0].numel() * 4
    T = gfr.PfTensor
    return gfr.pf_experts(T(w.gt.data_ptr(), E * stride), T(w.ut.data_ptr(), E * stride), E)


def _spans(gfr, w):
    T = gfr.PfTensor
    items = [T(w.dt.data_ptr(), w.dt.numel() * 4), (T(w.svh_d.data_ptr(), w.svh_d.numel() * 2),
                                                    T(w.suh_d.data_ptr(), w.suh_d.numel() * 2))]
    return gfr.pf_take(items, gfr.PF_BUDGET)


@pytest.mark.parametrize("rows", [1, 4])
def test_hints_leave_every_bit(gfr, rows):
    w, x, picks = _setup(gfr, rows, 401 + rows)
    g = gfr.Grouping(E + 1, SLOTS, rows)
    ex = gfr.ExpertGpu(D, N, SLOTS, SLOTS, rows)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g.run(picks, rows, stream=s)
        ex.run_rows(w, x, picks, g.ids, g.count, g.members, rows, rows, stream=s)
    s.synchronize()
    plain = ex.y[:rows * SLOTS].clone()

    pf = gfr.Prefetch()
    plan = _expert_plan(gfr, w)
    assert plan.bytes == 65536 and plan.stride == D // 16 * N // 16 * 8 * BITS * 4
    pf.add_experts(0, plan)
    spans = _spans(gfr, w)
    assert spans and sum(sp.bytes for sp in spans) <= gfr.PF_BUDGET
    pf.add_segments("down", spans)
    ex.y.zero_()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.run(picks, rows, stream=s)
        pf.experts(s, 0, rows, g.ids, g.count)
        pf.mark(s, "down", rows)
        ex.run_rows(w, x, picks, g.ids, g.count, g.members, rows, rows, stream=s)
        pf.join(s)
    s.synchronize()
    assert pf.stats["launches"] == 1 and pf.stats["expert_launches"] == 1
    assert torch.equal(ex.y[:rows * SLOTS], plain)


def test_prefill_sized_windows_take_no_hint(gfr):
    """rows_enabled: windows above 64 rows launch nothing (the reference's decode-only policy)."""
    w, _, _ = _setup(gfr, 1, 409)
    pf = gfr.Prefetch()
    pf.add_experts(0, _expert_plan(gfr, w))
    ids = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
    count = torch.ones(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    pf.experts(s, 0, 65, ids, count)
    pf.mark(s, "none", 1)
    pf.join(s)
    assert pf.stats["expert_launches"] == 0 and pf.stats["launches"] == 0 and not pf.pending


def test_out_of_range_ids_and_unaligned_entries_are_skipped(gfr):
    """Only ids in [0, experts) are read, at most min(count, maxu) of them; table entries that are unaligned, empty or
    null are skipped. The buffers read stay inside the weight tensors, and the device ids / count are unchanged."""
    w, _, _ = _setup(gfr, 1, 411)
    plan = _expert_plan(gfr, w)
    ids = torch.tensor([-1, E, 3, 2 ** 31 - 1, E - 1, 0, -5], dtype=torch.int32, device="cuda")
    count = torch.tensor([100], dtype=torch.int32, device="cuda")
    bases = torch.tensor(list(plan.bases), dtype=torch.int64, device="cuda")
    base = w.dt.data_ptr()
    table = torch.tensor([[base + 4, 64], [base, 0], [0, 4096], [base, 40], [base + 16, 4096], [base, -16]],
                         dtype=torch.int64, device="cuda")
    ids0, table0 = ids.clone(), table.clone()
    s = torch.cuda.Stream()
    L = gfr.lib()
    gfr._check(L.gfr_prefetch_experts(ids.data_ptr(), count.data_ptr(), ids.numel(), bases.data_ptr(), plan.stride,
                                      plan.bytes, E, 3, s.cuda_stream))
    gfr._check(L.gfr_prefetch_segments(table.data_ptr(), table.shape[0], 2, s.cuda_stream))
    s.synchronize()
    assert torch.equal(ids, ids0) and torch.equal(table, table0) and int(count.item()) == 100


def test_hints_in_a_captured_graph(gfr):
    """Fork, hints, layer and join captured once; every replay (with eager work and synchronisations between them)
    gives the eager bytes."""
    rows = 2
    w, x, picks = _setup(gfr, rows, 421)
    g = gfr.Grouping(E + 1, SLOTS, rows)
    ex = gfr.ExpertGpu(D, N, SLOTS, SLOTS, rows)
    pf = gfr.Prefetch()
    pf.add_experts(0, _expert_plan(gfr, w))
    pf.add_segments("down", _spans(gfr, w))
    s = torch.cuda.Stream()

    def step():
        g.run(picks, rows, stream=s)
        pf.experts(s, 0, rows, g.ids, g.count)
        pf.mark(s, "down", rows)
        ex.run_rows(w, x, picks, g.ids, g.count, g.members, rows, rows, stream=s)
        pf.join(s)

    with torch.cuda.stream(s):
        step()
    s.synchronize()
    eager = ex.y[:rows * SLOTS].clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()
    assert not pf.pending
    for _ in range(3):
        ex.y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ex.y[:rows * SLOTS], eager)
    cus, l2 = gfr.prefetch_properties()
    assert cus > 0 and l2 > 0
    assert not gfr.prefetch_capturing(s)


def _bytesum(t):
    return t.contiguous().view(torch.uint8).sum(dtype=torch.int64).item()


def test_many_segments_write_nothing(gfr):
    """A table of many short ranges (the reference plans up to 130 heads of 8,176 bytes for one matrix,
    l2_prefetch_plan.rs tests) over the down trellis, then the scales with what is left of a 1 MiB budget: launches
    at several grid sizes leave the weights unchanged."""
    w, _, _ = _setup(gfr, 1, 431)
    T = gfr.PfTensor
    base = w.dt.data_ptr()
    heads = [T(base + k * 65536, 8176) for k in range(128)]
    spans = gfr.pf_take(heads + [(T(w.svh_d.data_ptr(), w.svh_d.numel() * 2), T(w.suh_d.data_ptr(), w.suh_d.numel() * 2))],
                        1 << 20)
    assert len(spans) == 129 and spans[-1] == gfr.PfSpan(w.svh_d.data_ptr(), (1 << 20) - 128 * 8176)
    before = [_bytesum(t) for t in (w.dt, w.svh_d, w.suh_d)]
    pf = gfr.Prefetch()
    pf.add_segments("heads", spans)
    s = torch.cuda.Stream()
    table, n, _ = pf.tables["heads"]
    for grid in (1, 7, 256):
        gfr._check(gfr.lib().gfr_prefetch_segments(table.data_ptr(), n, grid, s.cuda_stream))
    pf.mark(s, "heads", 1)
    pf.join(s)
    s.synchronize()
    assert [_bytesum(t) for t in (w.dt, w.svh_d, w.suh_d)] == before
