"""The reference's own probe geometry: hidden 4096, intermediate 512, 288 EXL3 routed experts plus a shared expert
(id 288) that is not EXL3, 9 slots of which 8 are EXL3 (the reference runs its FP8 shared expert elsewhere).
  * experts::probe (experts.rs:146-173, 304-308): ExpertGpu on picks [0..7, 288] with the input
    bf((i * 73 % 997 - 498) / 512), every EXL3 slot against the oracle, graph replays byte-equal;
  * fast_experts::probe (fast_experts.rs:230-286): FastExperts with picks (r * 7 + slot) % 16 and the shared id last,
    input bf(((i * 73 + 23) % 257) / 128 - 1), including the 4097-row window with member stride 4097.
Weights are seeded synthetic tensors of the reference's shapes (its checkpoint is not available here)."""
import numpy as np
import pytest
import torch

from refs import DecodedExperts, assert_close, assert_decode_close, assert_rows_close, np_u16, window_reference

pytestmark = pytest.mark.gpu

D, N, E, SLOTS, EXL3_SLOTS, BITS, SHARED = 4096, 512, 288, 9, 8, 4, 288


@pytest.fixture(scope="module")
def weights():
    import synth
    return synth.experts(E, D, N, BITS, seed=288)


def _bf16_of(vals):
    return torch.tensor(vals, dtype=torch.float32).to(torch.bfloat16)


def test_experts_probe_reference_geometry(gfr, oracle, weights):
    x = _bf16_of([((i * 73 % 997) - 498) / 512 for i in range(D)]).reshape(1, D).cuda()
    picked = np.array([[0, 1, 2, 3, 4, 5, 6, 7, SHARED]], np.int32)
    picks = torch.from_numpy(picked).cuda()
    g = gfr.Grouping(E + 1, SLOTS, 1)
    ex = gfr.ExpertGpu(D, N, SLOTS, EXL3_SLOTS, 1)
    ex.y.fill_(7.0)
    g.run(picks, 1)
    ex.run_rows(weights, x, picks, g.ids, g.count, g.members, 1, 1)
    torch.cuda.synchronize()
    y = ex.y[:SLOTS].cpu().numpy()
    dec, ref = DecodedExperts(oracle, weights, rounded=False), DecodedExperts(oracle, weights)
    xb = np_u16(x)[0]
    for s in range(EXL3_SLOTS):
        assert_decode_close(y[s], dec.row(xb, s)[0], ref.row(xb, s)[0], what=f"slot {s}")
    assert np.all(y[EXL3_SLOTS] == 7.0), "the non-EXL3 slot's output must stay untouched"
    # experts.rs:309-316: the captured sequence replays to the eager bytes
    eager = ex.y.clone()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            g.run(picks, 1, stream=s)
            ex.run_rows(weights, x, picks, g.ids, g.count, g.members, 1, 1, stream=s)
    for _ in range(5):
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ex.y, eager)


@pytest.mark.parametrize("rows,maxm", [(65, 129), (4097, 4097)])
def test_fast_experts_probe_reference_geometry(gfr, oracle, weights, rows, maxm):
    picked = np.array([[(SHARED if s == SLOTS - 1 else (r * 7 + s) % 16) for s in range(SLOTS)] for r in range(rows)],
                      np.int32)
    picks = torch.from_numpy(picked).cuda()
    x = _bf16_of([((i * 73 + 23) % 257) / 128 - 1 for i in range(rows * D)]).reshape(rows, D).cuda()
    g = gfr.Grouping(E + 1, SLOTS, maxm)
    g.run(picks, rows)
    fx = gfr.FastExperts(D, N, SLOTS, EXL3_SLOTS, E, maxm)
    fx.output.fill_(7.0)
    fx.run(weights, x, picks, g.ids, g.count, g.members, rows, maxm, shared_x=False)
    torch.cuda.synchronize()
    out = fx.output[:rows * SLOTS].cpu().numpy()
    dec = DecodedExperts(oracle, weights)
    xb = np_u16(x)
    for r, s in [(0, 0), (rows - 1, EXL3_SLOTS - 1)]:
        want, _ = dec.row(xb[r], int(picked[r, s]), sk_gu=1, sk_d=1, warps=1)
        assert_close(out[r * SLOTS + s], want, what=f"rows {rows} row {r} slot {s}")
    shared_rows = out.reshape(rows, SLOTS, D)[:, SLOTS - 1]
    assert np.all(shared_rows == 7.0), "the non-EXL3 slot's output must stay untouched"
    # every EXL3 (row, slot) output of the window, as fast_experts.rs:353-361 checks every byte of its windows
    want = window_reference(oracle, weights, x, picked, exl3_slots=EXL3_SLOTS, workers=16)
    assert_rows_close(out.reshape(rows, SLOTS, D)[:, :EXL3_SLOTS], want[:, :EXL3_SLOTS],
                      what=f"rows {rows}, every EXL3 (row, slot)")


@pytest.mark.parametrize("rows,routed,hidden", [(1, 64, 2048), (3, 288, 4096), (70, 64, 2048), (5, 160, 5120)])
def test_router_logits_vs_float64(gfr, rows, routed, hidden):
    """gfr_router_logits (the reference's router_part + router_sum, moe.rs:77-87) against the float64 product of the
    same bf16 inputs; the fp32 sums agree to accumulation error. 70 rows take the 8-row programs, hidden 5120 two
    passes over the hidden size."""
    g = torch.Generator(device="cuda").manual_seed(rows + routed)
    x = torch.randn((rows, hidden), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((routed, hidden), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    got = gfr.router_logits(x, w)
    torch.cuda.synchronize()
    want = x.double().cpu().numpy() @ w.double().cpu().numpy().T
    scale = np.abs(x.double().cpu().numpy()) @ np.abs(w.double().cpu().numpy()).T
    err = np.abs(got.cpu().numpy() - want)
    assert np.all(err <= 1e-6 * scale + 1e-7), float((err / (scale + 1e-30)).max())


@pytest.mark.parametrize("rows", [1, 3, 40, 300])
def test_moe_reference_layout_shared_output(gfr, oracle, weights, rows):
    """Moe::run_prefetched at the reference's layout (moe.rs:77-181): router logits from the hidden rows, GLM's gate
    over 288 routed experts (top-8, bias, scale 2.5), the shared expert (id 288) not EXL3 and its output the caller's,
    added by the combine as the last slot. Every engine path: the bs = 1 launches (router fused into gate/up), a
    decode window, a split-K prefill window and full-K prefill items."""
    topk = 8
    g = torch.Generator(device="cuda").manual_seed(100 + rows)
    x = torch.randn((rows, D), generator=g, device="cuda").to(torch.bfloat16)
    router_w = (torch.randn((E, D), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    bias = torch.randn(E, generator=g, device="cuda") * 0.05
    shared = torch.randn((rows, D + 16), generator=g, device="cuda")    # a strided caller buffer
    m = gfr.Moe(D, N, E, topk, max(rows, 4), shared_exl3=False)
    m.set_router(bias, 2.5)
    # the combine reads the shared rows 16 bytes at a time: a view one float in (4-byte aligned) is refused
    with pytest.raises(gfr.GfrError, match="16-byte aligned"):
        m.run_router(weights, x, router_w, rows, shared=shared[:, 1:])
    m.run_router(weights, x, router_w, rows, shared=shared)
    torch.cuda.synchronize()
    out = m.output[:rows].cpu().numpy()
    assert np.all(np.isfinite(out))
    logits = gfr.router_logits(x, router_w).cpu().numpy()
    p, wt = oracle.route_biased(logits, bias.cpu().numpy(), 2.5, topk, E)
    gp, gw = m.picks[:rows].cpu().numpy(), m.weights[:rows].cpu().numpy()
    assert np.array_equal(gp[:, topk], np.full(rows, SHARED))
    dec = DecodedExperts(oracle, weights, rounded=rows > 4)
    xb = np_u16(x)
    sh = shared.cpu().numpy()
    for r in sorted({0, rows - 1, rows // 2}):
        ys = [dec.row(xb[r], int(e))[0] if rows <= 4 else dec.row(xb[r], int(e), sk_gu=1, sk_d=1, warps=1)[0]
              for e in gp[r, :topk]]
        want = oracle.combine(np.stack(ys + [sh[r, :D]]), gw[r:r + 1], 1, topk + 1)[0]
        assert_close(out[r], want, what=f"rows {rows} token {r}")
        choice = np.sort(1.0 / (1.0 + np.exp(-logits[r].astype(np.float64))) + bias.cpu().numpy())[::-1]
        if choice[topk - 1] - choice[topk] > 1e-5:      # no near-tie at the k-th place: the picks are the oracle's
            assert list(gp[r]) == list(p[r]), r
            np.testing.assert_allclose(gw[r], wt[r], rtol=2e-6)


@pytest.mark.parametrize("rows", [1, 3, 40, 300])
def test_shared_branch_overlap(gfr, weights, rows):
    """shared_expert.rs Branch::run (:60-78) through SharedBranch and gfr_moe_run_shared_branch: the shared expert's
    output is produced on the branch stream behind a long matmul (the buffer holds NaN until then), the routed layer
    runs on the main stream and only its combine waits for the branch. The output is byte-equal to the serial
    gfr_moe_run_shared, eagerly and in every replay of a captured graph (fork and join inside the capture)."""
    topk = 8
    g = torch.Generator(device="cuda").manual_seed(7 + rows)
    x = torch.randn((rows, D), generator=g, device="cuda").to(torch.bfloat16)
    logits = torch.randn((rows, E), generator=g, device="cuda")
    src = torch.randn((rows, D), generator=g, device="cuda")
    a = torch.randn((2048, 2048), generator=g, device="cuda")
    shared = torch.empty((rows, D), device="cuda")
    m = gfr.Moe(D, N, E, topk, max(rows, 4), shared_exl3=False)
    m.run(weights, x, logits, rows, shared=src)
    torch.cuda.synchronize()
    want = m.output[:rows].clone()
    branch = gfr.SharedBranch()
    main = torch.cuda.Stream()

    def layer():
        shared.fill_(float("nan"))

        def shared_fn(side):
            t = a
            for _ in range(4):
                t = t @ a * (1.0 / 64.0)
            shared.copy_(src + 0.0 * t[0, 0])

        branch.run(main, shared_fn, lambda ready: m.run(weights, x, logits, rows, stream=main, shared=shared,
                                                         shared_ready=ready))

    with torch.cuda.stream(main):
        m.output.zero_()
        layer()
    torch.cuda.synchronize()
    assert torch.equal(m.output[:rows], want)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(main):
        with torch.cuda.graph(graph, stream=main):
            layer()
    for _ in range(3):
        m.output.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(main):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.output[:rows], want)


def test_shared_branch_rejects_event_without_output(gfr, weights):
    m = gfr.Moe(D, N, E, 8, 4, shared_exl3=False)
    with pytest.raises(ValueError):
        m.run(weights, torch.zeros((1, D), dtype=torch.bfloat16, device="cuda"), torch.zeros((1, E), device="cuda"),
              1, shared_ready=torch.cuda.Event())
