"""Prefill path (FastExperts) on the GPU: MFMA grouped GEMMs against the CPU oracle (one full-K chain a row,
exl3_prefill.cu:14-23), the reference probe's row cases (fast_experts.rs:247-286), shared-X == separate-X,
graph replays byte-identical, and the MoE layer at the 8K-token prefill shape."""
import numpy as np
import pytest
import torch

from refs import DecodedExperts, assert_close, assert_rows_close, np_u16, window_reference

pytestmark = pytest.mark.gpu

D, N, BITS = 2048, 1536, 4


def _probe_picks(rows, E, slots):
    # fast_experts.rs:247-286: (r * 7 + slot) % 16 for the routed slots, the shared expert last
    return np.array([[(E if s == slots - 1 else (r * 7 + s) % 16) for s in range(slots)] for r in range(rows)],
                    np.int32)


@pytest.fixture(scope="module")
def weights():
    import synth
    return synth.experts(17, D, N, BITS, seed=77)


@pytest.mark.parametrize("rows,maxm", [(1, 129), (63, 129), (64, 129), (65, 129), (129, 129)])
def test_fast_experts_reference_cases(gfr, oracle, weights, rows, maxm):
    import synth
    slots = 5
    w = weights
    picks_np = _probe_picks(rows, 16, slots)
    picks = torch.from_numpy(picks_np).cuda()
    x = synth.activations(rows, D, 3 + rows)
    g = gfr.Grouping(17, slots, maxm)
    g.run(picks, rows)
    fx = gfr.FastExperts(D, N, slots, slots, 17, maxm)
    fx.run(w, x, picks, g.ids, g.count, g.members, rows, maxm, shared_x=False)
    torch.cuda.synchronize()
    y = fx.output[:rows * slots].cpu().numpy()
    assert np.all(np.isfinite(y))
    dec = DecodedExperts(oracle, w)
    xb = np_u16(x)
    for r, s in [(0, 0), (rows - 1, slots - 1)]:
        want, _ = dec.row(xb[r], int(picks_np[r, s]), sk_gu=1, sk_d=1, warps=1)
        assert_close(y[r * slots + s], want, what=f"rows {rows} row {r} slot {s}")
    # every (row, slot) output (fast_experts.rs:353-361 compares every output of the window)
    assert_rows_close(y, window_reference(oracle, w, x, picks_np).reshape(rows * slots, D), what=f"rows {rows}")


def test_shared_x_equals_separate_x(gfr, weights):
    """With suh_g == suh_u, the shared-rotation launch is byte-identical to the separate one (fast_experts.rs:369-381)."""
    import synth
    import dataclasses
    w = dataclasses.replace(weights, suh_u=weights.suh_g)
    rows, slots, maxm = 70, 5, 70
    picks = torch.from_numpy(_probe_picks(rows, 16, slots)).cuda()
    x = synth.activations(rows, D, 9)
    g = gfr.Grouping(17, slots, maxm)
    g.run(picks, rows)
    fx = gfr.FastExperts(D, N, slots, slots, 17, maxm)
    fx.run(w, x, picks, g.ids, g.count, g.members, rows, maxm, shared_x=True)
    a = fx.output[:rows * slots].clone()
    fx.run(w, x, picks, g.ids, g.count, g.members, rows, maxm, shared_x=False)
    assert torch.equal(a, fx.output[:rows * slots])


def test_prefill_graph_replays(gfr, weights):
    import synth
    rows, slots, maxm = 200, 5, 256
    picks = torch.from_numpy(_probe_picks(rows, 16, slots)).cuda()
    x = synth.activations(rows, D, 10)
    g = gfr.Grouping(17, slots, maxm)
    fx = gfr.FastExperts(D, N, slots, slots, 17, maxm)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g.run(picks, rows, stream=s)
        fx.run(weights, x, picks, g.ids, g.count, g.members, rows, maxm, False, stream=s)
        s.synchronize()
        eager = fx.output[:rows * slots].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            g.run(picks, rows, stream=s)
            fx.run(weights, x, picks, g.ids, g.count, g.members, rows, maxm, False, stream=s)
    for _ in range(3):
        fx.output.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(fx.output[:rows * slots], eager)


def test_moe_prefill_config4_tokens(gfr, oracle):
    """Config 4 shape: 8192 tokens, 64 routed + 1 shared, top-4, uniform routing: routing exact; three tokens against
    the oracle's own row order, and every token's output against the whole-window reference."""
    import synth
    E, topk, rows = 64, 4, 8192
    w = synth.experts(E + 1, D, N, BITS, seed=5)
    x = synth.activations(rows, D, 6)
    lg = synth.logits(rows, E, 7)
    m = gfr.Moe(D, N, E, topk, rows)
    m.run(w, x, lg, rows)
    torch.cuda.synchronize()
    out = m.output[:rows].cpu().numpy()
    assert np.all(np.isfinite(out))
    p, wt = oracle.route(lg.cpu().numpy(), topk, E)
    assert np.array_equal(m.picks[:rows].cpu().numpy(), p)
    dec = DecodedExperts(oracle, w)
    xb = np_u16(x)
    for r in (0, 4097, rows - 1):
        ys = np.stack([dec.row(xb[r], int(e), sk_gu=1, sk_d=1, warps=1)[0] for e in p[r]])
        want = oracle.combine(ys, wt[r:r + 1], 1, topk + 1)
        assert_close(out[r], want[0], what=f"token {r}")
    y = window_reference(oracle, w, x, p, workers=16)
    assert_rows_close(out, oracle.combine(y, wt, rows, topk + 1), what="config 4, every token")


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("rows", [40, 320])
def test_fast_experts_bit_widths(gfr, oracle, bits, rows):
    """K = 2, 3, 4, 5 (config 5's mixed bit rates) at C5's hidden size against the oracle: every width decodes its
    trellis straight into MFMA A fragments (K = 4 from word pairs, the others through one funnel shift a group of four
    values). 40 rows (360 pairs) run the split-K programs, 320 rows (2880 pairs) the full-K items with the fused
    epilogues."""
    import synth
    Dk, Nk, E, slots, maxm = 5120, 1536, 9, 9, rows
    w = synth.experts(E, Dk, Nk, bits, seed=90 + bits)
    picks_np = np.array([[(r * 3 + s) % (E - 1) if s < slots - 1 else E - 1 for s in range(slots)]
                         for r in range(rows)], np.int32)
    picks_np[:, :slots - 1] = np.sort(picks_np[:, :slots - 1], axis=1)
    picks = torch.from_numpy(picks_np).cuda()
    x = synth.activations(rows, Dk, 5 + bits)
    g = gfr.Grouping(E, slots, maxm)
    g.run(picks, rows)
    fx = gfr.FastExperts(Dk, Nk, slots, slots, E, maxm)
    fx.run(w, x, picks, g.ids, g.count, g.members, rows, maxm, shared_x=False)
    torch.cuda.synchronize()
    y = fx.output[:rows * slots].cpu().numpy()
    assert np.all(np.isfinite(y))
    dec = DecodedExperts(oracle, w)
    xb = np_u16(x)
    for r, s in [(0, 0), (rows - 1, 5)]:
        want, _ = dec.row(xb[r], int(picks_np[r, s]), sk_gu=1, sk_d=1, warps=1)
        assert_close(y[r * slots + s], want, what=f"K={bits} row {r} slot {s}")
    assert_rows_close(y, window_reference(oracle, w, x, picks_np).reshape(rows * slots, Dk),
                      what=f"K={bits} rows {rows}, every (row, slot)")


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_moe_prefill_config5_chunk(gfr, oracle, bits):
    """Config 5's prefill chunk at each of the stack's bit widths: 16384 tokens, hidden 5120, 160 routed + 1 shared,
    top-8, Zipf(1.1) routing; routing exact, the first, a middle and the last token against the oracle, and 64 spread
    tokens against the whole-window reference."""
    import synth
    E, Dk, Nk, topk, rows = 160, 5120, 1536, 8, 16384
    w = synth.experts(E + 1, Dk, Nk, bits, seed=71 if bits == 3 else 71 + 10 * bits)
    x = synth.activations(rows, Dk, 72)
    lg = synth.zipf_logits(rows, E, topk, 1.1, 73)
    m = gfr.Moe(Dk, Nk, E, topk, rows)
    m.run(w, x, lg, rows)
    torch.cuda.synchronize()
    out = m.output[:rows].cpu().numpy()
    assert np.all(np.isfinite(out))
    p, wt = oracle.route(lg.cpu().numpy(), topk, E)
    assert np.array_equal(m.picks[:rows].cpu().numpy(), p)
    dec = DecodedExperts(oracle, w)
    xb = np_u16(x)
    for r in (0, rows // 2 + 1, rows - 1):
        ys = np.stack([dec.row(xb[r], int(e), sk_gu=1, sk_d=1, warps=1)[0] for e in p[r]])
        want = oracle.combine(ys, wt[r:r + 1], 1, topk + 1)
        assert_close(out[r], want[0], what=f"config 5 K={bits} token {r}")
    sel = np.linspace(0, rows - 1, 64).astype(np.int64)
    y = window_reference(oracle, w, x[torch.from_numpy(sel).cuda()], p[sel], workers=16)
    assert_rows_close(out[sel], oracle.combine(y, wt[sel], len(sel), topk + 1), what=f"config 5 K={bits}, 64 tokens")


def _unpair(rows_u16):
    """Pair order of the prefill B operand (pair m of a 16-value k tile = (x[m + 8] low, x[m] high)) -> natural."""
    t = rows_u16.reshape(rows_u16.shape[0], -1, 8, 2)
    return np.concatenate([t[:, :, :, 1], t[:, :, :, 0]], axis=2).reshape(rows_u16.shape)


@pytest.mark.parametrize("hidden,slots,rows,shared_x", [
    (2048, 5, 37, False),     # the config 2-4 shape: 10 (slot, matrix) rows, up to 16 a launch form
    (1280, 5, 1, True),       # shared rotation: 5 rows
    (5120, 9, 13, False),     # config 5: 18 rows, up to 32
    (1280, 17, 3, False),     # 34 rows, up to 64
])
def test_prefill_rotation_bitexact(gfr, oracle, hidden, slots, rows, shared_x):
    """The prefill input rotation (prefill_rot_kernel) is rot_in (exl3.cu:224-241) bit for bit, for every pair and
    both matrices, at every (slot, matrix) row count the launch distinguishes."""
    import synth
    import dataclasses
    E = slots + 3
    w = synth.experts(E, hidden, 256, 2, seed=hidden + slots)
    if shared_x:
        w = dataclasses.replace(w, suh_u=w.suh_g)
    rng = np.random.default_rng(slots)
    picks_np = np.stack([rng.permutation(E)[:slots] for _ in range(rows)]).astype(np.int32)
    picks = torch.from_numpy(picks_np).cuda()
    x = synth.activations(rows, hidden, slots + 1)
    g = gfr.Grouping(E, slots, rows)
    g.run(picks, rows)
    fx = gfr.FastExperts(hidden, 256, slots, slots, E, rows)
    fx.run(w, x, picks, g.ids, g.count, g.members, rows, rows, shared_x=shared_x)
    torch.cuda.synchronize()
    xs = np_u16(x)
    for m in ((0,) if shared_x else (0, 1)):
        got = _unpair(np_u16(fx.rotated[m][:rows * slots]))
        suh = np_u16(w.suh_u if m else w.suh_g)
        for r in range(rows):
            for s in range(slots):
                want = oracle.rot(xs[r], suh[picks_np[r, s]])
                assert np.array_equal(got[r * slots + s], want), \
                    f"matrix {m} row {r} slot {s}: {np.sum(got[r * slots + s] != want)} values differ"


@pytest.mark.parametrize("hidden,routed,topk,rows,glm", [
    (2048, 64, 4, 37, False),     # config 3's shape: softmax gate, 5 slots
    (1024, 288, 8, 9, True),      # the reference's router: GLM's biased sigmoid gate over 288 experts, 9 slots
    (512, 16, 2, 256, False),     # the largest window of the route + group + rotation launch
    (512, 16, 2, 300, False),     # larger windows: the rotation rides on the grouping's scatter launch
    (1024, 288, 8, 260, True),    # ... with GLM's gate, full-K items
])
def test_moe_fused_rotation_bitexact(gfr, oracle, hidden, routed, topk, rows, glm):
    """Windows of at most 256 rows on the prefill engine route, group and rotate in one launch: workgroup 0 routes and
    groups, the others route their own token again and rotate its pairs; larger windows rotate in the grouping's
    scatter launch, from the routed picks. Both routings must pick the same experts:
    every rotated (pair, matrix) row against rot_in (exl3.cu:224-241) of the layer's pick for it, bit for bit, and
    the softmax gate's picks against the oracle's."""
    import synth
    w = synth.experts(routed + 1, hidden, 256, 2, seed=hidden + rows)
    x = synth.activations(rows, hidden, rows + 3)
    lg = synth.logits(rows, routed, rows + 4)
    m = gfr.Moe(hidden, 256, routed, topk, rows)
    bias = None
    if glm:
        bias = torch.randn(routed, generator=torch.Generator(device="cuda").manual_seed(5), device="cuda") * 0.1
        m.set_router(bias, 2.5)
    m.run(w, x, lg, rows)
    torch.cuda.synchronize()
    # the rotating workgroups must have used the picks workgroup 0 wrote (the routers themselves against the oracle,
    # near-ties of GLM's gate included, are tested with the decode path)
    p = m.picks[:rows].cpu().numpy()
    if not glm:
        assert np.array_equal(p, oracle.route(lg.cpu().numpy(), topk, routed)[0])
    xs = np_u16(x)
    for mat in (0, 1):
        got = _unpair(np_u16(m.rotated(mat, rows)))
        suh = np_u16(w.suh_u if mat else w.suh_g)
        for r in range(rows):
            for s in range(topk + 1):
                want = oracle.rot(xs[r], suh[p[r, s]])
                assert np.array_equal(got[r * (topk + 1) + s], want), \
                    f"matrix {mat} row {r} slot {s}: {np.sum(got[r * (topk + 1) + s] != want)} values differ"


@pytest.mark.parametrize("rows", [32, 300, 1024])
def test_moe_prefill_graph_replays(gfr, rows):
    """A captured prefill-engine layer replays to the eager bytes, across two weight sets and routings: a small window
    (route + group + rotation in one launch, split-K programs), a larger split-K window (the rotation in the
    grouping's scatter launch) and a full-K window. Each replay follows eager work that clears the output."""
    import synth
    E, D, N, bits, topk = 16, 512, 256, 4, 2
    ws = [synth.experts(E + 1, D, N, bits, seed=s) for s in (31, 32)]
    xs = [synth.activations(rows, D, 33 + j) for j in range(2)]
    lgs = [synth.logits(rows, E, 35 + j) for j in range(2)]
    m = gfr.Moe(D, N, E, topk, rows)
    s = torch.cuda.Stream()
    eager = []
    with torch.cuda.stream(s):
        for j in range(2):
            m.run(ws[j], xs[j], lgs[j], rows, stream=s)
            s.synchronize()
            eager.append(m.output[:rows].clone())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            m.run(ws[0], xs[0], lgs[0], rows, stream=s)
            m.run(ws[1], xs[1], lgs[1], rows, stream=s)
    assert not torch.equal(eager[0], eager[1])
    for _ in range(3):
        m.output.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.output[:rows], eager[1])


def test_split_window_with_many_experts(gfr, oracle):
    """A split-K window (at most 2048 pairs, 32-row items) whose routing spreads over 1023 experts with one member each
    plus a shared expert with every row: the plan holds 1023 + 32 items, more than an item count sized for 128-row
    items would hold. Sampled tokens against the oracle."""
    import synth
    routed, topk, rows, Dk, Nk, bits = 1023, 1, 1024, 512, 512, 4
    w = synth.experts(routed + 1, Dk, Nk, bits, seed=1023)
    x = synth.activations(rows, Dk, 11)
    lg = torch.randn((rows, routed), generator=torch.Generator(device="cuda").manual_seed(12), device="cuda")
    target = torch.arange(rows, device="cuda") % routed
    lg[torch.arange(rows, device="cuda"), target] = 10.0
    m = gfr.Moe(Dk, Nk, routed, topk, rows)
    m.run(w, x, lg, rows)
    torch.cuda.synchronize()
    out = m.output[:rows].cpu().numpy()
    assert np.all(np.isfinite(out))
    p, wt = oracle.route(lg.cpu().numpy(), topk, routed)
    assert np.array_equal(m.picks[:rows].cpu().numpy(), p)
    assert len(set(p[:, 0].tolist())) == routed
    dec = DecodedExperts(oracle, w)
    xb = np_u16(x)
    for r in (0, 511, 1022, 1023):
        ys = np.stack([dec.row(xb[r], int(e), sk_gu=1, sk_d=1, warps=1)[0] for e in p[r]])
        want = oracle.combine(ys, wt[r:r + 1], 1, topk + 1)
        assert_close(out[r], want[0], what=f"token {r}")
    y = window_reference(oracle, w, x, p, workers=16)
    assert_rows_close(out, oracle.combine(y, wt, rows, topk + 1), what="1023 experts, every token")
