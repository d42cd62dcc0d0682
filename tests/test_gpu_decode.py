"""Decode / verify path on the GPU against the CPU oracle: decoded weights bit-exact, grouping bit-exact, layer
outputs within the north star's 1e-2 relative (plus the reference probe's 1e-3 relative RMS, experts.rs:304-308)."""
import numpy as np
import pytest
import torch

from refs import DecodedExperts, assert_close, assert_decode_close, assert_rows_close, np_u16, np_u32, window_reference

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_decode_tiles_bitexact(gfr, oracle, bits):
    import synth
    kin, n = 64, 384
    w = synth.trellis((kin // 16, n // 16, 8 * bits), 77 + bits)
    w[0, 0].zero_()
    w[0, 1].fill_(-1)
    w[1, 2].zero_()
    w[1, 2, 3] = 1 << 7
    got = np_u16(gfr.decode_tiles(w, kin, n, bits))
    torch.cuda.synchronize()
    want = oracle.unpack(np_u32(w), kin, n, bits)
    assert np.array_equal(got, want), f"{np.sum(got != want)} of {got.size} decoded weights differ"


def _xorshift_picks(rows, concentrated, seed):
    M = (1 << 64) - 1
    picks = []
    for r in range(rows):
        seed ^= (seed << 13) & M
        seed ^= seed >> 7
        seed ^= (seed << 17) & M
        start = 0 if concentrated else seed % 288
        picks.append([(288 if s == 8 else (start + s * 37) % 288) for s in range(9)])
    return np.array(picks, np.int32), seed


@pytest.mark.parametrize("capacity,row_counts", [
    (8192, [8192, 1, 2, 31, 32, 33, 63, 64, 65, 129, 1024, 4097, 8191, 8192]),
    (16, [1, 2, 3, 8, 15, 16]),
])
def test_grouping_reference_probe(gfr, oracle, capacity, row_counts):
    """grouping.rs:123-215: seeded xorshift64 routing, poisoned outputs, exact count / ids / full members table,
    graph replays."""
    g = gfr.Grouping(289, 9, capacity)
    seed = 0x0123456789ABCDEF
    for rows in row_counts:
        for concentrated in (True, False):
            p, seed = _xorshift_picks(rows, concentrated, seed)
            picks = torch.from_numpy(p).cuda()
            c, ids, mem = oracle.group(p, rows, 9, 289, capacity)
            g.ids.fill_(-77)
            g.members.fill_(12345)
            g.run(picks, rows)
            torch.cuda.synchronize()

            def check():
                assert int(g.count.item()) == c, (rows, concentrated)
                assert np.array_equal(g.ids[:c].cpu().numpy(), ids), (rows, concentrated)
                assert np.array_equal(g.members.cpu().numpy(), mem), (rows, concentrated)

            check()
            if rows in (1, 65, 4097):
                graph = torch.cuda.CUDAGraph()
                s = torch.cuda.Stream()
                with torch.cuda.stream(s):
                    g.run(picks, rows, stream=s)   # warm
                    s.synchronize()
                    with torch.cuda.graph(graph, stream=s):
                        g.run(picks, rows, stream=s)
                for _ in range(3):
                    g.members.fill_(12345)
                    torch.cuda.synchronize()
                    graph.replay()
                    torch.cuda.synchronize()
                    check()


@pytest.mark.parametrize("E,slots,rows", [(65, 5, 1), (65, 5, 32), (161, 9, 16384), (65, 5, 8192), (161, 9, 300)])
def test_grouping_benchmark_shapes(gfr, oracle, E, slots, rows):
    import synth
    lg = synth.zipf_logits(rows, E - 1, slots - 1, 1.1, seed=rows + E) if rows <= 2048 else synth.logits(rows, E - 1, 5)
    p, _ = oracle.route(lg.cpu().numpy(), slots - 1, E - 1)
    g = gfr.Grouping(E, slots, rows)
    g.run(torch.from_numpy(p).cuda(), rows)
    torch.cuda.synchronize()
    c, ids, mem = oracle.group(p, rows, slots, E, rows)
    assert int(g.count.item()) == c
    assert np.array_equal(g.ids[:c].cpu().numpy(), ids)
    assert np.array_equal(g.members.cpu().numpy(), mem)


@pytest.mark.parametrize("kin,n,bits", [(2048, 1536, 4), (2048, 1536, 3), (768, 512, 2), (1280, 256, 5)])
def test_linear_config1(gfr, oracle, kin, n, bits):
    """one EXL3 linear 2048 -> 1536, K = 4, one fp16 token (and other widths / shapes: 768 and 1280
    inputs take the two-wave form of the fused-rotation GEMV)."""
    import synth
    t = synth.trellis((kin // 16, n // 16, 8 * bits), 11)
    suh, svh = synth.scales((kin,), 12), synth.scales((n,), 13)
    x = torch.randn(kin, generator=torch.Generator(device="cuda").manual_seed(14), device="cuda").half()
    y = torch.empty(n, device="cuda")
    lin = gfr.Linear(kin, n, bits)
    lin.run(x, t, suh, svh, y)
    torch.cuda.synchronize()
    want = [oracle.linear(np_u16(x), oracle.unpack_f32(np_u32(t), kin, n, bits, rounded), np_u16(suh), np_u16(svh))
            for rounded in (False, True)]
    assert_decode_close(y.cpu().numpy(), *want, what="linear")


DECODE_ROWS = 4   # Moe runs windows of up to this many rows on the decode engine (gfr_moe_set_decode_rows default)


def _check_tokens(oracle, w, x, picks, weights, out, tokens, slots, what=""):
    """Moe outputs of the given tokens against the oracle: windows on the decode engine against both weight forms
    (assert_decode_close), larger windows (the MFMA path, fp16 weights as the reference) at the tight bar."""
    rows = out.shape[0]
    decs = [DecodedExperts(oracle, w, rounded) for rounded in ((False, True) if rows <= DECODE_ROWS else (True,))]
    xb = np_u16(x)
    for r in tokens:
        want = [oracle.combine(np.stack([d.row(xb[r], int(e))[0] for e in picks[r]]), weights[r:r + 1], 1, slots)[0]
                for d in decs]
        if rows <= DECODE_ROWS:
            assert_decode_close(out[r], *want, what=f"{what} token {r}")
        else:
            assert_close(out[r], want[0], what=f"{what} token {r}")


def _moe_inputs(E_routed, D, N, bits, rows, topk, seed, zipf=False):
    import synth
    w = synth.experts(E_routed + 1, D, N, bits, seed=seed)
    x = synth.activations(rows, D, seed + 100)
    lg = synth.zipf_logits(rows, E_routed, topk, 1.1, seed + 200) if zipf else synth.logits(rows, E_routed, seed + 200)
    return w, x, lg


@pytest.mark.parametrize("rows,zipf", [(1, False), (4, True), (13, True)])
def test_experts_run_rows_vs_oracle(gfr, oracle, rows, zipf):
    """ExpertGpu::run_rows at the C2 / C3 shape (hidden 2048, inter 1536, 64 + 1 EXL3 experts, top-4 + shared); at 13
    rows the shared expert's members take two programs (chunks of 8)."""
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    slots = topk + 1
    w, x, lg = _moe_inputs(E, D, N, bits, rows, topk, 31 + rows, zipf)
    p, _ = oracle.route(lg.cpu().numpy(), topk, E)
    picks = torch.from_numpy(p).cuda()
    g = gfr.Grouping(E + 1, slots, 16)
    ex = gfr.ExpertGpu(D, N, slots, slots, 16)
    g.run(picks, rows)
    ex.run_rows(w, x, picks, g.ids, g.count, g.members, rows, 16)
    torch.cuda.synchronize()
    y = ex.y.cpu().numpy()
    dec, ref = DecodedExperts(oracle, w, rounded=False), DecodedExperts(oracle, w)
    xb = np_u16(x)
    for r in range(rows):
        for s in range(slots):
            e = int(p[r, s])
            assert_decode_close(y[r * slots + s], dec.row(xb[r], e)[0], ref.row(xb[r], e)[0],
                                what=f"row {r} slot {s} expert {e}")


def test_batched_rows_equal_serial_rows(gfr, oracle):
    """window_experts_probe.rs:14-188: a 16-row batched run is byte-identical to per-row runs (row independence),
    for identical, partially overlapping and disjoint routing."""
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    slots = topk + 1
    w, x, _ = _moe_inputs(E, D, N, bits, 16, topk, 5)
    g = gfr.Grouping(E + 1, slots, 16)
    ex = gfr.ExpertGpu(D, N, slots, slots, 16)
    one_g = gfr.Grouping(E + 1, slots, 1)
    one = gfr.ExpertGpu(D, N, slots, slots, 1)
    for pattern in range(3):
        p = np.array([[(s * 13 + (0 if pattern == 0 else r * 13 if pattern == 1 else r * 4)) % E for s in range(topk)]
                      + [E] for r in range(16)], np.int32)
        picks = torch.from_numpy(p).cuda()
        for rows in (1, 2, 7, 16):
            g.run(picks, rows)
            ex.run_rows(w, x, picks, g.ids, g.count, g.members, rows, 16)
            batched = ex.y[:rows * slots].clone()
            for r in range(rows):
                pr = picks[r:r + 1].contiguous()
                one_g.run(pr, 1)
                one.run_rows(w, x[r:r + 1], pr, one_g.ids, one_g.count, one_g.members, 1, 1)
                assert torch.equal(one.y[:slots], batched[r * slots:(r + 1) * slots]), (pattern, rows, r)


def test_experts_graph_replay_bytes(gfr):
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    slots = topk + 1
    w, x, lg = _moe_inputs(E, D, N, bits, 3, topk, 8)
    picks = torch.tensor([[1, 5, 9, 33, 64], [5, 2, 9, 40, 64], [63, 0, 1, 2, 64]], dtype=torch.int32, device="cuda")
    g = gfr.Grouping(E + 1, slots, 4)
    ex = gfr.ExpertGpu(D, N, slots, slots, 4)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g.run(picks, 3, stream=s)
        ex.run_rows(w, x, picks, g.ids, g.count, g.members, 3, 4, stream=s)
        s.synchronize()
        eager = ex.y.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            g.run(picks, 3, stream=s)
            ex.run_rows(w, x, picks, g.ids, g.count, g.members, 3, 4, stream=s)
    for _ in range(3):
        ex.y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ex.y, eager)


def test_moe_layer_decode_vs_oracle(gfr, oracle):
    """Moe layer, config 2 (bs = 1 decode): router -> grouping -> experts -> combine."""
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    w, x, lg = _moe_inputs(E, D, N, bits, 1, topk, 21)
    m = gfr.Moe(D, N, E, topk, 1)
    m.run(w, x, lg, 1)
    torch.cuda.synchronize()
    p, wt = oracle.route(lg.cpu().numpy(), topk, E)
    assert np.array_equal(m.picks.cpu().numpy(), p)
    np.testing.assert_allclose(m.weights.cpu().numpy(), wt, rtol=1e-6)
    want = []
    for rounded in (False, True):
        dec = DecodedExperts(oracle, w, rounded)
        ys = np.stack([dec.row(np_u16(x)[0], int(e))[0] for e in p[0]])
        want.append(oracle.combine(ys, wt, 1, topk + 1))
    assert_decode_close(m.output.cpu().numpy(), *want, what="moe output")


def test_moe_graph_replay_bytes(gfr):
    """A captured MoE layer (router .. combine) replays to the eager bytes, across different weights and routing."""
    import synth
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    ws = [synth.experts(E + 1, D, N, bits, seed=s) for s in (3, 4)]
    x = synth.activations(2, D, 1)
    lg = synth.logits(2, E, 2)
    m = gfr.Moe(D, N, E, topk, 1)
    s = torch.cuda.Stream()
    eager = []
    with torch.cuda.stream(s):
        for j in range(2):
            m.run(ws[j], x[j:j + 1], lg[j:j + 1], 1, stream=s)
            s.synchronize()
            eager.append(m.output.clone())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            m.run(ws[0], x[0:1], lg[0:1], 1, stream=s)
            m.run(ws[1], x[1:2], lg[1:2], 1, stream=s)
    for _ in range(3):
        m.output.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.output, eager[1])


def test_grouped_gemv_entry_matches_run_rows(gfr):
    """gfr_exl3_grouped_gemv (the exported GEMV) computes the Z partials run_rows uses: sum of splits equals the
    fp32 dot products of the rotated rows with the decoded weights to rounding."""
    import synth
    L = gfr.lib()
    E, D, N, bits = 3, 512, 256, 4
    w = synth.experts(E, D, N, bits, seed=9)
    g = gfr.Grouping(E, 2, 2)
    picks = torch.tensor([[0, 2], [2, 1]], dtype=torch.int32, device="cuda")
    g.run(picks, 2)
    X = torch.randn((2, 4, D), device="cuda").half()
    SK = L.gfr_exl3_gemv_splits(D)
    Z = torch.zeros((2, SK, 4, N), device="cuda")
    gfr._check(L.gfr_exl3_grouped_gemv(torch.cuda.current_stream().cuda_stream, X[0].data_ptr(), X[1].data_ptr(),
                                       w.gt.data_ptr(), w.ut.data_ptr(), g.ids.data_ptr(), g.count.data_ptr(),
                                       g.members.data_ptr(), Z.data_ptr(), D, N, 4, 2, 2, E, bits, 2, 4))
    torch.cuda.synchronize()
    p = picks.cpu().numpy().reshape(-1)
    for mat, t in enumerate((w.gt, w.ut)):
        for pair in range(4):
            W = gfr.decode_tiles(t[int(p[pair])], D, N, bits).float()
            want = X[mat, pair].float() @ W
            got = Z[mat, :, pair].sum(0)
            assert torch.allclose(got, want, rtol=1e-3, atol=1e-3 * want.abs().max().item())


@pytest.mark.parametrize("rows", [3, 32])
def test_moe_layer_verify_window_vs_oracle(gfr, oracle, rows):
    """Moe layer, config 3 shape (a verify window with Zipf(1.1)-skewed routing): every token's output."""
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    w, x, lg = _moe_inputs(E, D, N, bits, rows, topk, 40 + rows, zipf=True)
    m = gfr.Moe(D, N, E, topk, rows)
    m.run(w, x, lg, rows)
    torch.cuda.synchronize()
    p, wt = oracle.route(lg.cpu().numpy(), topk, E)
    assert np.array_equal(m.picks[:rows].cpu().numpy(), p)
    out = m.output[:rows].cpu().numpy()
    _check_tokens(oracle, w, x, p, wt, out, range(rows) if rows <= 4 else (0, 7, rows - 1), topk + 1)
    if rows > 4:     # every token of the window
        y = window_reference(oracle, w, x, p, workers=16)
        assert_rows_close(out, oracle.combine(y, wt, rows, topk + 1), what=f"{rows}-token window, every token")


def test_rotation_bitexact(gfr, oracle):
    """The 128-point transform (DPP / permlane butterflies) reproduces rot_in's fp32 sums bit for bit."""
    import synth
    rows, k, E = 7, 2048, 5
    suh = synth.scales((E, k), 3)
    x = synth.activations(rows, k, 4)
    ex = torch.tensor([0, 4, 2, 2, 1, 3, 0], dtype=torch.int32, device="cuda")
    got = np_u16(gfr.rotate(x, ex, suh))
    xs, ss = np_u16(x), np_u16(suh)
    for r in range(rows):
        want = oracle.rot(xs[r], ss[int(ex[r])])
        assert np.array_equal(got[r], want), f"row {r}: {np.sum(got[r] != want)} values differ"


@pytest.mark.parametrize("rows,E,topk", [(64, 64, 4), (33, 160, 8), (5, 1000, 8)])
def test_route_vs_oracle(gfr, oracle, rows, E, topk):
    """Router picks exact (ties to the lower id), weights to fp32 rounding."""
    g = torch.Generator().manual_seed(E)
    lg = torch.randn((rows, E), generator=g)
    lg[0, :] = 0.5                          # all tied: picks 0..k-1
    lg[1, 10:20] = 3.0                      # a tied block on top
    lg[2, [c for c in (70, 5, 130, 66, 69) if c < E]] = 4.0   # ties across 64-id blocks and lanes
    lg = lg.cuda()
    picks, w = gfr.route(lg, topk)
    torch.cuda.synchronize()
    p, wt = oracle.route(lg.cpu().numpy(), topk, E)
    assert np.array_equal(picks.cpu().numpy(), p)
    np.testing.assert_allclose(w.cpu().numpy(), wt, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_moe_layer_config5_decode_vs_oracle(gfr, oracle, bits):
    """Config 5's layer shape at bs = 1 (hidden 5120, 160 routed + 1 shared, top-8, inter 1536), each of the stack's
    bit widths K = 2, 3, 4, 5, through the Moe entry point against the oracle (routing exact, output within
    tolerance)."""
    import synth
    E, D, N, topk = 160, 5120, 1536, 8
    w = synth.experts(E + 1, D, N, bits, seed=60 + bits)
    x = synth.activations(1, D, 61)
    lg = synth.zipf_logits(1, E, topk, 1.1, 62)
    m = gfr.Moe(D, N, E, topk, 1)
    m.run(w, x, lg, 1)
    torch.cuda.synchronize()
    p, wt = oracle.route(lg.cpu().numpy(), topk, E)
    assert np.array_equal(m.picks.cpu().numpy(), p)
    _check_tokens(oracle, w, x, p, wt, m.output[:1].cpu().numpy(), (0,), topk + 1, what=f"config 5 K={bits}")


def test_config5_decode_graph_replays_match_eager(gfr):
    """Config 5's K = 5 layer at bs = 1 (hidden 5120: the gate/up launch's read-ahead of the down matrices takes two
    loads a lane there) over 4 tokens, captured in one graph and replayed 3 times with eager runs in between: every
    replay's outputs equal the eager ones bit for bit."""
    import synth
    E, D, N, topk, bits, T = 160, 5120, 1536, 8, 5, 4
    w = synth.experts(E + 1, D, N, bits, seed=70)
    x = synth.activations(T, D, 71)
    lg = synth.zipf_logits(T, E, topk, 1.1, 72)
    m = gfr.Moe(D, N, E, topk, 1)
    outs = torch.empty(T, D, device="cuda")
    s = torch.cuda.Stream()

    def run_all():
        for t in range(T):
            m.run(w, x[t:t + 1], lg[t:t + 1], 1, stream=s)
            outs[t].copy_(m.output[0])     # a device copy on the same stream, captured with the layer

    with torch.cuda.stream(s):
        run_all()
    s.synchronize()
    eager = outs.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            run_all()
    for _ in range(3):
        with torch.cuda.stream(s):
            outs.zero_()
            g.replay()
        s.synchronize()
        assert torch.equal(outs, eager)
        with torch.cuda.stream(s):
            run_all()
        s.synchronize()
        assert torch.equal(outs, eager)


def _biased_inputs(rows, E, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    logits = torch.randn(rows, E, generator=g, device="cuda")
    bias = torch.randn(E, generator=g, device="cuda") * 0.05
    return logits, bias


def _check_biased(oracle, picks, weights, logits, bias, topk, E):
    """GPU picks / weights of GLM's gate against the oracle; a near-tie at the k-th place may go either way."""
    p, wt = oracle.route_biased(logits.cpu().numpy(), bias.cpu().numpy(), 2.5, topk, E)
    gp, gw = picks.cpu().numpy(), weights.cpu().numpy()
    s = 1.0 / (1.0 + np.exp(-logits.cpu().numpy().astype(np.float64)))
    choice = s + bias.cpu().numpy()
    for r in range(p.shape[0]):
        srt = np.sort(choice[r])[::-1]
        if srt[topk - 1] - srt[topk] > 1e-5:
            assert list(gp[r]) == list(p[r]), r
            np.testing.assert_allclose(gw[r], wt[r], rtol=2e-6)
        else:   # the picks are a valid top-k of the biased scores
            assert set(gp[r, :topk]) <= set(np.argsort(-choice[r])[:topk + 1])
    return p, wt


@pytest.mark.parametrize("rows,E,topk", [(64, 64, 4), (33, 160, 8), (17, 288, 8)])
def test_route_biased_vs_oracle(gfr, oracle, rows, E, topk):
    """GLM's gate (the reference's topk(logits, bias, .., 2.5) call, moe.rs:89-99) at the benchmark's and the
    reference's (288 routed, top-8) shapes."""
    logits, bias = _biased_inputs(rows, E, 70 + E)
    picks, weights = gfr.route_biased(logits, bias, topk, 2.5)
    torch.cuda.synchronize()
    _check_biased(oracle, picks, weights, logits, bias, topk, E)


@pytest.mark.parametrize("rows", [1, 3, 32])
def test_moe_layer_biased_router_vs_oracle(gfr, oracle, rows):
    """A Moe layer with GLM's gate on every routing path: the router fused into the bs = 1 gate/up GEMV, the decode
    window's route + group launch and the split-K window's route + group + plan launch."""
    E, D, N, bits, topk = 64, 2048, 1536, 4, 4
    w, x, _ = _moe_inputs(E, D, N, bits, rows, topk, 90 + rows)
    logits, bias = _biased_inputs(rows, E, 95 + rows)
    m = gfr.Moe(D, N, E, topk, rows)
    m.set_router(bias, 2.5)
    m.run(w, x, logits, rows)
    torch.cuda.synchronize()
    p, wt = _check_biased(oracle, m.picks[:rows], m.weights[:rows], logits, bias, topk, E)
    gp, gw = m.picks[:rows].cpu().numpy(), m.weights[:rows].cpu().numpy()
    _check_tokens(oracle, w, x, gp, gw, m.output[:rows].cpu().numpy(), range(rows) if rows <= 3 else (0, rows - 1),
                  topk + 1)
    m.set_router(None)
    m.run(w, x, logits, rows)
    torch.cuda.synchronize()
    p2, _ = oracle.route(logits.cpu().numpy(), topk, E)
    assert np.array_equal(m.picks[:rows].cpu().numpy(), p2)
