"""The reference's FP8 shared expert (moe.rs:132-167: fmm(shared_gu, sk 8) -> reduce8_bf16 -> shared_swiglu ->
fmm(shared_down, sk 1)) through gfr_shared_fp8 and the layer entry points gfr_moe_run_fp8 / _run_router_fp8, at the
reference's geometry (hidden 4096, intermediate 512, 288 routed experts top-8 + the shared one), against the CPU
oracle's restatement of the reference's scalar oracle (front.rs:190-217, 669-675). Weights are seeded synthetic
tensors of the reference's shapes (its checkpoint is not available here)."""
import numpy as np
import pytest
import torch

from refs import DecodedExperts, assert_close, assert_rows_close, np_u16

pytestmark = pytest.mark.gpu

D, N, E, TOPK, BITS = 4096, 512, 288, 8, 4


@pytest.fixture(scope="module")
def sw():
    import synth
    return synth.fp8_shared(D, N, seed=77)


@pytest.fixture(scope="module")
def host_sw(sw):
    return (sw.gu.cpu().numpy(), np_u16(sw.gu_scale), sw.down.cpu().numpy(), np_u16(sw.down_scale))


def bf16_floats(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_bf16_ulps(got, want, what, max_frac=0.02):
    """bf16 results whose fp32 sums were added in another order: equal, or one bf16 step apart (a sum that sits next
    to a rounding boundary), and such steps rare."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    step = np.abs(want) * 2.0 ** -7 + 1e-30
    diff = np.abs(got - want)
    assert np.all(diff <= step), f"{what}: {int(np.sum(diff > step))} values more than one bf16 step apart"
    frac = float(np.mean(diff > 0))
    assert frac <= max_frac, f"{what}: {frac:.3%} of the values differ"


@pytest.mark.parametrize("rows", [1, 3, 16, 17, 40])
def test_shared_fp8_vs_oracle(gfr, oracle, sw, host_sw, rows):
    """Every row: gu (bf16) against reference_mm_at(sk 8, rounded), act against the SwiGLU of the kernel's own gu,
    out against reference_mm_at(sk 1) of the kernel's own act (the fp32 sums within their accumulation error), and
    the whole chain from x against the oracle's chain. 17 and 40 rows take partial 16-row blocks; the input has a
    padded row stride."""
    g = torch.Generator(device="cuda").manual_seed(rows)
    xs = torch.randn((rows, D + 24), generator=g, device="cuda").to(torch.bfloat16)
    x = xs[:, :D]
    sh = gfr.SharedFp8(D, N, 64)
    out = torch.full((rows, D + 8), float("nan"), device="cuda")
    sh.run(sw, x, rows, out=out)
    torch.cuda.synchronize()
    wgu, sgu, wd, sd = host_sw
    xb = np_u16(x)
    gu_k = bf16_floats(np_u16(sh.gu[:rows]))
    act_k = bf16_floats(np_u16(sh.act[:rows]))
    out_k = out[:, :D].cpu().numpy()
    assert np.all(np.isnan(out[:, D:].cpu().numpy())), "columns past hidden must stay untouched"
    wdv = oracle.fp8_values().astype(np.float64)[wd]
    sdv = bf16_floats(sd).astype(np.float64)
    chain = []
    for r in range(rows):
        gu_o, act_o, out_o = oracle.shared_fp8_row(xb[r], wgu, sgu, wd, sd)
        assert_bf16_ulps(gu_k[r], gu_o, f"rows {rows} row {r} gu")
        assert_bf16_ulps(act_k[r], oracle.shared_swiglu(gu_k[r], N), f"rows {rows} row {r} act", max_frac=0.01)
        want = oracle.fp8_matmul(act_k[r], wd, sd, 1, False)
        bound = (np.abs(wdv) @ np.abs(act_k[r]).astype(np.float64)) * sdv * N * 2.0 ** -23 + 1e-30
        assert np.all(np.abs(out_k[r] - want) <= bound), f"rows {rows} row {r} out"
        chain.append(out_o)
    assert_rows_close(out_k, np.stack(chain), rel_rms=1e-2, rel_max=5e-2, what=f"rows {rows} x -> out chain")


def test_shared_fp8_limit_clamps(gfr, oracle, host_sw):
    """Gate / up values far beyond the limit of 10 (scales x 64): the SwiGLU saturates as the oracle's does."""
    import synth
    big = synth.fp8_shared(D, N, seed=78)
    big.gu_scale = (big.gu_scale.float() * 64).to(torch.bfloat16)
    x = torch.randn((2, D), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda").to(torch.bfloat16)
    sh = gfr.SharedFp8(D, N, 2)
    sh.run(big, x, 2)
    torch.cuda.synchronize()
    gu_k = bf16_floats(np_u16(sh.gu[:2]))
    assert np.mean(np.abs(gu_k) > 10) > 0.2, "the test needs values beyond the limit"
    for r in range(2):
        assert_bf16_ulps(bf16_floats(np_u16(sh.act[r])), oracle.shared_swiglu(gu_k[r], N), f"row {r} act",
                         max_frac=0.01)


def test_shared_fp8_graph_replays(gfr, sw):
    """Captured and replayed, the two launches give the eager bytes (no allocation, no host sync in run)."""
    x = torch.randn((5, D), generator=torch.Generator(device="cuda").manual_seed(9), device="cuda").to(torch.bfloat16)
    sh = gfr.SharedFp8(D, N, 8)
    out = torch.zeros((5, D), device="cuda")
    sh.run(sw, x, 5, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            sh.run(sw, x, 5, out=out, stream=s)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_shared_fp8_rejects_misaligned(gfr, sw):
    sh = gfr.SharedFp8(D, N, 2)
    x = torch.zeros((2, D + 8), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(gfr.GfrError, match="16-byte aligned"):
        sh.run(sw, x[:, 1:], 2)
    out = torch.zeros((2, D + 4), device="cuda")
    with pytest.raises(gfr.GfrError, match="16-byte aligned"):
        sh.run(sw, x[:, :D], 2, out=out[:, 1:])


@pytest.fixture(scope="module")
def routed():
    import synth
    return synth.experts(E, D, N, BITS, seed=288)


@pytest.mark.parametrize("rows", [1, 3, 40])
def test_moe_run_fp8_reference_layout(gfr, oracle, sw, host_sw, routed, rows):
    """Moe::run_prefetched with its FP8 shared expert: the layer's output equals the combine of the routed experts
    with the shared expert's own output (byte for byte against gfr_moe_run_shared fed with gfr_shared_fp8's output),
    and sampled tokens match the oracle's routed rows + shared row combined."""
    g = torch.Generator(device="cuda").manual_seed(500 + rows)
    x = torch.randn((rows, D), generator=g, device="cuda").to(torch.bfloat16)
    router_w = (torch.randn((E, D), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    bias = torch.randn(E, generator=g, device="cuda") * 0.05
    m = gfr.Moe(D, N, E, TOPK, max(rows, 4), shared_exl3=False)
    m.set_router(bias, 2.5)
    m.run_router_fp8(routed, x, router_w, sw, rows)
    torch.cuda.synchronize()
    got = m.output[:rows].clone()
    shared = m.shared_output[:rows].clone()
    sh = gfr.SharedFp8(D, N, rows)
    torch.testing.assert_close(sh.run(sw, x, rows), shared, rtol=0, atol=0)
    m2 = gfr.Moe(D, N, E, TOPK, max(rows, 4), shared_exl3=False)
    m2.set_router(bias, 2.5)
    m2.run_router(routed, x, router_w, rows, shared=shared)
    torch.cuda.synchronize()
    assert torch.equal(m2.output[:rows], got)
    # with the logits given (gfr_moe_run_fp8): the same bytes
    logits = gfr.router_logits(x, router_w)
    m.output.zero_()
    m.run_fp8(routed, x, logits, sw, rows)
    torch.cuda.synchronize()
    assert torch.equal(m.output[:rows], got)
    # sampled tokens against the oracle: routed rows (the reference's fp16 weights) + the oracle's shared row
    gp, gw = m.picks[:rows].cpu().numpy(), m.weights[:rows].cpu().numpy()
    assert np.all(gp[:, TOPK] == E)
    dec = DecodedExperts(oracle, routed, rounded=rows > 4)
    xb = np_u16(x)
    wgu, sgu, wd, sd = host_sw
    for r in sorted({0, rows - 1}):
        ys = [dec.row(xb[r], int(e))[0] if rows <= 4 else dec.row(xb[r], int(e), sk_gu=1, sk_d=1, warps=1)[0]
              for e in gp[r, :TOPK]]
        ys.append(oracle.shared_fp8_row(xb[r], wgu, sgu, wd, sd)[2])
        want = oracle.combine(np.stack(ys), gw[r:r + 1], 1, TOPK + 1)[0]
        assert_close(got[r].cpu().numpy(), want, rel_rms=1e-2, rel_max=5e-2, what=f"rows {rows} token {r}")


def test_prepared_shared_fp8(gfr, sw, routed, tmp_path):
    """The prepared-weight format carries the shared expert (weights.layers[L].moe.shared.{gu,down}.{weight,scale},
    float8_e4m3fn / bfloat16); gfr_prepared_shared_fp8 finds it and the loaded tensors give the same output."""
    import synth
    small = synth.experts(4, 512, 256, BITS, seed=3)
    sw_small = synth.fp8_shared(512, 256, seed=5)
    path = gfr.write_prepared(str(tmp_path / "p"), [small], shared=[sw_small])
    p = gfr.Prepared(path)
    p.expect("weights.layers[0].moe.shared.gu.weight", "float8_e4m3fn", [512, 512])
    p.expect("weights.layers[0].moe.shared.down.scale", "bfloat16", [512])
    p.load()
    loaded = p.shared_fp8(0)
    assert loaded.hidden == 512 and loaded.inter == 256
    assert torch.equal(loaded.gu, sw_small.gu) and torch.equal(loaded.down_scale, sw_small.down_scale)
    x = torch.randn((3, 512), generator=torch.Generator(device="cuda").manual_seed(1), device="cuda").to(torch.bfloat16)
    sh = gfr.SharedFp8(512, 256, 3)
    a = sh.run(loaded, x, 3)
    b = sh.run(sw_small, x, 3)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    with pytest.raises(gfr.GfrError):
        p.shared_fp8(1)


@pytest.mark.parametrize("routed,topk,H,I", [(16, 4, 512, 256), (4, 4, 512, 256), (64, 4, 2048, 1536),
                                             (24, 8, 5120, 1536)])
def test_moe_run_fp8_one_token_forms(gfr, oracle, routed, topk, H, I):
    """One token: with at least `slots` routed experts the shared expert rides on the EXL3 gate/up and down launches
    (the shared slot's workgroups); with fewer (4 routed, top-4: the grid has no shared unit) it runs its own two
    launches first. Both give the bytes of gfr_moe_run_shared fed with gfr_shared_fp8's output, eagerly and in every
    replay of a captured graph; at config 2's shape (one-wave down programs) and config 5's (hidden 5120: two output
    blocks a down workgroup, 10 gate/up splits) as well."""
    import synth
    w = synth.experts(routed, H, I, BITS, seed=routed)
    sw1 = synth.fp8_shared(H, I, seed=routed + 1)
    x = torch.randn((1, H), generator=torch.Generator(device="cuda").manual_seed(2), device="cuda").to(torch.bfloat16)
    lg = synth.logits(1, routed, 3)
    m = gfr.Moe(H, I, routed, topk, 1, shared_exl3=False)
    m.run_fp8(w, x, lg, sw1, 1)
    torch.cuda.synchronize()
    got = m.output[:1].clone()
    shared = gfr.SharedFp8(H, I, 1).run(sw1, x, 1)
    torch.cuda.synchronize()
    assert torch.equal(m.shared_output[:1], shared)
    m2 = gfr.Moe(H, I, routed, topk, 1, shared_exl3=False)
    m2.run(w, x, lg, 1, shared=shared)
    torch.cuda.synchronize()
    assert torch.equal(m2.output[:1], got)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            m.run_fp8(w, x, lg, sw1, 1, stream=s)
    for _ in range(3):
        m.output.zero_()
        m.shared_output.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.output[:1], got)


# ---- the prefill form (prefill.rs:55-150, batch.rs:1183-1195): bf16 weight copies and library GEMMs -----------------
@pytest.fixture(scope="module")
def sw_prepared():
    import synth
    w = synth.fp8_shared(D, N, seed=79)
    w.prepare_bf16()
    torch.cuda.synchronize()
    return w


def test_prepare_bf16_bit_exact(oracle, sw_prepared):
    """gfr_fp8_prepare_bf16 against the oracle's f8_b16_copy, bit for bit, both matrices."""
    w = sw_prepared
    got_gu = np_u16(w.gu_bf16)
    got_d = np_u16(w.down_bf16)
    np.testing.assert_array_equal(got_gu, oracle.fp8_b16_copy(w.gu.cpu().numpy(), np_u16(w.gu_scale)))
    np.testing.assert_array_equal(got_d, oracle.fp8_b16_copy(w.down.cpu().numpy(), np_u16(w.down_scale)))


@pytest.mark.parametrize("rows", [17, 300, 2048])
def test_shared_fp8_prefill_form(gfr, oracle, sw_prepared, rows):
    """More than 16 rows with the bf16 copies: gu = bf16(x . gu_bf16^T) within one bf16 step of the float64 product
    (the library's fp32 order), act within one step of the oracle's SwiGLU of the kernel's gu, out within the fp32
    accumulation bound of act . down_bf16^T; sampled rows, first, middle and last, and every row's chain within 1e-2
    of the slice arithmetic's (the two forms differ by the weights' bf16 rounding)."""
    w = sw_prepared
    g = torch.Generator(device="cuda").manual_seed(rows)
    x = torch.randn((rows, D), generator=g, device="cuda").to(torch.bfloat16)
    sh = gfr.SharedFp8(D, N, rows)
    out = sh.run(w, x, rows)
    torch.cuda.synchronize()
    gu_k = bf16_floats(np_u16(sh.gu[:rows]))
    act_k = bf16_floats(np_u16(sh.act[:rows]))
    out_k = out.cpu().numpy()
    wg = bf16_floats(np_u16(w.gu_bf16)).astype(np.float64)
    wd = bf16_floats(np_u16(w.down_bf16)).astype(np.float64)
    xf = bf16_floats(np_u16(x)).astype(np.float64)
    for r in sorted({0, rows // 2, rows - 1}):
        gu64 = wg @ xf[r]
        gu_o = torch.from_numpy(gu64.astype(np.float32)).to(torch.bfloat16).float().numpy()
        assert_bf16_ulps(gu_k[r], gu_o, f"rows {rows} row {r} gu")
        assert_bf16_ulps(act_k[r], oracle.shared_swiglu(gu_k[r], N), f"rows {rows} row {r} act", max_frac=0.01)
        want = wd @ act_k[r].astype(np.float64)
        bound = np.abs(wd) @ np.abs(act_k[r]).astype(np.float64) * N * 2.0 ** -23 + 1e-30
        assert np.all(np.abs(out_k[r] - want) <= bound), f"rows {rows} row {r} out"
    slice_form = sh.run(gfr.Fp8SharedWeights(w.gu, w.gu_scale, w.down, w.down_scale), x, rows)
    torch.cuda.synchronize()
    assert_rows_close(out_k, slice_form.cpu().numpy(), rel_rms=1e-2, rel_max=5e-2, what=f"rows {rows} vs slices")


def test_shared_fp8_prefill_form_graph_replays(gfr, sw_prepared):
    """The library GEMMs captured into a graph (their workspace set at create) replay to the eager bytes."""
    rows = 64
    x = torch.randn((rows, D), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda").to(torch.bfloat16)
    sh = gfr.SharedFp8(D, N, rows)
    out = torch.zeros((rows, D), device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        sh.run(sw_prepared, x, rows, out=out, stream=s)
    s.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            sh.run(sw_prepared, x, rows, out=out, stream=s)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_moe_run_fp8_prefill_form(gfr, sw_prepared, routed):
    """A 40-row window of the layer with the bf16 copies: the shared slot gets the prefill form's output, byte-equal
    to gfr_moe_run_shared fed gfr_shared_fp8's."""
    rows = 40
    g = torch.Generator(device="cuda").manual_seed(41)
    x = torch.randn((rows, D), generator=g, device="cuda").to(torch.bfloat16)
    lg = torch.randn((rows, E), generator=g, device="cuda")
    m = gfr.Moe(D, N, E, TOPK, rows, shared_exl3=False)
    m.run_fp8(routed, x, lg, sw_prepared, rows)
    torch.cuda.synchronize()
    got = m.output[:rows].clone()
    shared = gfr.SharedFp8(D, N, rows).run(sw_prepared, x, rows)
    torch.cuda.synchronize()
    assert torch.equal(m.shared_output[:rows], shared)
    m2 = gfr.Moe(D, N, E, TOPK, rows, shared_exl3=False)
    m2.run(routed, x, lg, rows, shared=shared)
    torch.cuda.synchronize()
    assert torch.equal(m2.output[:rows], got)


def test_moe_reference_prefill_window_with_fp8_shared(gfr, oracle, sw_prepared, routed):
    """The reference's own prefill shape (4096 rows, fast_experts.rs:230-286's window size) through the whole layer
    with its FP8 shared expert in the prefill form: sampled tokens (first, middle, last) against the oracle's routed
    rows (the reference's fp16 weights, full-K order) plus the prefill form's shared row (float64 over the bf16
    copies); and a row permutation of the window permutes the outputs bit for bit (rows are independent)."""
    rows = 4096
    g = torch.Generator(device="cuda").manual_seed(4096)
    x = torch.randn((rows, D), generator=g, device="cuda").to(torch.bfloat16)
    lg = torch.randn((rows, E), generator=g, device="cuda")
    m = gfr.Moe(D, N, E, TOPK, rows, shared_exl3=False)
    m.run_fp8(routed, x, lg, sw_prepared, rows)
    torch.cuda.synchronize()
    got = m.output[:rows].clone()
    gp, gw = m.picks[:rows].cpu().numpy(), m.weights[:rows].cpu().numpy()
    dec = DecodedExperts(oracle, routed)
    xb = np_u16(x)
    wg = bf16_floats(np_u16(sw_prepared.gu_bf16)).astype(np.float64)
    wd = bf16_floats(np_u16(sw_prepared.down_bf16)).astype(np.float64)
    for r in (0, rows // 2, rows - 1):
        ys = [dec.row(xb[r], int(e), sk_gu=1, sk_d=1, warps=1)[0] for e in gp[r, :TOPK]]
        gu = torch.from_numpy((wg @ bf16_floats(xb[r]).astype(np.float64)).astype(np.float32))
        gu = gu.to(torch.bfloat16).float().numpy()
        act = oracle.shared_swiglu(gu, N)
        ys.append((wd @ act.astype(np.float64)).astype(np.float32))
        want = oracle.combine(np.stack(ys), gw[r:r + 1], 1, TOPK + 1)[0]
        assert_close(got[r].cpu().numpy(), want, rel_rms=1e-2, rel_max=5e-2, what=f"token {r}")
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(7)).cuda()
    m.run_fp8(routed, x[perm].contiguous(), lg[perm].contiguous(), sw_prepared, rows)
    torch.cuda.synchronize()
    assert torch.equal(m.output[:rows], got[perm])
