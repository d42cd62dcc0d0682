"""The CPU oracle pinned against the reference's own tests (experts.rs:566-583), independent restatements of the
format (exl3.cu decode_tile's lane form, a big-integer bitstream model), textbook identities and the committed golden
vectors."""
import numpy as np
import pytest
import torch

HAD = np.float32(0.08838834764831845)


def test_had_constant_matches_reference_literal():
    # experts.rs:11 writes 0.088_388_346; exl3.cu:18 writes 0.08838834764831845f: the same fp32
    assert np.float32(0.088388346) == HAD
    assert HAD == np.float32(1 / np.sqrt(128))   # the nearest fp32 to 1/sqrt(128)


def test_codebook_finite(oracle):
    # experts.rs:577-582
    t = oracle.codebook_table().view(np.float16).astype(np.float32)
    assert np.all(np.isfinite(t))


def test_codebook_independent_numpy(oracle):
    # experts.rs:43-46 restated with numpy's IEEE float16 add (round to nearest even)
    s = np.arange(65536, dtype=np.uint64)
    x = ((s * 0xCBAC1FED) & 0xFFFFFFFF) & 0x8FFF8FFF ^ 0x3B603B60
    lo = (x & 0xFFFF).astype(np.uint16).view(np.float16)
    hi = (x >> 16).astype(np.uint16).view(np.float16)
    want = (lo + hi).view(np.uint16)
    assert np.array_equal(oracle.codebook_table(), want)


def test_codebook_sum(oracle):
    # the decode GEMV's weight: the two halves summed without the final fp16 rounding. Independently restated in
    # numpy (float32 add of the two float16 halves), exact (float64 sum agrees), and rounding it to fp16 gives the
    # reference's codebook for every state
    s = np.arange(65536, dtype=np.uint64)
    x = ((s * 0xCBAC1FED) & 0xFFFFFFFF) & 0x8FFF8FFF ^ 0x3B603B60
    lo = (x & 0xFFFF).astype(np.uint16).view(np.float16)
    hi = (x >> 16).astype(np.uint16).view(np.float16)
    got = oracle.codebook_sums()
    assert np.array_equal(got, lo.astype(np.float32) + hi.astype(np.float32))
    assert np.array_equal(got.astype(np.float64), lo.astype(np.float64) + hi.astype(np.float64))
    assert np.array_equal(got.astype(np.float16).view(np.uint16), oracle.codebook_table())
    r16 = oracle.codebook_table().view(np.float16)
    assert np.all(np.abs(got - r16.astype(np.float32)) <= np.abs(got) * 2.0 ** -11)   # fp16's unit roundoff a weight
    # the unrounded unpack places the same values as the rounded one
    rng = np.random.default_rng(5)
    words = rng.integers(0, 2 ** 32, size=(4, 3, 32), dtype=np.uint64).astype(np.uint32)
    a, b = oracle.unpack_f32(words, 64, 48, 4, False), oracle.unpack_f32(words, 64, 48, 4)
    assert np.array_equal(a.astype(np.float16).astype(np.float32), b)


def test_hadamard_involution(oracle):
    # experts.rs:569-576: had(had(x)) == 128 x exactly for x = i - 64
    x = np.arange(128, dtype=np.float32) - 64
    assert np.array_equal(oracle.had(oracle.had(x)), 128 * x)


def test_hadamard_is_sylvester(oracle):
    # the butterflies at strides 1..64 equal multiplication by the Sylvester-ordered Hadamard matrix (fp64, exact
    # on small integers), per 128-block
    H = np.array([[1.0]])
    for _ in range(7):
        H = np.block([[H, H], [H, -H]])
    rng = np.random.default_rng(3)
    x = rng.integers(-50, 50, size=384).astype(np.float32)
    y = oracle.had(x)
    for b in range(3):
        assert np.array_equal(y[128 * b:128 * b + 128], (H @ x[128 * b:128 * b + 128].astype(np.float64)).astype(np.float32))


def test_f16_conversion_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001, 6.1e-5,
                  np.inf, -np.inf], np.float32)])
    L = oracle.lib()
    got = np.array([L.gfro_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))
    h = np.arange(65536, dtype=np.uint16)
    back = np.array([L.gfro_f16_to_f32(int(v)) for v in h[::7]], np.float32)
    ref = h[::7].view(np.float16).astype(np.float32)
    same = (back == ref) | (np.isnan(back) & np.isnan(ref))
    assert same.all()


def test_bf_matches_torch(oracle):
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(5000).astype(np.float32) * 10.0 ** rng.integers(-20, 20, 5000)
    got = np.array([oracle.lib().gfro_bf(float(v)) for v in vals], np.float32)
    want = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, want)


def _decode_tile_lane_form(tile):
    """Independent restatement of exl3.cu:33-40 (decode_tile): lane L of 32 decodes values 8L..8L+7 from words L-1,
    L with a funnel shift, laid out as m16n8k16 B fragments (b0: column g, b1: column g+8; rows 2t,2t+1,2t+8,2t+9)."""
    cb = lambda s: _cb(int(s))
    W = np.zeros((16, 16), np.uint16)
    for lane in range(32):
        w = int(tile[lane])
        p = int(tile[(lane + 31) % 32])
        s = ((p << 32 | w) >> 20) & 0xFFFFFFFF
        b0 = [(cb((s >> 8) & 0xFFFF), cb((s >> 4) & 0xFFFF)), (cb(s & 0xFFFF), cb(w >> 16))]
        b1 = [(cb((w >> 12) & 0xFFFF), cb((w >> 8) & 0xFFFF)), (cb((w >> 4) & 0xFFFF), cb(w & 0xFFFF))]
        g, t = lane // 4, lane % 4
        for half, frag in ((0, b0), (1, b1)):
            col = g + 8 * half
            W[2 * t, col], W[2 * t + 1, col] = frag[0]
            W[2 * t + 8, col], W[2 * t + 9, col] = frag[1]
    return W


_CB = None


def _cb(s):
    global _CB
    if _CB is None:
        import oracle as o
        _CB = o.codebook_table()
    return int(_CB[s])


def _bitstream_form(tile, bits):
    """Big-integer model of the format: the tile's words concatenated MSB-first into one 256*bits-bit circular
    stream; value p is the 16-bit window ending at bit (p+1)*bits; position from experts.rs:65-69."""
    B = 256 * bits
    stream = 0
    for w in tile:
        stream = (stream << 32) | int(w)
    W = np.zeros((16, 16), np.uint16)
    for p in range(256):
        end = ((p + 1) * bits) % B
        # bits [end-16, end) counted from the stream's MSB, circular
        state = 0
        for q in range(16):
            pos = (end - 16 + q) % B
            state = (state << 1) | ((stream >> (B - 1 - pos)) & 1)
        lane, j = p // 8, p % 8
        row = 2 * (lane % 4) + (j & 1) + 8 * ((j >> 1) & 1)
        col = lane // 4 + 8 * (j >> 2)
        W[row, col] = _cb(state)
    return W


def test_unpack_matches_decode_tile_lane_form(oracle):
    rng = np.random.default_rng(7)
    tiles = [rng.integers(0, 2 ** 32, 32, dtype=np.uint64).astype(np.uint32) for _ in range(6)]
    tiles += [np.zeros(32, np.uint32), np.full(32, 0xFFFFFFFF, np.uint32)]
    for b in (0, 5, 17, 31, 400, 1023):  # single-bit tiles
        t = np.zeros(32, np.uint32)
        t[b // 32] = np.uint32(1 << (31 - b % 32))
        tiles.append(t)
    for t in tiles:
        assert np.array_equal(oracle.unpack(t.reshape(1, 1, 32), 16, 16, 4), _decode_tile_lane_form(t))


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_unpack_matches_bitstream_model(oracle, bits):
    rng = np.random.default_rng(100 + bits)
    TW = 8 * bits
    words = rng.integers(0, 2 ** 32, (2, 3, TW), dtype=np.uint64).astype(np.uint32)   # 2x3 tiles: kin 32, n 48
    got = oracle.unpack(words, 32, 48, bits)
    for kt in range(2):
        for nt in range(3):
            assert np.array_equal(got[16 * kt:16 * kt + 16, 16 * nt:16 * nt + 16], _bitstream_form(words[kt, nt], bits))


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_single_bit_reaches_exactly_its_windows(oracle, bits):
    # flipping bit b of the stream changes exactly the values whose 16-bit window covers b (16 / bits of them)
    B = 256 * bits
    base = np.zeros((1, 1, 8 * bits), np.uint32)
    ref = oracle.unpack(base, 16, 16, bits)
    for b in (0, 1, 31, 32, B // 2 + 3, B - 1):
        t = base.copy()
        t[0, 0, b // 32] ^= np.uint32(1 << (31 - b % 32))
        changed = set()
        got = oracle.unpack(t, 16, 16, bits)
        for p in range(256):
            lane, j = p // 8, p % 8
            row = 2 * (lane % 4) + (j & 1) + 8 * ((j >> 1) & 1)
            col = lane // 4 + 8 * (j >> 2)
            end = ((p + 1) * bits) % B
            if (b - (end - 16)) % B < 16:
                changed.add((row, col))
        diff = {(int(r), int(c)) for r, c in zip(*np.nonzero(got != ref))}
        assert diff <= changed      # a state change may map to the same codebook value, never the reverse
        assert len(changed) == (16 + bits - 1) // bits or len(changed) == 16 // bits


def test_matmul_order_and_value(oracle):
    rng = np.random.default_rng(2)
    k, n = 256, 48
    x = rng.standard_normal(k).astype(np.float32)
    w = rng.standard_normal((k, n)).astype(np.float32)
    y = oracle.matmul(x, w, 4, 4)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.astype(np.float64), rtol=1e-4, atol=1e-4)
    # sk = warps = 1 is the plain ascending fp32 sum
    seq = np.zeros(n, np.float32)
    for j in range(k):
        seq = (seq + x[j] * w[j]).astype(np.float32)
    assert np.array_equal(oracle.matmul(x, w, 1, 1), seq)
    # the reference's order: 16 ranges of 16, summed warp by warp then split by split
    ranges = [np.float32(0)] * 0
    want = np.zeros(n, np.float32)
    for split in range(4):
        part = None
        for wp in range(4):
            a = np.zeros(n, np.float32)
            for j in range((split * 4 + wp) * 16, (split * 4 + wp) * 16 + 16):
                a = (a + x[j] * w[j]).astype(np.float32)
            part = a if part is None else (part + a).astype(np.float32)
        want = (want + part).astype(np.float32)
    assert np.array_equal(y, want)


def _xorshift_cases(capacity, row_counts, E=289, slots=9):
    """grouping.rs:139-160: xorshift64 from 0x0123456789abcdef, concentrated or spread (start + slot*37) % 288."""
    seed = 0x0123456789ABCDEF
    M = (1 << 64) - 1
    for rows in row_counts:
        for concentrated in (True, False):
            picks = []
            for r in range(rows):
                seed ^= (seed << 13) & M
                seed ^= seed >> 7
                seed ^= (seed << 17) & M
                start = 0 if concentrated else seed % 288
                picks.append([(288 if s == 8 else (start + s * 37) % 288) for s in range(slots)])
            yield rows, concentrated, np.array(picks, np.int32).reshape(rows, slots)


def _group_bruteforce(picks, E, maxm):
    rows, slots = picks.shape
    lists = {e: [] for e in range(E)}
    for r in range(rows):
        seen = set()
        for s in range(slots):
            e = int(picks[r, s])
            if e not in seen:
                seen.add(e)
                lists[e].append(r * 32 + s)
    ids = [e for e in range(E) if lists[e]]
    members = np.full((E, maxm), -1, np.int32)
    for u, e in enumerate(ids):
        members[u, :len(lists[e])] = lists[e]
    return len(ids), np.array(ids, np.int32), members


def test_group_reference_cases(oracle):
    for rows, conc, picks in _xorshift_cases(64, [1, 2, 31, 32, 33, 63, 64]):
        c, ids, mem = oracle.group(picks, rows, 9, 289, 64)
        c2, ids2, mem2 = _group_bruteforce(picks, 289, 64)
        assert c == c2 and np.array_equal(ids, ids2) and np.array_equal(mem, mem2), (rows, conc)


def test_group_duplicates_first_slot(oracle):
    picks = np.array([[3, 3, 5], [5, 1, 5]], np.int32)
    c, ids, mem = oracle.group(picks, 2, 3, 8, 4)
    assert c == 3 and list(ids) == [1, 3, 5]
    assert list(mem[0]) == [33, -1, -1, -1] and list(mem[1]) == [0, -1, -1, -1] and list(mem[2]) == [2, 32, -1, -1]


def test_route(oracle):
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((50, 64)).astype(np.float32)
    picks, w = oracle.route(logits, 4, 64)
    for r in range(50):
        order = np.argsort(-logits[r], kind="stable")[:4]
        assert list(picks[r, :4]) == list(order) and picks[r, 4] == 64
        p = np.exp(logits[r].astype(np.float64) - logits[r].max())
        p /= p.sum()
        np.testing.assert_allclose(w[r, :4], p[order] / p[order].sum(), rtol=1e-6)
        assert w[r, 4] == 1.0


def _biased_reference(logits, bias, k, scale):
    """An independent numpy restatement of the published GLM / DeepSeek-V3 gate."""
    s = (1.0 / (1.0 + np.exp(-logits.astype(np.float32)))).astype(np.float32)
    choice = (s + bias.astype(np.float32)).astype(np.float32)
    order = np.argsort(-choice, kind="stable")
    pk = order[:k]
    w = s[pk] / (s[pk].sum(dtype=np.float32) + np.float32(1e-20)) * np.float32(scale)
    gap = choice[order[k - 1]] - choice[order[k]] if k < len(order) else np.inf
    return pk, w, gap


@pytest.mark.parametrize("E,k", [(64, 4), (160, 8), (288, 8)])
def test_route_biased(oracle, E, k):
    rng = np.random.default_rng(E + k)
    logits = rng.standard_normal((40, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    picks, w = oracle.route_biased(logits, bias, 2.5, k, E)
    for r in range(40):
        pk, wr, gap = _biased_reference(logits[r], bias, k, 2.5)
        if gap > 1e-6:                      # a near-tie at the k-th place may round either way
            assert list(picks[r, :k]) == list(pk)
            np.testing.assert_allclose(w[r, :k], wr, rtol=1e-6)
        assert picks[r, k] == E and w[r, k] == 1.0
        np.testing.assert_allclose(w[r, :k].sum(), 2.5, rtol=1e-6)


def _swiglu_limited(g, u, limit=10.0):
    g = np.minimum(g, limit)
    u = np.clip(u, -limit, limit)
    return g / (1 + np.exp(-g)) * u


def test_expert_row_vs_float64(oracle):
    # experts.rs:113-146 composed in float64 without the fp16 / bf16 roundings: agreement to rounding level
    rng = np.random.default_rng(9)
    D, N, bits = 256, 256, 4
    wg = oracle.unpack_f32(rng.integers(0, 2 ** 32, (D // 16, N // 16, 32), dtype=np.uint64).astype(np.uint32), D, N, 4)
    wu = oracle.unpack_f32(rng.integers(0, 2 ** 32, (D // 16, N // 16, 32), dtype=np.uint64).astype(np.uint32), D, N, 4)
    wd = oracle.unpack_f32(rng.integers(0, 2 ** 32, (N // 16, D // 16, 32), dtype=np.uint64).astype(np.uint32), N, D, 4)
    sc = lambda n: ((rng.integers(0, 2, n) * 2 - 1) * (rng.random(n) + 0.5)).astype(np.float16)
    suh_g, suh_u, svh_d = sc(D), sc(D), sc(D)
    suh_d, svh_g, svh_u = sc(N), sc(N), sc(N)
    x = torch.randn(D, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    xf = x.float().numpy().astype(np.float64)
    y, xd = oracle.expert_row(xb, wg, wu, wd, *(a.view(np.uint16) for a in (suh_g, suh_u, suh_d, svh_g, svh_u, svh_d)))
    H = np.array([[1.0]])
    for _ in range(7):
        H = np.block([[H, H], [H, -H]])
    Hb = lambda v: np.concatenate([H @ v[i:i + 128] for i in range(0, len(v), 128)]) / np.sqrt(128)
    f = lambda a: a.astype(np.float64)
    g = Hb(Hb(xf * f(suh_g)) @ f(wg)) * f(svh_g)
    u = Hb(Hb(xf * f(suh_u)) @ f(wu)) * f(svh_u)
    a = _swiglu_limited(g, u)
    want = Hb(Hb(a * f(suh_d)) @ f(wd)) * f(svh_d)
    err = np.sqrt(np.mean((y - want) ** 2) / np.mean(want ** 2))
    assert err < 2e-2, err     # bf16 roundings of the epilogue dominate


def test_combine(oracle):
    rng = np.random.default_rng(4)
    y = rng.standard_normal((3 * 5, 32)).astype(np.float32)
    w = rng.random((3, 5)).astype(np.float32)
    out = oracle.combine(y, w, 3, 5)
    np.testing.assert_allclose(out, np.einsum("rs,rsn->rn", w, y.reshape(3, 5, 32)), rtol=1e-6, atol=1e-6)


def test_linear_vs_float64(oracle):
    """gfro_linear (config 1's checker: rot_in on an fp16 token, one GEMV, the down epilogue, exl3.cu:224-241 and
    :300-321) against the same composition in float64 with the dense Sylvester Hadamard of each 128-block. The only
    rounding of the oracle, fp16 of the rotated activations, is applied at the same point, so the two agree to fp32
    accumulation error; a kin != n shape catches a transposed weight, and a dropped scale, 1/sqrt(128) or block
    transform fails by orders of magnitude."""
    rng = np.random.default_rng(21)
    H = np.array([[1.0]])
    for _ in range(7):
        H = np.block([[H, H], [H, -H]])
    Hb = lambda v: np.concatenate([H @ v[i:i + 128] for i in range(0, len(v), 128)]) / np.sqrt(128)
    for kin, n in ((384, 256), (2048, 1536)):
        words = rng.integers(0, 2 ** 32, (kin // 16, n // 16, 32), dtype=np.uint64).astype(np.uint32)
        w = oracle.unpack_f32(words, kin, n, 4)
        sc = lambda m: ((rng.integers(0, 2, m) * 2 - 1) * (rng.random(m) + 0.5)).astype(np.float16)
        suh, svh = sc(kin), sc(n)
        x = rng.standard_normal(kin).astype(np.float16)
        y = oracle.linear(x.view(np.uint16), w, suh.view(np.uint16), svh.view(np.uint16))
        xh = Hb(x.astype(np.float64) * suh.astype(np.float64)).astype(np.float16).astype(np.float64)
        want = Hb(xh @ w.astype(np.float64)) * svh.astype(np.float64)
        err = np.sqrt(np.mean((y - want) ** 2) / np.mean(want ** 2))
        assert err < 5e-5, (kin, n, err)
        # the same without the fp16 rounding of the activations: within fp16 rounding of the result
        want_exact = Hb(Hb(x.astype(np.float64) * suh.astype(np.float64)) @ w.astype(np.float64)) * svh.astype(np.float64)
        err2 = np.sqrt(np.mean((y - want_exact) ** 2) / np.mean(want_exact ** 2))
        assert err2 < 2e-3, (kin, n, err2)


def test_row_batches_are_loops_of_the_row_functions(oracle):
    """gfro_rot_rows / gfro_gateup_epilogue_rows / gfro_down_epilogue_rows equal the single-row functions, bit for
    bit, row by row (including a repeated and an out-of-order row index)."""
    rng = np.random.default_rng(21)
    D, N = 384, 256
    x = (rng.standard_normal((6, D)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    suh = ((rng.integers(0, 2, D) * 2 - 1) * (rng.random(D) + 0.5)).astype(np.float16).view(np.uint16)
    rows = np.array([4, 0, 4, 2], np.int32)
    got = oracle.rot_rows(x, rows, suh)
    for i, r in enumerate(rows):
        assert np.array_equal(got[i], oracle.rot(x[r], suh))
    sc = lambda n: ((rng.integers(0, 2, n) * 2 - 1) * (rng.random(n) + 0.5)).astype(np.float16).view(np.uint16)
    svh_g, svh_u, suh_d, svh_d = sc(N), sc(N), sc(N), sc(D)
    g = rng.standard_normal((3, N)).astype(np.float32) * 4
    u = rng.standard_normal((3, N)).astype(np.float32) * 4
    xd = oracle.gateup_epilogue_rows(g, u, svh_g, svh_u, suh_d)
    z = rng.standard_normal((3, D)).astype(np.float32)
    y = oracle.down_epilogue_rows(z, svh_d)
    L = oracle.lib()
    for r in range(3):
        gg, uu, one = g[r].copy(), u[r].copy(), np.empty(N, np.uint16)
        L.gfro_gateup_epilogue(gg.ctypes.data, uu.ctypes.data, svh_g.ctypes.data, svh_u.ctypes.data, suh_d.ctypes.data,
                               N, 10.0, one.ctypes.data)
        assert np.array_equal(xd[r], one)
        zz, yy = z[r].copy(), np.empty(D, np.float32)
        L.gfro_down_epilogue(zz.ctypes.data, svh_d.ctypes.data, D, yy.ctypes.data)
        assert np.array_equal(y[r], yy)


def test_window_reference_matches_expert_row(oracle):
    """The whole-window checker of the GPU tests (refs.window_reference: per-expert fp32 GEMMs of the oracle's decoded
    fp16 weights around the oracle's rotation and epilogues) against gfro_expert_row on every (row, slot), with a
    non-EXL3 slot left NaN."""
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "glm-flash-rs_amd"))
    import synth
    from refs import DecodedExperts, assert_rows_close, window_reference
    E, D, N, bits, rows = 4, 256, 256, 3, 5
    w = synth.experts(E, D, N, bits, seed=3, device="cpu")
    x = synth.activations(rows, D, 4, device="cpu")
    picks = np.array([[0, 2, 4], [1, 3, 4], [3, 0, 4], [2, 2, 4], [1, 0, 4]], np.int32)   # id 4: not EXL3
    y = window_reference(oracle, w, x, picks, workers=2)
    assert np.all(np.isnan(y[:, 2]))
    dec = DecodedExperts(oracle, w)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    want = np.stack([np.stack([dec.row(xb[r], int(picks[r, s]), sk_gu=1, sk_d=1, warps=1)[0] for s in range(2)])
                     for r in range(rows)])
    assert_rows_close(y[:, :2], want, what="window reference")


# ---- the FP8 shared expert (moe.rs:132-167) ----------------------------------------------------------------------
def test_fp8_values_reference_cases_and_torch(oracle):
    """front.rs:716-722 known answers, and every non-NaN e4m3 byte against torch's float8_e4m3fn conversion (an
    independent decoder); the NaN codes 0x7f / 0xff decode to +-480 as front.rs:173-182 computes them."""
    v = oracle.fp8_values()
    assert v[0x38] == 1.0 and v[0xB8] == -1.0 and v[0x7E] == 448.0 and v[0x01] == 1.0 / 512.0
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(v[codes], want)
    assert v[0x7F] == 480.0 and v[0xFF] == -480.0


@pytest.mark.parametrize("sk", [1, 8])
def test_fp8_matmul_vs_float64(oracle, sk):
    """reference_mm_at (front.rs:190-217) within fp32 accumulation error of the float64 product, every output row,
    with and without the bf16 rounding; a transposed operand, a dropped slice or a wrong scale index fails it."""
    rng = np.random.default_rng(5 + sk)
    n, k = 48, 1024
    w = rng.integers(0, 256, (n, k), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x38
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(torch.bfloat16).float().numpy()
    sc = torch.from_numpy((rng.random(n) + 0.5).astype(np.float32) / 64).to(torch.bfloat16)
    s64 = sc.float().numpy().astype(np.float64)
    wv = oracle.fp8_values().astype(np.float64)[w]
    y64 = (wv @ x.astype(np.float64)) * s64
    bound = (np.abs(wv) @ np.abs(x).astype(np.float64)) * s64 * k * 2.0 ** -23
    y = oracle.fp8_matmul(x, w, sc.view(torch.int16).numpy().view(np.uint16), sk, False)
    assert np.all(np.abs(y - y64) <= bound), np.max(np.abs(y - y64) / bound)
    yr = oracle.fp8_matmul(x, w, sc.view(torch.int16).numpy().view(np.uint16), sk, True)
    np.testing.assert_array_equal(yr, torch.from_numpy(y).to(torch.bfloat16).float().numpy())


def test_fp8_matmul_exact_slices(oracle):
    """Integer weights and activations with a power-of-two scale: every product and partial sum is exact in fp32, so
    the slice sums, the scale and the ordered sum of slices must reproduce the float64 result bit for bit."""
    rng = np.random.default_rng(11)
    n, k, sk = 16, 512, 8
    codes = np.array([0x38, 0x40, 0x44, 0x48, 0xB8, 0xC0, 0x00], np.uint8)   # 1, 2, 3, 4, -1, -2, 0
    w = codes[rng.integers(0, len(codes), (n, k))]
    x = rng.integers(-3, 4, k).astype(np.float32)
    sc = np.full(n, 0x3E80, np.uint16)                                        # bf16 0.25
    y = oracle.fp8_matmul(x, w, sc, sk, False)
    wv = oracle.fp8_values().astype(np.float64)[w]
    np.testing.assert_array_equal(y, ((wv @ x.astype(np.float64)) * 0.25).astype(np.float32))


def test_shared_swiglu_closed_form(oracle):
    """front.rs:669-675: act = bf16(bf16(silu(min(g, 10))) * clamp(u, -10, 10)) against the float64 formula to one
    bf16 rounding, including gate values above the limit and up values beyond +-limit."""
    inter = 64
    g = np.concatenate([np.linspace(-12, 12, 48), [10.0, 10.5, 30.0, -30.0] * 4]).astype(np.float32)
    u = np.concatenate([np.linspace(-14, 14, 48), [15.0, -15.0, 9.5, -9.75] * 4]).astype(np.float32)
    act = oracle.shared_swiglu(np.concatenate([g, u]), inter)
    gg = np.minimum(g.astype(np.float64), 10.0)
    uu = np.clip(u.astype(np.float64), -10.0, 10.0)
    want = gg / (1 + np.exp(-gg)) * uu
    np.testing.assert_allclose(act, want, rtol=2 * 2.0 ** -8, atol=1e-30)
    # above the limit the gate saturates at silu(10): g = 10.5 and g = 30 give the act of g = 10
    np.testing.assert_array_equal(oracle.shared_swiglu(np.array([10.0, 30.0, 2.0, 2.0], np.float32), 2),
                                  oracle.shared_swiglu(np.array([10.0, 10.0, 2.0, 2.0], np.float32), 2))


def test_fp8_b16_copy_vs_torch(oracle):
    """prefill.cu:7-17 (the prefill form's weight copies): bf16_rn(fp8 * row scale) against torch's float8_e4m3fn
    decode, an fp32 product and torch's bf16 rounding, every non-NaN byte value times several scales; the NaN codes
    stay NaN."""
    codes = np.arange(256, dtype=np.uint8)
    scales = torch.tensor([1.0, 0.3, -2.5, 1e-3, 3.1e4], dtype=torch.bfloat16)
    w = np.tile(codes, (len(scales), 1))
    got = oracle.fp8_b16_copy(w, scales.view(torch.int16).numpy().view(np.uint16))
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    want = (vals[None, :] * scales.float()[:, None]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ok = (codes & 0x7F) != 0x7F
    np.testing.assert_array_equal(got[:, ok], want[:, ok])
    gotf = (got.astype(np.uint32) << 16).view(np.float32)
    assert np.all(np.isnan(gotf[:, ~ok]))
