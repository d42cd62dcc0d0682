"""Host-side references for the GPU tests: synthetic tensors copied to numpy and pushed through the CPU oracle."""
import numpy as np
import torch


def np_u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def np_u32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


class DecodedExperts:
    """Decodes (and caches) experts of an Exl3Experts through the oracle. rounded: the reference's fp16 weights;
    otherwise the unrounded sums of the two codebook halves that the decode GEMV multiplies (gfro_codebook_sum)."""

    def __init__(self, oracle, w, rounded=True):
        self.o, self.w, self.rounded = oracle, w, rounded
        self.cache = {}
        self.vec = {n: np_u16(getattr(w, n)) for n in ("suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")}

    def mats(self, e):
        if e not in self.cache:
            w, D, N, b = self.w, self.w.hidden, self.w.inter, self.w.bits
            r = self.rounded
            self.cache[e] = (self.o.unpack_f32(np_u32(w.gt[e]), D, N, b, r), self.o.unpack_f32(np_u32(w.ut[e]), D, N, b, r),
                             self.o.unpack_f32(np_u32(w.dt[e]), N, D, b, r))
        return self.cache[e]

    def row(self, x_bf16_u16, e, sk_gu=4, sk_d=1, warps=4):
        wg, wu, wd = self.mats(e)
        v = self.vec
        return self.o.expert_row(x_bf16_u16, wg, wu, wd, v["suh_g"][e], v["suh_u"][e], v["suh_d"][e], v["svh_g"][e],
                                 v["svh_u"][e], v["svh_d"][e], sk_gu, sk_d, warps)


# The north star's bar for a layer's outputs against the reference's arithmetic: 1e-2 relative.
NORTH_STAR_REL = 1e-2


def assert_close(got, want, rel_rms=1e-3, rel_max=1e-2, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = got - want
    rms = np.sqrt(np.mean(err ** 2) / max(np.mean(want ** 2), 1e-30))
    mx = np.max(np.abs(err)) / max(np.max(np.abs(want)), 1e-30)
    assert rms < rel_rms and mx < rel_max, f"{what}: relative RMS {rms:.3g}, max {mx:.3g}"
    return rms, mx


def assert_decode_close(got, want_gemv, want_ref, what=""):
    """A decode-GEMV result against the oracle with the GEMV's own weights (unrounded codebook sums, fp32 order of the
    kernels: the tight bar) and against the reference's fp16 weights (the north star's 1e-2)."""
    assert_close(got, want_gemv, what=what)
    return assert_close(got, want_ref, rel_rms=NORTH_STAR_REL, rel_max=NORTH_STAR_REL, what=what + " vs reference weights")


def window_reference(oracle, w, x, picks, exl3_slots=None, workers=8):
    """Every EXL3 (row, slot) output y [rows][slots][D] fp32 of a window (NaN where a slot's expert is not EXL3), for
    whole-window checks. Per used expert: its trellis decoded once to the reference's fp16 weights (gfro_unpack_f32),
    the rows rotated by gfro_rot (rot_in), the two GEMMs as fp32 products of those fp16 values (torch on the CPU:
    every product exact, only the fp32 summation order differs from the oracle's fixed order), and the gate/up and
    down epilogues by the oracle's own functions, row by row."""
    from concurrent.futures import ThreadPoolExecutor
    xb = np_u16(x)
    picks = np.asarray(picks)
    rows, slots = picks.shape
    S = slots if exl3_slots is None else exl3_slots
    D, N, bits, E = w.hidden, w.inter, w.bits, int(w.gt.shape[0])
    vec = {n: np_u16(getattr(w, n)) for n in ("suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")}
    by_e = {}
    for r in range(rows):
        for s in range(S):
            e = int(picks[r, s])
            if 0 <= e < E:
                by_e.setdefault(e, []).append((r, s))
    words = {e: (np_u32(w.gt[e]), np_u32(w.ut[e]), np_u32(w.dt[e])) for e in by_e}
    y = np.full((rows, slots, D), np.nan, np.float32)

    def f16(a):
        return torch.from_numpy(a.view(np.float16).astype(np.float32))

    def work(e):
        lst = by_e[e]
        rr = np.array([r for r, _ in lst], np.int32)
        gt, ut, dt = words[e]
        wg = torch.from_numpy(oracle.unpack_f32(gt, D, N, bits))
        wu = torch.from_numpy(oracle.unpack_f32(ut, D, N, bits))
        wd = torch.from_numpy(oracle.unpack_f32(dt, N, D, bits))
        g = f16(oracle.rot_rows(xb, rr, vec["suh_g"][e])) @ wg
        u = f16(oracle.rot_rows(xb, rr, vec["suh_u"][e])) @ wu
        xd = oracle.gateup_epilogue_rows(g.numpy(), u.numpy(), vec["svh_g"][e], vec["svh_u"][e], vec["suh_d"][e])
        z = f16(xd) @ wd
        yy = oracle.down_epilogue_rows(z.numpy(), vec["svh_d"][e])
        for i, (r, s) in enumerate(lst):
            y[r, s] = yy[i]

    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(work, sorted(by_e)))
    return y


def assert_rows_close(got, want, rel_rms=1e-3, rel_max=1e-2, what=""):
    """Every row of got [rows][n] against want: each row's relative RMS error below rel_rms, and the whole array's
    maximum error below rel_max of its largest value."""
    got = np.asarray(got, np.float64).reshape(-1, np.shape(got)[-1])
    want = np.asarray(want, np.float64).reshape(got.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert np.all(np.isfinite(want)), f"{what}: non-finite reference"
    err = got - want
    rms = np.sqrt(np.mean(err ** 2, axis=1) / np.maximum(np.mean(want ** 2, axis=1), 1e-30))
    worst = int(np.argmax(rms))
    mx = np.max(np.abs(err)) / max(np.max(np.abs(want)), 1e-30)
    assert rms[worst] < rel_rms and mx < rel_max, \
        f"{what}: worst row {worst} relative RMS {rms[worst]:.3g} (median {np.median(rms):.3g}), max {mx:.3g}"
    return float(rms[worst]), float(mx)
