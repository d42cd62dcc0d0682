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
