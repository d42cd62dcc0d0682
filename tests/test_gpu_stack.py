"""Config 5's 4-layer stack chained (hidden 5120, 160 routed + 1 shared EXL3 experts, top-8, inter 1536, K = 2, 3, 4,
5 a layer): each layer's output, RMS-normalised per row and rounded to bf16, is the next layer's input, and its router
logits come from that input (gfr_router_logits against a seeded bf16 router weight), as in a model's forward pass
(the MoE block's input is the normed hidden state). Every layer's routing is checked exactly and its outputs against
the oracle's whole-window reference on the same input. (The stack as a whole is not compared with the oracle run as
a stack, its own outputs fed forward: over four layers the two chains' inputs drift apart by each layer's rounding
differences, which the next layers amplify -- 13 % after four layers at bs = 1 -- so only per-layer agreement pins
anything.)

Without the norm the synthetic layers' outputs grow to thousands, nearly every gate and up value sits at the SwiGLU
limit, and a one-ulp bf16 difference in a single activation moves its whole 128-value block after the transform: the
oracle itself then differs by 4.5 % between the reference's fp16 weights and the unrounded codebook sums on 2 of 9
experts of such a layer (measured on the CPU)."""
import numpy as np
import pytest
import torch

from refs import NORTH_STAR_REL, assert_rows_close, window_reference

pytestmark = pytest.mark.gpu

E, D, N, TOPK = 160, 5120, 1536, 8


@pytest.fixture(scope="module")
def stack():
    import synth
    layers = [synth.experts(E + 1, D, N, b, seed=500 + 10 * b) for b in (2, 3, 4, 5)]
    g = torch.Generator(device="cuda").manual_seed(5)
    routers = [(torch.randn((E, D), generator=g, device="cuda") * 0.05).to(torch.bfloat16) for _ in layers]
    return layers, routers


def _normed(out):
    """The next layer's input: each row over its RMS (the pre-MoE RMSNorm without its weight), in bf16."""
    out = out.float()
    return (out * torch.rsqrt((out * out).mean(dim=1, keepdim=True) + 1e-6)).to(torch.bfloat16)


def _layer_ref(oracle, w, x, logits):
    p, wt = oracle.route(logits.cpu().numpy(), TOPK, E)
    y = window_reference(oracle, w, x, p, workers=16)
    return p, oracle.combine(y, wt, x.shape[0], TOPK + 1)


@pytest.mark.parametrize("rows", [1, 64, 300])
def test_config5_stack_chained(gfr, oracle, stack, rows):
    """rows 1: the bs = 1 launches (decode GEMV: against the reference's fp16 weights at the north star's 1e-2);
    64: the split-K prefill programs; 300 (2700 pairs): full-K prefill items (both at the 1e-3 bar)."""
    import synth
    layers, routers = stack
    m = gfr.Moe(D, N, E, TOPK, rows)
    x = synth.activations(rows, D, 900 + rows)
    bar = NORTH_STAR_REL if rows == 1 else 1e-3
    for li, (w, rw) in enumerate(zip(layers, routers)):
        lg = gfr.router_logits(x, rw)
        m.run(w, x, lg, rows)
        torch.cuda.synchronize()
        out = m.output[:rows].cpu().numpy()
        p, want = _layer_ref(oracle, w, x, lg)
        assert np.array_equal(m.picks[:rows].cpu().numpy(), p), f"layer {li}: routing"
        assert_rows_close(out, want, rel_rms=bar, rel_max=max(bar, 1e-2), what=f"rows {rows} layer {li} (K={w.bits})")
        x = _normed(m.output[:rows])
