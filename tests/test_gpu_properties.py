"""Size-independent properties of the MoE layer at the benchmark's full sizes, bit for bit (no oracle needed):
a row's result depends only on its own input and logits, so permuting the tokens permutes the outputs exactly, and
splitting a window into two windows leaves every row's output unchanged. Checked on the prefill engine at config 4's
8192 tokens, on the split-K programs at config 3's 32-token window and on the decode engine at 4 rows, and at config 5's
shape for every bit width on all three engine paths."""
import pytest
import torch

pytestmark = pytest.mark.gpu

D, N, BITS, E, TOPK = 2048, 1536, 4, 64, 4


@pytest.fixture(scope="module")
def layer():
    import synth
    w = synth.experts(E + 1, D, N, BITS, seed=611)
    x = synth.activations(8192, D, 612)
    lg = synth.logits(8192, E, 613)
    return w, x, lg


def _run(gfr, w, x, lg, rows):
    m = gfr.Moe(D, N, E, TOPK, rows)
    m.run(w, x.contiguous(), lg.contiguous(), rows)
    torch.cuda.synchronize()
    return m.output[:rows].clone(), m.picks[:rows].clone()


@pytest.mark.parametrize("rows", [4, 32, 8192])
def test_token_permutation_permutes_the_outputs(gfr, layer, rows):
    w, x, lg = layer
    x, lg = x[:rows], lg[:rows]
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(rows)).cuda()
    out, picks = _run(gfr, w, x, lg, rows)
    out_p, picks_p = _run(gfr, w, x[perm], lg[perm], rows)
    assert torch.isfinite(out).all()
    assert torch.equal(picks_p, picks[perm])
    diff = (out_p != out[perm]).any(dim=1).nonzero().flatten().tolist()
    assert not diff, f"{len(diff)} of {rows} rows differ after permuting the tokens, first {diff[:5]}"


@pytest.mark.parametrize("rows,cut", [(8192, 4096), (8192, 1000), (32, 12)])
def test_split_windows_equal_the_whole(gfr, layer, rows, cut):
    """Each part runs on the same engine as the whole (8192 / 4096 / 1000 / 7192 rows: full-K items; 32 / 12 / 20
    rows: split-K programs) but with other item plans and other neighbours in its items."""
    w, x, lg = layer
    whole, _ = _run(gfr, w, x[:rows], lg[:rows], rows)
    a, _ = _run(gfr, w, x[:cut], lg[:cut], cut)
    b, _ = _run(gfr, w, x[cut:rows], lg[cut:rows], rows - cut)
    parts = torch.cat([a, b])
    diff = (parts != whole).any(dim=1).nonzero().flatten().tolist()
    assert not diff, f"{len(diff)} of {rows} rows differ between the split and the whole window, first {diff[:5]}"


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("rows", [3, 100, 600])
def test_token_permutation_config5_widths(gfr, bits, rows):
    """Config 5's layer shape (hidden 5120, 160 + 1 experts, top-8) at every bit width, on the decode engine (3 rows),
    the split-K programs (100 rows, 900 pairs) and full-K items (600 rows)."""
    import synth
    D5, N5, E5, K5 = 5120, 1536, 160, 8
    w = synth.experts(E5 + 1, D5, N5, bits, seed=620 + bits)
    x = synth.activations(rows, D5, 621)
    lg = synth.zipf_logits(rows, E5, K5, 1.1, 622)
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(rows + bits)).cuda()
    outs = []
    for xi, li in ((x, lg), (x[perm].contiguous(), lg[perm].contiguous())):
        m = gfr.Moe(D5, N5, E5, K5, rows)
        m.run(w, xi, li, rows)
        torch.cuda.synchronize()
        outs.append(m.output[:rows].clone())
    assert torch.isfinite(outs[0]).all()
    diff = (outs[1] != outs[0][perm]).any(dim=1).nonzero().flatten().tolist()
    assert not diff, f"{len(diff)} of {rows} rows differ after permuting the tokens, first {diff[:5]}"
