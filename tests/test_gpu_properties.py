"""Size-independent properties of the MoE layer at the benchmark's full sizes, bit for bit (no oracle needed):
a row's result depends only on its own input and logits, so permuting the tokens permutes the outputs exactly, and
splitting a window into two windows leaves every row's output unchanged. Checked on the prefill engine at config 4's
8192 tokens, on the split-K programs at config 3's 32-token window and on the decode engine at 4 rows."""
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
