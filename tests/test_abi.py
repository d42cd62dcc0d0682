"""The C-ABI library loads and exports every symbol include/gfr_moe.h declares; argument checks run on the host
before any device call (no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gfr_moe.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gfr_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_reference_surface():
    names = declared()
    for must in ["gfr_grouping_create", "gfr_grouping_run", "gfr_experts_run_rows", "gfr_fast_experts_run",
                 "gfr_moe_run", "gfr_exl3_decode_tiles", "gfr_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    import gfr_moe
    lib = ctypes.CDLL(gfr_moe.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_error_string():
    import gfr_moe
    assert b"gfx950" in gfr_moe.lib().gfr_version()


@pytest.mark.parametrize("args,needle", [
    ((0, 9, 16), "grouping experts"), ((289, 0, 16), "grouping slots"), ((289, 33, 16), "grouping slots"),
    ((289, 9, 0), "grouping capacity"),
])
def test_grouping_create_rejects(args, needle):
    import gfr_moe
    h = ctypes.c_void_p()
    rc = gfr_moe.lib().gfr_grouping_create(ctypes.byref(h), *args)
    assert rc == gfr_moe.GFR_EINVAL and not h
    assert needle in gfr_moe.lib().gfr_last_error().decode()


@pytest.mark.parametrize("args,needle", [
    ((2048, 1536, 5, 5, 65), "scratch bound"), ((2048, 1500, 5, 5, 1), "multiples"), ((2048, 1536, 5, 6, 1), "slots"),
])
def test_experts_create_rejects(args, needle):
    import gfr_moe
    h = ctypes.c_void_p()
    rc = gfr_moe.lib().gfr_experts_create(ctypes.byref(h), *args)
    assert rc == gfr_moe.GFR_EINVAL and needle in gfr_moe.lib().gfr_last_error().decode()


def test_run_rejects_null_engine():
    import gfr_moe
    L = gfr_moe.lib()
    assert L.gfr_grouping_run(None, None, None, 1) == gfr_moe.GFR_EINVAL
    assert L.gfr_experts_run_rows(None, None, None, None, 0, None, None, None, None, 1, 1) == gfr_moe.GFR_EINVAL
    assert L.gfr_moe_run(None, None, None, None, None, 1) == gfr_moe.GFR_EINVAL
    assert L.gfr_exl3_decode_tiles(None, None, 16, 16, 4, None) == gfr_moe.GFR_EINVAL


def test_grouped_gemv_rejects_wide_member_stride():
    # an expert's members are read one a lane: more than 64 would be dropped, so the call refuses them
    import ctypes
    import gfr_moe
    L = gfr_moe.lib()
    p = ctypes.c_void_p(16)   # never dereferenced: the arguments are checked first
    rc = L.gfr_exl3_grouped_gemv(None, p, p, p, p, p, p, p, p, 256, 128, 4, 65, 2, 3, 4, 2, 2)
    assert rc == gfr_moe.GFR_EINVAL and "maxm 65" in L.gfr_last_error().decode()


def test_moe_create_rejects():
    import gfr_moe
    h = ctypes.c_void_p()
    L = gfr_moe.lib()
    assert L.gfr_moe_create(ctypes.byref(h), 2048, 1536, 64, 0, 1) == gfr_moe.GFR_EINVAL
    assert L.gfr_moe_create(ctypes.byref(h), 2048, 1536, 64, 65, 1) == gfr_moe.GFR_EINVAL
    assert L.gfr_moe_create(ctypes.byref(h), 2048, 1536, 2000, 4, 1) == gfr_moe.GFR_EINVAL


@pytest.mark.parametrize("stride,ptr_off", [(2044, 0), (2048, 8)])
def test_router_logits_row_alignment(stride, ptr_off):
    """The logits kernel reads input and weight rows 16 bytes at a time: an input stride that is not a multiple of 8
    or an input pointer off 16-byte alignment is refused before any device work."""
    import gfr_moe
    L = gfr_moe.lib()
    x = ctypes.c_void_p(0x10000 + ptr_off)     # never dereferenced on the refused paths
    w = ctypes.c_void_p(0x20000)
    out = ctypes.c_void_p(0x30000)
    rc = L.gfr_router_logits(None, x, stride, w, 2040, 64, 1, out)
    assert rc == gfr_moe.GFR_EINVAL and "16-byte aligned" in L.gfr_last_error().decode()


@pytest.mark.parametrize("args,needle", [((4000, 512, 1), "multiple of 512"), ((4096, 500, 1), "of 64"),
                                         ((4096, 512, 0), "max_rows")])
def test_shared_fp8_create_rejects(args, needle):
    import gfr_moe
    h = ctypes.c_void_p()
    rc = gfr_moe.lib().gfr_shared_fp8_create(ctypes.byref(h), *args)
    assert rc == gfr_moe.GFR_EINVAL and not h and needle in gfr_moe.lib().gfr_last_error().decode()


def test_shared_fp8_run_rejects_null_and_moe_fp8_without_engine():
    import gfr_moe
    L = gfr_moe.lib()
    assert L.gfr_shared_fp8_run(None, None, None, None, 4096, 1, None, 4096) == gfr_moe.GFR_EINVAL
    assert L.gfr_moe_run_fp8(None, None, None, None, None, None, 1) == gfr_moe.GFR_EINVAL
    assert L.gfr_moe_run_router_fp8(None, None, None, None, None, None, 1) == gfr_moe.GFR_EINVAL


def test_fp8_shared_weights_host_checks():
    """Fp8SharedWeights refuses tensors of the wrong shape, dtype or device before any library call (no GPU)."""
    import torch
    import gfr_moe
    H, I = 512, 64
    ok = dict(gu=torch.zeros((2 * I, H), dtype=torch.uint8), gu_scale=torch.zeros(2 * I, dtype=torch.bfloat16),
              down=torch.zeros((H, I), dtype=torch.uint8), down_scale=torch.zeros(H, dtype=torch.bfloat16))
    w = gfr_moe.Fp8SharedWeights(**ok)
    assert w.hidden == H and w.inter == I
    with pytest.raises(ValueError, match="GPU"):          # host tensors
        w.check()
    bad = dict(ok, gu_scale=torch.zeros(2 * I, dtype=torch.float16))
    with pytest.raises(ValueError, match="gu_scale"):
        gfr_moe.Fp8SharedWeights(**bad).check()
    bad = dict(ok, down=torch.zeros((I, H), dtype=torch.uint8))
    with pytest.raises(ValueError, match="down"):
        gfr_moe.Fp8SharedWeights(**bad).check()
    half = gfr_moe.Fp8SharedWeights(**ok, gu_bf16=torch.zeros((2 * I, H), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bf16"):          # one copy without the other
        half.check()


def test_fp8_prepare_and_prepared_lookup_reject():
    import gfr_moe
    L = gfr_moe.lib()
    assert L.gfr_fp8_prepare_bf16(None, None, None, None) == gfr_moe.GFR_EINVAL
    assert L.gfr_prepared_shared_fp8(None, 0, None) != 0
