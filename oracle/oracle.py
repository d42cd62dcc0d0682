"""ctypes binding of the CPU oracle (oracle/libgfr_oracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the checker (or the
timed CPU baseline); the product path never does. Arrays are numpy; fp16 / bf16 values travel as uint16 bits.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgfr_oracle.so")


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    I = ctypes.c_int
    F = ctypes.c_float
    sigs = {
        "gfro_f32_to_f16": ([F], ctypes.c_uint16), "gfro_f16_to_f32": ([ctypes.c_uint16], F),
        "gfro_bf": ([F], F), "gfro_hf": ([F], F), "gfro_codebook": ([ctypes.c_uint32], ctypes.c_uint16),
        "gfro_codebook_table": ([P], None), "gfro_state": ([P, I, I], ctypes.c_uint32),
        "gfro_unpack": ([P, I, I, I, P], None), "gfro_unpack_f32": ([P, I, I, I, P], None),
        "gfro_unpack_f32_sum": ([P, I, I, I, P], None), "gfro_codebook_sum": ([ctypes.c_uint32], F),
        "gfro_had": ([P, ctypes.c_long], None), "gfro_matmul": ([P, P, I, I, I, I, P], None),
        "gfro_rot": ([P, P, I, P], None),
        "gfro_gateup_epilogue": ([P, P, P, P, P, I, F, P], None), "gfro_down_epilogue": ([P, P, I, P], None),
        "gfro_rot_rows": ([P, ctypes.c_long, P, I, P, I, P], None),
        "gfro_gateup_epilogue_rows": ([P, P, P, P, P, I, I, F, P], None), "gfro_down_epilogue_rows": ([P, P, I, I, P], None),
        "gfro_expert_row": ([P, I, I, P, P, P, P, P, P, P, P, P, I, I, I, F, P, P], None),
        "gfro_linear": ([P, I, I, P, P, P, P], None),
        "gfro_group": ([P, I, I, I, I, P, P, P], I), "gfro_route": ([P, I, I, I, I, P, P], None),
        "gfro_route_biased": ([P, P, ctypes.c_float, I, I, I, I, P, P], None),
        "gfro_combine": ([P, P, I, I, I, P], None),
        "gfro_fp8": ([ctypes.c_uint8], F), "gfro_fp8_matmul": ([P, P, P, I, I, I, I, P], None),
        "gfro_shared_swiglu": ([P, I, F, P], None), "gfro_fp8_b16_copy": ([P, P, I, I, P], None),
        "gfro_baseline_decode": ([P, I, I, I, I, P, P, P, P, P, P, P, P, P, P, P], ctypes.c_double),
    }
    for n, (a, r) in sigs.items():
        f = getattr(L, n)
        f.argtypes = a
        f.restype = r
    return L


_L = None


def lib():
    global _L
    if _L is None:
        _L = _load()
    return _L


def _p(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def codebook_table():
    out = np.empty(65536, np.uint16)
    lib().gfro_codebook_table(_p(out))
    return out


def unpack(words, kin, n, bits):
    """Trellis words [kin/16, n/16, 8*bits] (u32/i32) -> fp16 bits [kin, n] (experts.rs:47-74)."""
    w = np.ascontiguousarray(words).view(np.uint32)
    out = np.empty((kin, n), np.uint16)
    lib().gfro_unpack(_p(w), kin, n, bits, _p(out))
    return out


def unpack_f32(words, kin, n, bits, rounded=True):
    """fp32 weights [kin, n]: the reference's fp16 codebook values (rounded) or the unrounded sums of the two fp16
    halves (gfro_codebook_sum), which this library's decode GEMV multiplies."""
    w = np.ascontiguousarray(words).view(np.uint32)
    out = np.empty((kin, n), np.float32)
    (lib().gfro_unpack_f32 if rounded else lib().gfro_unpack_f32_sum)(_p(w), kin, n, bits, _p(out))
    return out


def codebook_sums():
    """gfro_codebook_sum of all 65536 states (fp32)."""
    return np.array([lib().gfro_codebook_sum(s) for s in range(65536)], np.float32)


def had(x):
    y = np.array(x, np.float32, copy=True, order="C")
    lib().gfro_had(_p(y), y.size)
    return y


def matmul(x, w, sk, warps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty(w.shape[1], np.float32)
    lib().gfro_matmul(_p(x), _p(w), w.shape[0], w.shape[1], sk, warps, _p(y))
    return y


def rot(x_bf16, suh):
    x = np.ascontiguousarray(x_bf16, np.uint16)
    s = np.ascontiguousarray(suh, np.uint16)
    out = np.empty(x.shape[-1], np.uint16)
    lib().gfro_rot(_p(x), _p(s), x.shape[-1], _p(out))
    return out


def rot_rows(x_bf16, rows, suh):
    """gfro_rot of the listed rows of x [*][k] bf16 bits with one scale vector -> fp16 bits [len(rows)][k]."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    r = np.ascontiguousarray(rows, np.int32)
    s = np.ascontiguousarray(suh, np.uint16)
    k = x.shape[-1]
    out = np.empty((len(r), k), np.uint16)
    lib().gfro_rot_rows(_p(x), k, _p(r), len(r), _p(s), k, _p(out))
    return out


def gateup_epilogue_rows(g, u, svh_g, svh_u, suh_d, limit=10.0):
    """gfro_gateup_epilogue of each row of g, u [rows][n] fp32 (copies; the inputs are left alone) -> xd fp16 bits."""
    g = np.array(g, np.float32, copy=True, order="C")
    u = np.array(u, np.float32, copy=True, order="C")
    rows, n = g.shape
    xd = np.empty((rows, n), np.uint16)
    vecs = [np.ascontiguousarray(a, np.uint16) for a in (svh_g, svh_u, suh_d)]
    lib().gfro_gateup_epilogue_rows(_p(g), _p(u), *[_p(v) for v in vecs], rows, n, limit, _p(xd))
    return xd


def down_epilogue_rows(z, svh_d):
    """gfro_down_epilogue of each row of z [rows][d] fp32 (a copy) -> y fp32 [rows][d]."""
    z = np.array(z, np.float32, copy=True, order="C")
    rows, d = z.shape
    y = np.empty((rows, d), np.float32)
    lib().gfro_down_epilogue_rows(_p(z), _p(np.ascontiguousarray(svh_d, np.uint16)), rows, d, _p(y))
    return y


def expert_row(x_bf16, wg, wu, wd, suh_g, suh_u, suh_d, svh_g, svh_u, svh_d, sk_gu=4, sk_d=1, warps=4, limit=10.0):
    """experts.rs:113-146 for one row: returns (y fp32 [D], xd fp16 bits [N])."""
    D, N = wg.shape
    y = np.empty(D, np.float32)
    xd = np.empty(N, np.uint16)
    args = [np.ascontiguousarray(a, np.uint16) for a in (x_bf16,)]
    lib().gfro_expert_row(_p(args[0]), D, N, _p(wg), _p(wu), _p(wd),
                          *[_p(np.ascontiguousarray(a, np.uint16)) for a in (suh_g, suh_u, suh_d, svh_g, svh_u, svh_d)],
                          sk_gu, sk_d, warps, limit, _p(y), _p(xd))
    return y, xd


def linear(x_f16, w, suh, svh):
    kin, n = w.shape
    y = np.empty(n, np.float32)
    lib().gfro_linear(_p(np.ascontiguousarray(x_f16, np.uint16)), kin, n, _p(np.ascontiguousarray(w, np.float32)),
                      _p(np.ascontiguousarray(suh, np.uint16)), _p(np.ascontiguousarray(svh, np.uint16)), _p(y))
    return y


def group(picks, rows, slots, E, maxm):
    """grouping.rs:141-192 host oracle; returns (count, ids[:count], members [E, maxm])."""
    p = np.ascontiguousarray(picks, np.int32)
    ids = np.full(E, -77, np.int32)
    count = np.zeros(1, np.int32)
    members = np.empty((E, maxm), np.int32)
    rc = lib().gfro_group(_p(p), rows, slots, E, maxm, _p(ids), _p(count), _p(members))
    if rc:
        raise ValueError("grouping precondition")
    return int(count[0]), ids[: count[0]].copy(), members


def route(logits, topk, shared_id):
    l = np.ascontiguousarray(logits, np.float32)
    rows, E = l.shape
    picks = np.empty((rows, topk + 1), np.int32)
    weights = np.empty((rows, topk + 1), np.float32)
    lib().gfro_route(_p(l), rows, E, topk, shared_id, _p(picks), _p(weights))
    return picks, weights


def route_biased(logits, bias, scale, topk, shared_id):
    l = np.ascontiguousarray(logits, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    rows, E = l.shape
    picks = np.empty((rows, topk + 1), np.int32)
    weights = np.empty((rows, topk + 1), np.float32)
    lib().gfro_route_biased(_p(l), _p(b), scale, rows, E, topk, shared_id, _p(picks), _p(weights))
    return picks, weights


def fp8_values():
    """front.rs:173-182: the value of every e4m3 byte 0..255."""
    return np.array([lib().gfro_fp8(v) for v in range(256)], np.float32)


def fp8_matmul(x, w, scale_bf16, sk, round_bf16):
    """front.rs:190-217 reference_mm_at for one row x [k] (f32) against w [n][k] (uint8) with bf16 scales [n]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(scale_bf16, np.uint16)
    n, k = w.shape
    y = np.empty(n, np.float32)
    lib().gfro_fp8_matmul(_p(x), _p(w), _p(sc), k, n, sk, 1 if round_bf16 else 0, _p(y))
    return y


def fp8_b16_copy(w, scale_bf16):
    """prefill.cu:7-17 f8_b16_copy: bf16 bits [n][k] of bf16_rn(fp8(w) * row scale)."""
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(scale_bf16, np.uint16)
    n, k = w.shape
    out = np.empty((n, k), np.uint16)
    lib().gfro_fp8_b16_copy(_p(w), _p(sc), n, k, _p(out))
    return out


def shared_swiglu(gu, inter, limit=10.0):
    gu = np.ascontiguousarray(gu, np.float32)
    act = np.empty(inter, np.float32)
    lib().gfro_shared_swiglu(_p(gu), inter, limit, _p(act))
    return act


def shared_fp8_row(x_bf16, w_gu, s_gu, w_d, s_d):
    """The FP8 shared expert for one token row as moe.rs:132-167 runs it: fmm(shared_gu, sk 8) + reduce8_bf16 ->
    gu (bf16), shared_swiglu (limit 10) -> act (bf16), fmm(shared_down, sk 1) -> fp32. Returns (gu, act, out)."""
    x = (np.asarray(x_bf16, np.uint16).astype(np.uint32) << 16).view(np.float32)
    inter = w_gu.shape[0] // 2
    gu = fp8_matmul(x, w_gu, s_gu, 8, True)
    act = shared_swiglu(gu, inter)
    out = fp8_matmul(act, w_d, s_d, 1, False)
    return gu, act, out


def combine(y, weights, rows, slots):
    y = np.ascontiguousarray(y, np.float32)
    w = np.ascontiguousarray(weights, np.float32)
    D = y.shape[-1]
    out = np.empty((rows, D), np.float32)
    lib().gfro_combine(_p(y), _p(w), rows, slots, D, _p(out))
    return out


def baseline_decode(x_bf16, D, N, bits, experts, gt, ut, dt, suh_g, suh_u, suh_d, svh_g, svh_u, svh_d):
    """Timed scalar decode + matvec of the listed experts for one token; returns (seconds, y [n, D])."""
    ex = np.ascontiguousarray(experts, np.int32)
    y = np.empty((len(ex), D), np.float32)
    arrs = [np.ascontiguousarray(a) for a in (gt, ut, dt)]
    vecs = [np.ascontiguousarray(a, np.uint16) for a in (suh_g, suh_u, suh_d, svh_g, svh_u, svh_d)]
    t = lib().gfro_baseline_decode(_p(np.ascontiguousarray(x_bf16, np.uint16)), D, N, bits, len(ex), _p(ex),
                                   *[_p(a) for a in arrs], *[_p(v) for v in vecs], _p(y))
    return t, y
