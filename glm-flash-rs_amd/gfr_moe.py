"""Python mirror of the reference's expert-dispatch surface over libgfr_moe.so (include/gfr_moe.h).

Class names and call shapes follow glm-flash-rs: Grouping (src/grouping.rs:12-112), ExpertGpu (src/experts.rs:365-564),
FastExperts (src/fast_experts.rs:27-208), Moe (src/moe.rs:1-183). Device memory and streams come from PyTorch-ROCm
(plumbing only); every computation runs in the HIP library. Importing this module on a machine without the built
library raises: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgfr_moe.so")

GFR_EINVAL = -1


class GfrError(RuntimeError):
    """A failed library call: code < 0 is a precondition (the reference's ensure!), code > 0 a hipError_t."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"gfr error {code}: {msg}")
        self.code = code


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    P, I, VP = ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p
    sig = {
        "gfr_last_error": ([], ctypes.c_char_p),
        "gfr_version": ([], ctypes.c_char_p),
        "gfr_grouping_create": ([ctypes.POINTER(VP), I, I, I], I),
        "gfr_grouping_run": ([VP, P, P, I], I),
        "gfr_grouping_ids": ([VP], P),
        "gfr_grouping_count": ([VP], P),
        "gfr_grouping_members": ([VP], P),
        "gfr_grouping_destroy": ([VP], I),
        "gfr_experts_create": ([ctypes.POINTER(VP), I, I, I, I, I], I),
        "gfr_experts_run_rows": ([VP, P, P, P, I, P, P, P, P, I, I], I),
        "gfr_experts_y": ([VP], P),
        "gfr_experts_xd": ([VP], P),
        "gfr_experts_destroy": ([VP], I),
        "gfr_fast_experts_create": ([ctypes.POINTER(VP), I, I, I, I, I, I], I),
        "gfr_fast_experts_run": ([VP, P, P, P, I, P, P, P, P, I, I, I], I),
        "gfr_fast_experts_output": ([VP], P),
        "gfr_fast_experts_xd": ([VP], P),
        "gfr_fast_experts_rotated": ([VP, I], P),
        "gfr_fast_experts_destroy": ([VP], I),
        "gfr_moe_create": ([ctypes.POINTER(VP), I, I, I, I, I], I),
        "gfr_moe_run": ([VP, P, P, P, P, I], I),
        "gfr_moe_output": ([VP], P),
        "gfr_moe_picks": ([VP], P),
        "gfr_moe_weights": ([VP], P),
        "gfr_moe_rotated": ([VP, I], P),
        "gfr_moe_set_decode_rows": ([VP, I], I),
        "gfr_moe_create_shared": ([ctypes.POINTER(VP), I, I, I, I, I, I], I),
        "gfr_moe_run_shared": ([VP, P, P, P, P, P, I, I], I),
        "gfr_moe_run_shared_branch": ([VP, P, P, P, P, P, I, I, P], I),
        "gfr_moe_run_router": ([VP, P, P, P, P, P, I, I], I),
        "gfr_router_logits": ([P, P, I, P, I, I, I, P], I),
        "gfr_moe_set_launches": ([VP, I], I),
        "gfr_moe_token_static": ([P, ctypes.POINTER(_Exl3Struct), I, I, P, P, P, P, P], I),
        "gfr_moe_destroy": ([VP], I),
        "gfr_shared_fp8_create": ([ctypes.POINTER(VP), I, I, I], I),
        "gfr_fp8_prepare_bf16": ([P, ctypes.POINTER(_Fp8Struct), P, P], I),
        "gfr_shared_fp8_run": ([VP, P, ctypes.POINTER(_Fp8Struct), P, I, I, P, I], I),
        "gfr_shared_fp8_gu": ([VP], P),
        "gfr_shared_fp8_act": ([VP], P),
        "gfr_shared_fp8_destroy": ([VP], I),
        "gfr_moe_run_fp8": ([VP, P, ctypes.POINTER(_Exl3Struct), P, P, ctypes.POINTER(_Fp8Struct), I], I),
        "gfr_moe_run_router_fp8": ([VP, P, ctypes.POINTER(_Exl3Struct), P, P, ctypes.POINTER(_Fp8Struct), I], I),
        "gfr_moe_shared_output": ([VP], P),
        "gfr_prepared_shared_fp8": ([VP, I, ctypes.POINTER(_Fp8Struct)], I),
        "gfr_linear_create": ([ctypes.POINTER(VP), I, I, I], I),
        "gfr_linear_run": ([VP, P, P, P, P, P, P], I),
        "gfr_linear_destroy": ([VP], I),
        "gfr_exl3_decode_tiles": ([P, P, I, I, I, P], I),
        "gfr_exl3_gemv_splits": ([I], I),
        "gfr_exl3_rotate": ([P, P, I, I, P, P, I, I, P], I),
        "gfr_route_topk": ([P, P, I, I, I, P, P], I),
        "gfr_route_topk_biased": ([P, P, P, ctypes.c_float, I, I, I, P, P], I),
        "gfr_moe_set_router": ([VP, P, ctypes.c_float], I),
        "gfr_exl3_grouped_gemv": ([P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I], I),
        "gfr_prepared_open": ([ctypes.POINTER(VP), ctypes.c_char_p], I),
        "gfr_prepared_tensor_count": ([VP], I),
        "gfr_prepared_tensor_name": ([VP, I], ctypes.c_char_p),
        "gfr_prepared_tensor": ([VP, ctypes.c_char_p, ctypes.POINTER(TensorInfo)], I),
        "gfr_prepared_expect": ([VP, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64), I], I),
        "gfr_prepared_read_tensor": ([VP, ctypes.c_char_p, ctypes.c_uint64, ctypes.c_uint64, P], I),
        "gfr_prepared_load": ([VP, ctypes.POINTER(ctypes.c_char_p), I], I),
        "gfr_prepared_loaded": ([VP, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_double)], I),
        "gfr_prepared_pointer": ([VP, ctypes.c_char_p, ctypes.POINTER(VP)], I),
        "gfr_prepared_experts": ([VP, I, ctypes.POINTER(_Exl3Struct)], I),
        "gfr_prepared_destroy": ([VP], I),
        "gfr_sha256_hex": ([P, ctypes.c_uint64, ctypes.c_char_p], I),
        "gfr_prefetch_abi": ([], ctypes.c_uint32),
        "gfr_prefetch_properties": ([ctypes.POINTER(I), ctypes.POINTER(I)], I),
        "gfr_prefetch_capturing": ([P, ctypes.POINTER(I)], I),
        "gfr_prefetch_segments": ([P, I, I, P], I),
        "gfr_prefetch_experts": ([P, P, I, P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, I, P], I),
        "gfr_tensor_extent": ([ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64), I, I,
                               ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)], I),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    return lib


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _check(rc: int):
    if rc != 0:
        raise GfrError(rc, lib().gfr_last_error().decode())


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class _DeviceArray:
    """__cuda_array_interface__ over library-owned device memory."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr, "data": (ptr, False),
                                         "version": 3, "strides": None}


_TYPESTR = {torch.float32: "<f4", torch.int32: "<i4", torch.float16: "<f2", torch.int16: "<i2", torch.uint8: "|u1"}


def _view(ptr: int, shape, dtype, device) -> torch.Tensor:
    """A torch tensor over library-owned device memory (no copy; valid while the engine lives)."""
    if dtype == torch.bfloat16:
        return _view(ptr, shape, torch.int16, device).view(torch.bfloat16)
    t = torch.as_tensor(_DeviceArray(ptr, shape, _TYPESTR[dtype]), device=device)
    assert t.data_ptr() == ptr
    return t


@dataclass
class Exl3Experts:
    """One layer's EXL3 expert tensors (the reference's weights.layers[L].moe.experts.*, experts.rs:146-156).

    gt, ut: [E, hidden/16, inter/16, 8*bits] int32; dt: [E, inter/16, hidden/16, 8*bits] int32;
    suh_g, suh_u, svh_d: [E, hidden] fp16; suh_d, svh_g, svh_u: [E, inter] fp16.
    """

    gt: torch.Tensor
    ut: torch.Tensor
    dt: torch.Tensor
    suh_g: torch.Tensor
    suh_u: torch.Tensor
    suh_d: torch.Tensor
    svh_g: torch.Tensor
    svh_u: torch.Tensor
    svh_d: torch.Tensor
    bits: int

    @property
    def experts(self) -> int:
        return self.gt.shape[0]

    @property
    def hidden(self) -> int:
        return self.suh_g.shape[1]

    @property
    def inter(self) -> int:
        return self.suh_d.shape[1]

    def check(self):
        E, D, N, b = self.experts, self.hidden, self.inter, self.bits
        want = {
            "gt": ((E, D // 16, N // 16, 8 * b), torch.int32), "ut": ((E, D // 16, N // 16, 8 * b), torch.int32),
            "dt": ((E, N // 16, D // 16, 8 * b), torch.int32),
            "suh_g": ((E, D), torch.float16), "suh_u": ((E, D), torch.float16), "svh_d": ((E, D), torch.float16),
            "suh_d": ((E, N), torch.float16), "svh_g": ((E, N), torch.float16), "svh_u": ((E, N), torch.float16),
        }
        for name, (shape, dtype) in want.items():
            t = getattr(self, name)
            if tuple(t.shape) != shape or t.dtype != dtype or not t.is_contiguous() or t.device.type != "cuda":
                raise ValueError(f"{name}: {tuple(t.shape)} {t.dtype}, want {shape} {dtype} contiguous on GPU")

    def struct(self) -> "_Exl3Struct":
        self.check()
        return _Exl3Struct(self.experts, self.hidden, self.inter, self.bits, *(
            _ptr(getattr(self, n)) for n in ("gt", "ut", "dt", "suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")))


class _Exl3Struct(ctypes.Structure):
    _fields_ = [("experts", ctypes.c_int), ("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("bits", ctypes.c_int)] + [
        (n, ctypes.c_void_p) for n in ("gt", "ut", "dt", "suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")]


@dataclass
class Fp8SharedWeights:
    """The reference's FP8 shared expert, weights.layers[L].moe.shared.{gu,down}.{weight,scale} (moe.rs:136-161):
    gu [2 inter, hidden] and down [hidden, inter] float8_e4m3fn bytes (torch.uint8 or torch.float8_e4m3fn),
    gu_scale [2 inter] and down_scale [hidden] bf16; contiguous on the GPU, 16-byte aligned."""

    gu: torch.Tensor
    gu_scale: torch.Tensor
    down: torch.Tensor
    down_scale: torch.Tensor
    gu_bf16: torch.Tensor = None      # the prefill form's bf16 copies (prepare_bf16), or None
    down_bf16: torch.Tensor = None

    @property
    def hidden(self) -> int:
        return self.gu.shape[1]

    @property
    def inter(self) -> int:
        return self.gu.shape[0] // 2

    def prepare_bf16(self, stream=None) -> "Fp8SharedWeights":
        """The reference's prefill weight copies (f8_b16_copy, prefill.cu:7-17: bf16(fp8 * row scale)) via
        gfr_fp8_prepare_bf16; windows of more than 16 rows then run the reference's prefill arithmetic."""
        H, I = self.hidden, self.inter
        self.gu_bf16 = torch.empty((2 * I, H), dtype=torch.bfloat16, device=self.gu.device)
        self.down_bf16 = torch.empty((H, I), dtype=torch.bfloat16, device=self.gu.device)
        st = self.struct()
        _check(lib().gfr_fp8_prepare_bf16(_stream(stream), ctypes.byref(st), _ptr(self.gu_bf16), _ptr(self.down_bf16)))
        return self

    def check(self):
        H, I = self.hidden, self.inter
        want = {"gu": (2 * I, H), "gu_scale": (2 * I,), "down": (H, I), "down_scale": (H,)}
        if self.gu_bf16 is not None or self.down_bf16 is not None:
            want.update({"gu_bf16": (2 * I, H), "down_bf16": (H, I)})
        for name, shape in want.items():      # shapes and dtypes first, then where the tensors live
            t = getattr(self, name)
            bf = name.endswith("scale") or name.endswith("bf16")
            if t is None or tuple(t.shape) != shape or (t.dtype == torch.bfloat16) != bf or t.element_size() != (
                    2 if bf else 1):
                got = "missing" if t is None else f"{tuple(t.shape)} {t.dtype}"
                raise ValueError(f"{name}: {got}, want {shape} {'bf16' if bf else 'e4m3 bytes'}")
        for name in want:
            t = getattr(self, name)
            if not t.is_contiguous() or t.device.type != "cuda":
                raise ValueError(f"{name}: want a contiguous tensor on the GPU")

    def struct(self) -> "_Fp8Struct":
        self.check()
        return _Fp8Struct(self.hidden, self.inter, *(_ptr(getattr(self, n)) for n in (
            "gu", "gu_scale", "down", "down_scale", "gu_bf16", "down_bf16")))


class _Fp8Struct(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int)] + [
        (n, ctypes.c_void_p) for n in ("gu", "gu_scale", "down", "down_scale", "gu_bf16", "down_bf16")]


class _Engine:
    _destroy = None

    def __init__(self):
        self._h = ctypes.c_void_p()

    def close(self):
        if self._h:
            getattr(lib(), self._destroy)(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Grouping(_Engine):
    """Grouping::new / run (grouping.rs:29-112). ids, count, members are views of the engine's buffers."""

    _destroy = "gfr_grouping_destroy"

    def __init__(self, experts: int, slots: int, max_rows: int, device="cuda"):
        super().__init__()
        _check(lib().gfr_grouping_create(ctypes.byref(self._h), experts, slots, max_rows))
        self.experts, self.slots, self.max_rows = experts, slots, max_rows
        L = lib()
        self.ids = _view(L.gfr_grouping_ids(self._h), (experts,), torch.int32, device)
        self.count = _view(L.gfr_grouping_count(self._h), (1,), torch.int32, device)
        self.members = _view(L.gfr_grouping_members(self._h), (experts, max_rows), torch.int32, device)

    def run(self, picks: torch.Tensor, rows: int, stream=None):
        if picks.dtype != torch.int32 or not picks.is_contiguous():
            raise ValueError("picks must be contiguous int32")
        _check(lib().gfr_grouping_run(self._h, _stream(stream), _ptr(picks), rows))


class ExpertGpu(_Engine):
    """ExpertGpu::with_policy / run_rows (experts.rs:385-563); y: [max_rows * slots, hidden] fp32."""

    _destroy = "gfr_experts_destroy"

    def __init__(self, hidden: int, inter: int, slots: int, exl3_slots: int, max_rows: int, device="cuda"):
        super().__init__()
        _check(lib().gfr_experts_create(ctypes.byref(self._h), hidden, inter, slots, exl3_slots, max_rows))
        self.hidden, self.inter, self.slots, self.max_rows = hidden, inter, slots, max_rows
        P = max_rows * slots
        self.y = _view(lib().gfr_experts_y(self._h), (P, hidden), torch.float32, device)
        self.xd = _view(lib().gfr_experts_xd(self._h), (P, inter), torch.float16, device)

    def run_rows(self, w: Exl3Experts, input: torch.Tensor, picks, ids, count, members, rows: int, maxm: int,
                 stream=None):
        if input.dtype != torch.bfloat16:
            raise ValueError("input must be bf16 [rows, stride]")
        ws = w.struct()
        _check(lib().gfr_experts_run_rows(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), input.stride(0),
                                          _ptr(picks), _ptr(ids), _ptr(count), _ptr(members), rows, maxm))


class FastExperts(_Engine):
    """FastExperts::new / run (fast_experts.rs:43-208); output: [max_rows * slots, hidden] fp32."""

    _destroy = "gfr_fast_experts_destroy"

    def __init__(self, hidden: int, inter: int, slots: int, exl3_slots: int, experts: int, max_rows: int,
                 device="cuda"):
        super().__init__()
        _check(lib().gfr_fast_experts_create(ctypes.byref(self._h), hidden, inter, slots, exl3_slots, experts,
                                             max_rows))
        P = max_rows * slots
        self.output = _view(lib().gfr_fast_experts_output(self._h), (P, hidden), torch.float32, device)
        self.xd = _view(lib().gfr_fast_experts_xd(self._h), (P, inter), torch.float16, device)
        # parity probe: the rotated input rows of the last run, k tiles in pair order (see gfr_fast_experts_rotated)
        self.rotated = [_view(lib().gfr_fast_experts_rotated(self._h, m), (P, hidden), torch.float16, device)
                        for m in (0, 1)]

    def run(self, w: Exl3Experts, input, picks, ids, count, members, rows: int, maxm: int, shared_x: bool,
            stream=None):
        ws = w.struct()
        _check(lib().gfr_fast_experts_run(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), input.stride(0),
                                          _ptr(picks), _ptr(ids), _ptr(count), _ptr(members), rows, maxm,
                                          int(shared_x)))


class Moe(_Engine):
    """Moe::run_prefetched (moe.rs:66-182): router (the benchmark's softmax top-k, or GLM's sigmoid + bias gate via
    set_router) -> grouping -> EXL3 experts -> combine. shared_exl3=True: the shared expert is the weights' last EXL3
    expert (the benchmark configs); False: the reference's layout, whose shared expert is not EXL3 and whose output
    the caller passes to run (the reference's combine(y, shared, weights, out), moe.rs:171-181)."""

    _destroy = "gfr_moe_destroy"

    def __init__(self, hidden: int, inter: int, routed: int, topk: int, max_rows: int, device="cuda",
                 shared_exl3: bool = True):
        super().__init__()
        _check(lib().gfr_moe_create_shared(ctypes.byref(self._h), hidden, inter, routed, topk, max_rows,
                                           int(shared_exl3)))
        self.hidden, self.routed, self.topk, self.max_rows = hidden, routed, topk, max_rows
        L = lib()
        self.output = _view(L.gfr_moe_output(self._h), (max_rows, hidden), torch.float32, device)
        self.picks = _view(L.gfr_moe_picks(self._h), (max_rows, topk + 1), torch.int32, device)
        self.weights = _view(L.gfr_moe_weights(self._h), (max_rows, topk + 1), torch.float32, device)

    def set_decode_rows(self, n: int):
        _check(lib().gfr_moe_set_decode_rows(self._h, n))

    def rotated(self, mat: int, rows: int) -> torch.Tensor:
        """Parity probe (gfr_moe_rotated): the rotated input rows of the last prefill-engine run, [rows * (topk + 1),
        hidden] fp16, k tiles in pair order."""
        return _view(lib().gfr_moe_rotated(self._h, mat), (rows * (self.topk + 1), self.hidden), torch.float16,
                     self.output.device)

    def set_launches(self, n: int):
        """Measurement aid (gfr_moe_set_launches): a one-row run issues only its first n launches (0: all)."""
        _check(lib().gfr_moe_set_launches(self._h, n))

    def set_router(self, bias: torch.Tensor = None, scale: float = 2.5):
        """GLM's gate (the reference's topk(logits, bias, picks, weights, 2.5), moe.rs:89-99) with this fp32 bias
        [routed]; None: back to the softmax gate. The tensor must outlive the runs."""
        self._router_bias = bias
        _check(lib().gfr_moe_set_router(self._h, _ptr(bias), float(scale) if bias is not None else 1.0))

    def run(self, w: Exl3Experts, input: torch.Tensor, logits: torch.Tensor, rows: int, stream=None,
            shared: torch.Tensor = None, shared_ready: "torch.cuda.Event" = None):
        """shared: the non-EXL3 shared expert's output [rows, >= hidden] fp32 (a layer made with shared_exl3=False).
        shared_ready: an event recorded (on another stream) once `shared` is written; only the combine waits for it
        (gfr_moe_run_shared_branch; SharedBranch drives the fork and the join)."""
        ws = w.struct()
        if shared_ready is not None:
            if shared is None:
                raise ValueError("shared_ready without a shared output")
            _check(lib().gfr_moe_run_shared_branch(self._h, _stream(stream), ctypes.byref(ws), _ptr(input),
                                                   _ptr(logits), _ptr(shared), shared.stride(0), rows,
                                                   ctypes.c_void_p(shared_ready.cuda_event)))
        elif shared is None:
            _check(lib().gfr_moe_run(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), _ptr(logits), rows))
        else:
            _check(lib().gfr_moe_run_shared(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), _ptr(logits),
                                            _ptr(shared), shared.stride(0), rows))

    def run_fp8(self, w: Exl3Experts, input: torch.Tensor, logits: torch.Tensor, sw: Fp8SharedWeights, rows: int,
                stream=None):
        """Moe::run_prefetched with its FP8 shared expert (a layer made with shared_exl3=False): the shared expert
        into shared_output, then the routed layer and the combine."""
        ws, ss = w.struct(), sw.struct()
        _check(lib().gfr_moe_run_fp8(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), _ptr(logits),
                                     ctypes.byref(ss), rows))

    def run_router_fp8(self, w: Exl3Experts, input: torch.Tensor, router_weight: torch.Tensor,
                       sw: Fp8SharedWeights, rows: int, stream=None):
        """run_fp8 with the router logits computed from the hidden rows first (router_weight [routed, hidden])."""
        ws, ss = w.struct(), sw.struct()
        _check(lib().gfr_moe_run_router_fp8(self._h, _stream(stream), ctypes.byref(ws), _ptr(input),
                                            _ptr(router_weight), ctypes.byref(ss), rows))

    @property
    def shared_output(self) -> torch.Tensor:
        """[max_rows, hidden] fp32: the FP8 shared expert's output of the last run_fp8 (shared_exl3=False)."""
        p = lib().gfr_moe_shared_output(self._h)
        if not p:
            raise ValueError("the layer has no FP8 shared expert")
        return _view(p, (self.max_rows, self.hidden), torch.float32, self.output.device)

    def run_router(self, w: Exl3Experts, input: torch.Tensor, router_weight: torch.Tensor, rows: int, stream=None,
                   shared: torch.Tensor = None):
        """The layer from the hidden rows: router logits (router_weight [routed, hidden] bf16) then run."""
        ws = w.struct()
        _check(lib().gfr_moe_run_router(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), _ptr(router_weight),
                                        _ptr(shared), shared.stride(0) if shared is not None else 0, rows))


class SharedBranch:
    """The shared / routed expert fork of the reference's shared_expert.rs Branch (:18-78): the shared expert's
    kernels run on this branch's own stream (default priority), the routed experts on the caller's, and the two join
    before the combine. run(main, shared_fn, routed_fn): shared_fn(stream) launches the shared expert on the branch
    stream; routed_fn(ready) launches the routed layer on `main` with ready as its shared-ready event (Moe.run(...,
    shared=..., shared_ready=ready)). The main stream is joined to the branch even when routed_fn raises, so the
    caller's buffers are safe to reuse after main's later work. Works under stream capture (a fork and a join of
    events)."""

    def __init__(self, device="cuda"):
        self.stream = torch.cuda.Stream(device)
        self.fork = torch.cuda.Event()
        self.joined = torch.cuda.Event()

    def run(self, main, shared_fn, routed_fn):
        self.fork.record(main)
        self.stream.wait_event(self.fork)
        with torch.cuda.stream(self.stream):
            shared_fn(self.stream)
        self.joined.record(self.stream)
        try:
            routed_fn(self.joined)
        finally:
            main.wait_event(self.joined)


# ---- Cache-warming read hints (src/l2_prefetch_plan.rs, src/l2_prefetch.rs; kernels in csrc/prefetch.hip) -------
# The plan functions restate the reference's host policy (same constants, bounds and rounding), so a caller that
# plans with them gets the spans the reference would plan; a failed bound raises ValueError where the reference's
# ensure! returns an error.
PF_ALIGN = 16
PF_BUDGET = 8 << 20
PF_L2_FALLBACK = 24 << 20
PF_EXPERT_BYTES = 64 << 10
PF_MAX_ROWS = 64
PF_CHUNK = 32 << 10         # the reference's bulk-prefetch piece: one instruction a 32 KiB chunk
PF_THREADS = 128
PF_LINE_CHUNK = 2 << 10     # a thread's share here: 16 lines of 128 bytes, one dword load a line


@dataclass(frozen=True)
class PfTensor:
    """A weight tensor's device range (l2_prefetch_plan.rs Tensor)."""
    address: int
    bytes: int
    contiguous: bool = True


@dataclass(frozen=True)
class PfSpan:
    address: int
    bytes: int


@dataclass(frozen=True)
class ExpertPlan:
    bases: tuple
    stride: int
    bytes: int
    experts: int


def _pf_ensure(ok, msg):
    if not ok:
        raise ValueError(msg)


def pf_budget(l2_bytes: int) -> int:
    """Bytes a site may hint: half the L2, at most 8 MiB (l2_prefetch_plan.rs:80-82)."""
    return min(PF_BUDGET, (PF_L2_FALLBACK if l2_bytes == 0 else l2_bytes) // 2)


def pf_rows_enabled(rows: int) -> bool:
    """Hints are for decode rounds only: 1..64 rows (l2_prefetch_plan.rs:83-85)."""
    return 0 < rows <= PF_MAX_ROWS


def pf_grid(nbytes: int, cus: int, chunk: int = PF_CHUNK) -> int:
    """Workgroups of a segment launch: one thread a chunk, 128 threads a workgroup, 1..cus (l2_prefetch_plan.rs:86-92;
    the default chunk is the reference's, Prefetch passes PF_LINE_CHUNK for this library's line reads)."""
    _pf_ensure(0 < nbytes <= PF_BUDGET and cus > 0, "L2 segment grid bounds")
    pieces = -(-nbytes // chunk)
    return max(1, min(cus, -(-pieces // PF_THREADS)))


def pf_expert_grid(rows: int, experts: int, capacity: int, cus: int):
    """(maxu, grid) of an expert hint: the window's min(rows * 8, experts) routed experts plus the shared slot, one
    workgroup an expert up to the CU count (l2_prefetch_plan.rs:93-111)."""
    _pf_ensure(pf_rows_enabled(rows) and experts > 0 and cus > 0, "L2 expert grid policy")
    maxu = min(rows * 8, experts) + 1
    _pf_ensure(maxu <= capacity and maxu <= 2 ** 31 - 1, "L2 expert group capacity")
    return maxu, min(cus, maxu)


def pf_span(t: PfTensor, left: int):
    """The 16-byte aligned part of a tensor that fits in `left` bytes, or None (l2_prefetch_plan.rs Tensor::span)."""
    if not t.contiguous or t.bytes == 0 or left < PF_ALIGN:
        return None
    _pf_ensure(t.address != 0, "null L2 prefetch address")
    end = t.address + t.bytes
    _pf_ensure(end < 2 ** 64, "L2 tensor extent overflow")
    _pf_ensure(t.address + PF_ALIGN - 1 < 2 ** 64, "L2 alignment overflow")
    address = (t.address + PF_ALIGN - 1) // PF_ALIGN * PF_ALIGN
    n = min(left, max(0, end - address)) // PF_ALIGN * PF_ALIGN
    return PfSpan(address, n) if n > 0 else None


def pf_take(items, budget: int):
    """Spans of the items in order until the budget is spent (l2_prefetch_plan.rs take, without its test-only Q4
    item). An item is a PfTensor, or a (scale, weight) pair of PfTensors: the scales first."""
    _pf_ensure(0 < budget <= PF_BUDGET, "L2 site budget bound")
    spans, left = [], budget
    for it in items:
        if left < PF_ALIGN:
            break
        for t in (it if isinstance(it, tuple) else (it,)):
            sp = pf_span(t, left)
            if sp is not None:
                left -= sp.bytes
                spans.append(sp)
    return spans


def pf_experts(gate: PfTensor, up: PfTensor, count: int):
    """The routed-expert hint of one layer: the first min(64 KiB, stride) bytes of each expert in the gate and up
    trellis tensors, or None when the layout does not allow it (l2_prefetch_plan.rs:183-219)."""
    if count == 0 or gate.bytes != up.bytes or not gate.contiguous or not up.contiguous or gate.bytes % count:
        return None
    stride = gate.bytes // count
    n = min(PF_EXPERT_BYTES, stride) // PF_ALIGN * PF_ALIGN
    if n == 0 or stride % PF_ALIGN or gate.address % PF_ALIGN or up.address % PF_ALIGN:
        return None
    _pf_ensure(gate.address != 0 and up.address != 0, "null L2 expert address")
    _pf_ensure(gate.address + gate.bytes < 2 ** 64 and up.address + up.bytes < 2 ** 64, "L2 expert extent overflow")
    _pf_ensure(count < 2 ** 63 and stride < 2 ** 63, "L2 expert launch bounds")
    return ExpertPlan((gate.address, up.address), stride, n, count)


def prefetch_properties():
    """(CU count, L2 bytes) of the current device (gfr_prefetch_properties)."""
    cus, l2 = ctypes.c_int(), ctypes.c_int()
    _check(lib().gfr_prefetch_properties(ctypes.byref(cus), ctypes.byref(l2)))
    return cus.value, l2.value


def prefetch_capturing(stream) -> bool:
    active = ctypes.c_int()
    _check(lib().gfr_prefetch_capturing(_stream(stream), ctypes.byref(active)))
    return active.value == 1


class Prefetch:
    """Side-stream read hints (src/l2_prefetch.rs Owner:214-407, the per-layer tables without the model's attention
    sites): segment tables and routed-expert plans registered once (device tables allocated here, at setup), then
    mark / experts fork a side stream from `main` and launch the read kernels on it, and join(main) makes main wait
    for them. The kernels write nothing, so a hint never changes a result. The weights, tables and ids must stay
    alive until the join; under capture, a fork and a join must both fall in the same capture (as the reference's)."""

    def __init__(self, device="cuda"):
        self.device = torch.device(device)
        self.cus, self.l2 = prefetch_properties()
        _pf_ensure(lib().gfr_prefetch_abi() == 1, "prefetch ABI mismatch")
        self.budget = pf_budget(self.l2)
        self.side = torch.cuda.Stream(self.device)
        self.fork_ev = torch.cuda.Event()
        self.joined = torch.cuda.Event()
        self.tables = {}
        self.expert_plans = {}
        self.pending = False
        self.captured = False
        self.stats = {"launches": 0, "expert_launches": 0, "skipped_rows": 0, "bytes_planned": 0}

    def add_segments(self, key, spans):
        _pf_ensure(0 < len(spans) < 2 ** 31, "L2 span table bounds")
        total = sum(sp.bytes for sp in spans)
        table = torch.tensor([[sp.address, sp.bytes] for sp in spans], dtype=torch.int64, device=self.device)
        self.tables[key] = (table, len(spans), pf_grid(total, self.cus, PF_LINE_CHUNK))
        self.stats["bytes_planned"] += total

    def add_experts(self, layer, plan: ExpertPlan):
        bases = torch.tensor(list(plan.bases), dtype=torch.int64, device=self.device)
        self.expert_plans[layer] = (bases, plan)

    def _fork(self, main):
        capture = prefetch_capturing(main)
        if self.pending and capture != self.captured:
            self.pending = False
        self.fork_ev.record(main)
        self.side.wait_event(self.fork_ev)
        self.captured = capture
        self.pending = True

    def mark(self, main, key, rows: int):
        if not pf_rows_enabled(rows):
            self.stats["skipped_rows"] += 1
            return
        if key not in self.tables:
            return
        table, n, grid = self.tables[key]
        self._fork(main)
        _check(lib().gfr_prefetch_segments(_ptr(table), n, grid, _stream(self.side)))
        self.stats["launches"] += 1

    def experts(self, main, layer, rows: int, ids: torch.Tensor, count: torch.Tensor):
        """Call right after grouped routing (ids / count: the grouping's device output), before the shared expert."""
        if not pf_rows_enabled(rows) or layer not in self.expert_plans:
            return
        _pf_ensure(ids.dtype == torch.int32 and ids.numel() > 0 and count.numel() >= 1, "L2 routing buffer bounds")
        bases, plan = self.expert_plans[layer]
        maxu, grid = pf_expert_grid(rows, plan.experts, ids.numel(), self.cus)
        self._fork(main)
        _check(lib().gfr_prefetch_experts(_ptr(ids), _ptr(count), maxu, _ptr(bases), plan.stride, plan.bytes,
                                          plan.experts, grid, _stream(self.side)))
        self.stats["expert_launches"] += 1

    def join(self, main):
        if self.pending:
            if prefetch_capturing(main) == self.captured:
                self.joined.record(self.side)
                main.wait_event(self.joined)
            self.pending = False


class Linear(_Engine):
    """One EXL3 linear on one fp16 token (benchmark config 1)."""

    _destroy = "gfr_linear_destroy"

    def __init__(self, kin: int, n: int, bits: int):
        super().__init__()
        _check(lib().gfr_linear_create(ctypes.byref(self._h), kin, n, bits))

    def run(self, x, trellis, suh, svh, y, stream=None):
        _check(lib().gfr_linear_run(self._h, _stream(stream), _ptr(x), _ptr(trellis), _ptr(suh), _ptr(svh), _ptr(y)))


def moe_token_static(w: Exl3Experts, routed: int, topk: int, input: torch.Tensor, logits: torch.Tensor,
                     out: torch.Tensor, picks: torch.Tensor = None, weights: torch.Tensor = None, stream=None):
    """gfr_moe_token_static: one token through the bs = 1 layer with the library's fixed scratch (no allocation)."""
    ws = w.struct()
    _check(lib().gfr_moe_token_static(_stream(stream), ctypes.byref(ws), routed, topk, _ptr(input), _ptr(logits),
                                      _ptr(out), _ptr(picks), _ptr(weights)))


def router_logits(input: torch.Tensor, router_weight: torch.Tensor, stream=None) -> torch.Tensor:
    """gfr_router_logits: [rows, routed] fp32 logits of bf16 rows [rows, hidden] and a bf16 weight [routed, hidden]."""
    if input.dtype != torch.bfloat16 or router_weight.dtype != torch.bfloat16:
        raise ValueError("router logits take bf16 rows and a bf16 weight")
    rows, hidden = input.shape
    routed = router_weight.shape[0]
    out = torch.empty((rows, routed), dtype=torch.float32, device=input.device)
    _check(lib().gfr_router_logits(_stream(stream), _ptr(input), input.stride(0), _ptr(router_weight), hidden, routed,
                                   rows, _ptr(out)))
    return out


def route(logits: torch.Tensor, topk: int, stream=None):
    """The router alone: (picks [rows, topk + 1] int32, weights [rows, topk + 1] fp32), shared id = routed."""
    rows, routed = logits.shape
    picks = torch.empty((rows, topk + 1), dtype=torch.int32, device=logits.device)
    weights = torch.empty((rows, topk + 1), dtype=torch.float32, device=logits.device)
    _check(lib().gfr_route_topk(_stream(stream), _ptr(logits), rows, routed, topk, _ptr(picks), _ptr(weights)))
    return picks, weights


def route_biased(logits: torch.Tensor, bias: torch.Tensor, topk: int, scale: float = 2.5, stream=None):
    """GLM's gate alone (gfr_route_topk_biased): (picks, weights) [rows, topk + 1], shared id = routed."""
    rows, routed = logits.shape
    picks = torch.empty((rows, topk + 1), dtype=torch.int32, device=logits.device)
    weights = torch.empty((rows, topk + 1), dtype=torch.float32, device=logits.device)
    _check(lib().gfr_route_topk_biased(_stream(stream), _ptr(logits), _ptr(bias), float(scale), rows, routed, topk,
                                       _ptr(picks), _ptr(weights)))
    return picks, weights


def rotate(x: torch.Tensor, expert: torch.Tensor, suh: torch.Tensor, stream=None) -> torch.Tensor:
    """rot_in's formula (exl3.cu:224-241) on rows x [rows, k] (bf16 or fp16) with per-row experts: fp16 [rows, k]."""
    rows, k = x.shape
    out = torch.empty((rows, k), dtype=torch.float16, device=x.device)
    _check(lib().gfr_exl3_rotate(_stream(stream), _ptr(x), x.stride(0), int(x.dtype == torch.float16), _ptr(expert),
                                 _ptr(suh), k, rows, _ptr(out)))
    return out


def decode_tiles(trellis: torch.Tensor, kin: int, n: int, bits: int, stream=None) -> torch.Tensor:
    """Decoded fp16 weights [kin, n] of one trellis matrix (bit-exact parity entry point)."""
    out = torch.empty((kin, n), dtype=torch.float16, device=trellis.device)
    _check(lib().gfr_exl3_decode_tiles(_stream(stream), _ptr(trellis), kin, n, bits, _ptr(out)))
    return out


# ---- prepared weights (src/prepared.rs) ------------------------------------------------------------------------------

class TensorInfo(ctypes.Structure):
    """gfr_tensor_info: one tensor view of a prepared model (the reference's prepared::Tensor, prepared.rs:32-41)."""
    _fields_ = [("storage", ctypes.c_int), ("dtype", ctypes.c_char * 24), ("rank", ctypes.c_int),
                ("shape", ctypes.c_uint64 * 8), ("stride", ctypes.c_uint64 * 8), ("off", ctypes.c_uint64),
                ("cuda", ctypes.c_int), ("extent_bytes", ctypes.c_uint64)]


def _u64s(xs):
    return (ctypes.c_uint64 * max(len(xs), 1))(*xs)


def sha256_hex(data: bytes) -> str:
    """The prepared format's chunk hash (FIPS 180-4 SHA-256), computed by the library."""
    out = ctypes.create_string_buffer(65)
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    _check(lib().gfr_sha256_hex(ctypes.addressof(buf), len(data), out))
    return out.value.decode()


def tensor_extent(dtype: str, shape, stride, off: int) -> int:
    """Tensor::extent (prepared.rs:51-71): bytes from the storage start past the view's last element."""
    out = ctypes.c_uint64()
    _check(lib().gfr_tensor_extent(dtype.encode(), _u64s(shape), _u64s(stride), len(shape), len(stride), off,
                                   ctypes.byref(out)))
    return out.value


class SharedFp8(_Engine):
    """The reference's FP8 shared expert (moe.rs:132-167: shared_gu, reduce8_bf16, shared_swiglu, shared_down) in
    two launches; gu [max_rows, 2 inter] and act [max_rows, inter] bf16 views of the last run's intermediates."""

    _destroy = "gfr_shared_fp8_destroy"

    def __init__(self, hidden: int, inter: int, max_rows: int, device="cuda"):
        super().__init__()
        _check(lib().gfr_shared_fp8_create(ctypes.byref(self._h), hidden, inter, max_rows))
        self.hidden, self.inter, self.max_rows = hidden, inter, max_rows
        self.gu = _view(lib().gfr_shared_fp8_gu(self._h), (max_rows, 2 * inter), torch.bfloat16, device)
        self.act = _view(lib().gfr_shared_fp8_act(self._h), (max_rows, inter), torch.bfloat16, device)

    def run(self, w: Fp8SharedWeights, input: torch.Tensor, rows: int, out: torch.Tensor = None, stream=None):
        """input [rows, >= hidden] bf16 -> out [rows, >= hidden] fp32 (allocated when None; returned)."""
        if input.dtype != torch.bfloat16:
            raise ValueError("input must be bf16 [rows, stride]")
        if out is None:
            out = torch.empty((rows, self.hidden), dtype=torch.float32, device=input.device)
        ws = w.struct()
        _check(lib().gfr_shared_fp8_run(self._h, _stream(stream), ctypes.byref(ws), _ptr(input), input.stride(0),
                                        rows, _ptr(out), out.stride(0)))
        return out


class Prepared(_Engine):
    """Prepared::open / tensor / expect / read_tensor / load_selected + Loaded::pointer (src/prepared.rs) over the
    library's loader. open and read_tensor need no GPU; load copies the selected storages into device memory."""

    _destroy = "gfr_prepared_destroy"

    def __init__(self, manifest_path: str):
        super().__init__()
        _check(lib().gfr_prepared_open(ctypes.byref(self._h), str(manifest_path).encode()))

    def names(self):
        L = lib()
        return [L.gfr_prepared_tensor_name(self._h, i).decode() for i in range(L.gfr_prepared_tensor_count(self._h))]

    def tensor(self, path: str) -> TensorInfo:
        info = TensorInfo()
        _check(lib().gfr_prepared_tensor(self._h, path.encode(), ctypes.byref(info)))
        return info

    def expect(self, path: str, dtype: str, shape):
        _check(lib().gfr_prepared_expect(self._h, path.encode(), dtype.encode(), _u64s(shape), len(shape)))

    def read_tensor(self, path: str, offset: int = 0, length: int = None) -> bytes:
        """read_tensor / read_tensor_segment: bytes of the view's extent past its start, from disk."""
        if length is None:
            t = self.tensor(path)
            eb = {"bool": 1, "uint8": 1, "int8": 1, "float8_e4m3fn": 1, "float8_e5m2": 1, "bfloat16": 2, "float16": 2,
                  "int16": 2, "uint16": 2, "float32": 4, "int32": 4, "uint32": 4, "float64": 8, "int64": 8,
                  "uint64": 8}[t.dtype.decode()]
            length = t.extent_bytes - t.off * eb - offset
        buf = ctypes.create_string_buffer(max(length, 1))
        _check(lib().gfr_prepared_read_tensor(self._h, path.encode(), offset, length, ctypes.addressof(buf)))
        return buf.raw[:length]

    def load(self, prefixes=()):
        arr = (ctypes.c_char_p * max(len(prefixes), 1))(*[p.encode() for p in prefixes])
        _check(lib().gfr_prepared_load(self._h, arr, len(prefixes)))
        b, s = ctypes.c_uint64(), ctypes.c_double()
        _check(lib().gfr_prepared_loaded(self._h, ctypes.byref(b), ctypes.byref(s)))
        return b.value, s.value

    def pointer(self, path: str) -> int:
        p = ctypes.c_void_p()
        _check(lib().gfr_prepared_pointer(self._h, path.encode(), ctypes.byref(p)))
        return p.value

    def experts(self, layer: int, device="cuda") -> Exl3Experts:
        """weights.layers[layer].moe.experts.* as an Exl3Experts of views into the loaded storages (no copy; valid
        while this object lives)."""
        st = _Exl3Struct()
        _check(lib().gfr_prepared_experts(self._h, layer, ctypes.byref(st)))
        E, D, N, b = st.experts, st.hidden, st.inter, st.bits
        _TYPESTR.setdefault(torch.int32, "<i4")
        v = lambda name, shape, dt: _view(getattr(st, name), shape, dt, device)
        return Exl3Experts(gt=v("gt", (E, D // 16, N // 16, 8 * b), torch.int32),
                           ut=v("ut", (E, D // 16, N // 16, 8 * b), torch.int32),
                           dt=v("dt", (E, N // 16, D // 16, 8 * b), torch.int32),
                           suh_g=v("suh_g", (E, D), torch.float16), suh_u=v("suh_u", (E, D), torch.float16),
                           suh_d=v("suh_d", (E, N), torch.float16), svh_g=v("svh_g", (E, N), torch.float16),
                           svh_u=v("svh_u", (E, N), torch.float16), svh_d=v("svh_d", (E, D), torch.float16), bits=b)


    def shared_fp8(self, layer: int, device="cuda") -> Fp8SharedWeights:
        """weights.layers[layer].moe.shared.* as Fp8SharedWeights of views into the loaded storages."""
        st = _Fp8Struct()
        _check(lib().gfr_prepared_shared_fp8(self._h, layer, ctypes.byref(st)))
        H, I = st.hidden, st.inter
        return Fp8SharedWeights(gu=_view(st.gu, (2 * I, H), torch.uint8, device),
                                gu_scale=_view(st.gu_scale, (2 * I,), torch.bfloat16, device),
                                down=_view(st.down, (H, I), torch.uint8, device),
                                down_scale=_view(st.down_scale, (H,), torch.bfloat16, device))


def write_prepared(directory: str, layers, chunk: int = 64 << 20, shared=None) -> str:
    """Write expert tensors in the reference's prepared format (src/prepared.rs:15-40): manifest.json + data.bin, one
    storage per tensor, tree weights.layers[L].moe.experts.{gt, ut, dt, suh_*, svh_*}, chunk hashes by hashlib.
    `layers`: a list of Exl3Experts (or dicts name -> numpy array). `shared`: optionally, per layer, the FP8 shared
    expert (Fp8SharedWeights or None) as weights.layers[L].moe.shared.{gu,down}.{weight,scale}. Returns the manifest
    path (for Prepared)."""
    import hashlib
    import json
    names = ("gt", "ut", "dt", "suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")
    os.makedirs(directory, exist_ok=True)
    data_path = os.path.join(directory, "data.bin")
    storages, nodes, off = [], [], 0
    hashes, pending = [], bytearray()
    with open(data_path, "wb") as f:
        def put(t):
            nonlocal off, pending
            if isinstance(t, torch.Tensor):
                dtype = {torch.int32: "int32", torch.float16: "float16", torch.bfloat16: "bfloat16",
                         torch.uint8: "float8_e4m3fn", torch.float8_e4m3fn: "float8_e4m3fn"}[t.dtype]
                arr = t.contiguous().view(torch.int16 if t.element_size() == 2 else
                                          torch.uint8 if t.element_size() == 1 else torch.int32).cpu().numpy()
            else:
                arr = t
                dtype = {"int32": "int32", "float16": "float16"}[str(arr.dtype)]
            blob = arr.tobytes()
            shape = list(arr.shape)
            stride, acc = [], 1
            for n in reversed(shape):
                stride.insert(0, acc)
                acc *= n
            node = {"T": len(storages), "dtype": dtype, "shape": shape, "stride": stride, "off": 0, "dev": "cuda"}
            storages.append({"offset": off, "nbytes": len(blob), "dev": "cuda"})
            f.write(blob)
            off += len(blob)
            pending += blob
            while len(pending) >= chunk:
                hashes.append(hashlib.sha256(bytes(pending[:chunk])).hexdigest())
                del pending[:chunk]
            return node

        for li, layer in enumerate(layers):
            fields = {name: put(layer[name] if isinstance(layer, dict) else getattr(layer, name)) for name in names}
            moe = {"experts": {"O": "Experts", "f": fields}}
            sw = shared[li] if shared is not None else None
            if sw is not None:
                moe["shared"] = {"O": "Shared", "f": {
                    "gu": {"O": "Fp8", "f": {"weight": put(sw.gu), "scale": put(sw.gu_scale)}},
                    "down": {"O": "Fp8", "f": {"weight": put(sw.down), "scale": put(sw.down_scale)}}}}
            nodes.append({"O": "Layer", "f": {"moe": {"O": "Moe", "f": moe}}})
    if pending:
        hashes.append(hashlib.sha256(bytes(pending)).hexdigest())
    manifest = {"format": 1, "file_size": off, "chunk": chunk, "chunk_sha256": hashes, "storages": storages,
                "tree": {"O": "Weights", "f": {"layers": {"L": nodes}}}, "key": {"rank": 0, "world": 1}}
    path = os.path.join(directory, "manifest.json")
    with open(path, "w") as f:
        json.dump(manifest, f)
    return path
