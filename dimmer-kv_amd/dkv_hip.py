"""ctypes binding of libdimmerkv_hip.so (the C ABI declared in include/dimmerkv.h).

The library is loaded from this directory.  There is no fallback: if the
library is missing, or a tensor is not on a GPU, the call raises.  Return
codes map to the reference's exception types (scripts/kvtc.py:226-227,
289-290 ValueError; scripts/progressive.py:189-190 AssertionError;
scripts/methods.py:136-137 RuntimeError).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libdimmerkv_hip.so"
ABI_VERSION = 3

DKV_F32, DKV_F16, DKV_BF16 = 0, 1, 2
DKV_FMT_PLANES, DKV_FMT_LADDER = 0, 1
_DTYPE = {torch.float32: DKV_F32, torch.float16: DKV_F16, torch.bfloat16: DKV_BF16}

EXPORTS = [
    "dkv_abi_version", "dkv_last_error", "dkv_pack_planes", "dkv_pack_ladder", "dkv_unpack_dequant", "dkv_dequantize_codes",
    "dkv_prepare_key_basis", "dkv_prepare_value_basis", "dkv_attend_workspace_bytes", "dkv_attend_prepare",
    "dkv_attend_layer",
    "dkv_attend_scores", "dkv_attend_values",
    "dkv_score_workspace_bytes", "dkv_score_begin", "dkv_score_layer", "dkv_topk_workspace_bytes", "dkv_topk",
    "dkv_gather_cold", "dkv_refine_rows", "dkv_wire_pack", "dkv_wire_unpack", "dkv_attend_layer_noalloc",
    "dkv_quantize8", "dkv_centered_rows",
]
NOALLOC_MAX_BYTES = 64 << 20  # DKV_NOALLOC_MAX_BYTES: the static workspace of dkv_attend_layer_noalloc

c_i32, c_i64, c_f32, c_vp, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t


class Order(ctypes.Structure):
    _fields_ = [("groups", c_i32), ("pieces", c_i32), ("planes", c_vp), ("seg_off", c_vp), ("cold_off", c_vp),
                ("prefix_bytes", c_vp)]


class Ladder(ctypes.Structure):
    _fields_ = [("groups", c_i32), ("rungs", c_i32), ("bits", c_vp), ("seg_off", c_vp), ("rung_bytes", c_vp)]


class Stream(ctypes.Structure):
    _fields_ = [("blob", c_vp), ("tok_off", c_vp), ("pieces", c_vp), ("order", Order), ("format", c_i32),
                ("ladder", Ladder)]


class Wire(ctypes.Structure):
    """Where each (rung, width) section of the byte-storage layout lies (dkv_wire_t)."""
    _fields_ = [("section", c_vp), ("count", c_vp), ("rank", c_vp), ("slot", c_vp), ("nwidth", c_vp),
                ("bytes", c_i64)]


class AttendArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("q_len", c_i32),
        ("layers", c_i32), ("layer", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32), ("q_heads", c_i32),
        ("rank", c_i32),
        ("scaling", c_f32),
        ("key", Stream), ("value", Stream),
        ("cu_seqlens", c_vp), ("cu_seqlens_host", c_vp), ("positions", c_vp),
        ("key_basis", c_vp), ("value_basis", c_vp), ("mean_k", c_vp), ("mean_v", c_vp),
        ("rope_cos", c_vp), ("rope_sin", c_vp), ("rope_rows", c_i32),
        ("query", c_vp), ("query_dtype", c_i32),
        ("cu_exact", c_vp), ("cu_exact_host", c_vp), ("key_exact", c_vp), ("value_exact", c_vp), ("mask", c_vp),
        ("out", c_vp), ("out_dtype", c_i32), ("exact_dtype", c_i32),
    ]


class DkvError(RuntimeError):
    pass


_lib = None


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise loudly if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(python dimmer-kv_amd/build_lib.py); there is no CPU fallback")
        handle = ctypes.CDLL(str(LIB_PATH))
        handle.dkv_abi_version.restype = c_i32
        handle.dkv_last_error.restype = ctypes.c_char_p
        for name in ("dkv_attend_workspace_bytes", "dkv_score_workspace_bytes", "dkv_topk_workspace_bytes"):
            getattr(handle, name).restype = c_sz
        handle.dkv_topk_workspace_bytes.argtypes = [c_i32]
        if handle.dkv_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {handle.dkv_abi_version()}, expected {ABI_VERSION}")
        _lib = handle
    return _lib


def _check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = f"{what}: {lib().dkv_last_error().decode()} (code {rc})"
    if rc in (-1, -2):
        raise ValueError(msg)
    if rc == -5:
        raise AssertionError(msg)
    raise DkvError(msg)


def addr(t: torch.Tensor) -> int:
    """Address of ``t``'s first element.  torch reports 0 for every empty tensor; an empty view of an
    allocation gets the address its storage gives it, so arrays of zero tokens still pass the C ABI's
    non-null checks (nothing is read through them)."""
    if t.numel():
        return t.data_ptr()
    return t.untyped_storage().data_ptr() + t.storage_offset() * t.element_size()


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("dimmer-kv HIP kernels need GPU tensors (no CPU path)")
    if not t.is_contiguous():
        raise ValueError("dimmer-kv HIP kernels need contiguous tensors")
    return addr(t)


try:  # the raw handle of the current stream, without a Python stream object per call
    from torch._C import _cuda_getCurrentRawStream as _raw_stream, _cuda_getDevice as _current_device
except ImportError:  # pragma: no cover - older torch
    _raw_stream = _current_device = None


def stream_handle() -> int:
    """The current HIP stream of the current device (what torch.cuda.current_stream().cuda_stream gives)."""
    if _raw_stream is not None:
        return _raw_stream(_current_device())
    return torch.cuda.current_stream().cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in _DTYPE:
        raise ValueError(f"unsupported dtype {dtype}")
    return _DTYPE[dtype]


# ----------------------------------------------------------------- wrappers

def pack_planes(codes, low, span, pieces, order: Order, hot, hot_off, cold=None, cold_off=None) -> None:
    n = codes.shape[0]
    _check(lib().dkv_pack_planes(c_vp(ptr(codes)), c_vp(ptr(low)), c_vp(ptr(span)), c_vp(ptr(pieces)), c_i32(n),
                                 order, c_vp(ptr(hot)), c_vp(ptr(hot_off)), c_vp(ptr(cold)), c_vp(ptr(cold_off)),
                                 c_vp(stream_handle())), "dkv_pack_planes")


def pack_ladder(codes, low, scale, rung, ladder: Ladder, blob, tok_off) -> None:
    n = codes.shape[0]
    _check(lib().dkv_pack_ladder(c_vp(ptr(codes)), c_vp(ptr(low)), c_vp(ptr(scale)), c_vp(ptr(rung)), c_i32(n),
                                 ladder, c_vp(ptr(blob)), c_vp(ptr(tok_off)), c_vp(stream_handle())),
           "dkv_pack_ladder")


def wire_pack(codes, low, scale, rung, ladder: Ladder, wire: Wire, out) -> None:
    """codes u8 [n, G, 64], shifts/scales (int16 views of fp16) [n, G], rung int16 [n] -> storage sections."""
    _check(lib().dkv_wire_pack(c_vp(ptr(codes)), c_vp(ptr(low)), c_vp(ptr(scale)), c_vp(ptr(rung)),
                               c_i32(rung.numel()), ladder, wire, c_vp(ptr(out)), c_vp(stream_handle())),
           "dkv_wire_pack")


def wire_unpack(data, rung, ladder: Ladder, wire: Wire, codes, low, scale) -> None:
    """Storage sections -> codes u8 [n, G, 64], shifts/scales (int16 views of fp16) [n, G]."""
    _check(lib().dkv_wire_unpack(c_vp(ptr(data)), c_vp(ptr(rung)), c_i32(rung.numel()), ladder, wire,
                                 c_vp(ptr(codes)), c_vp(ptr(low)), c_vp(ptr(scale)), c_vp(stream_handle())),
           "dkv_wire_unpack")


def unpack_dequant(stream: Stream, t0: int, nt: int, out: torch.Tensor) -> None:
    _check(lib().dkv_unpack_dequant(ctypes.byref(stream), c_i32(t0), c_i32(nt), c_vp(ptr(out)),
                                    c_i32(dtype_code(out.dtype)), c_vp(stream_handle())), "dkv_unpack_dequant")


def centered_rows(tensors, cos, sin, mean, start: int, end: int, out) -> None:
    """Per-layer caches [1, H, T, D] (fp16/bf16/fp32, one device) -> out f32 [end - start, L*H*D]:
    the token-matrix rows start..end - 1 minus ``mean``, keys de-rotated when cos/sin are given."""
    first = tensors[0]
    if first.dtype not in _DTYPE:
        raise ValueError(f"centered_rows: cache dtype {first.dtype} not supported")
    if first.dim() != 4 or first.shape[0] != 1:
        raise ValueError(f"centered_rows: caches must be [1, heads, tokens, head_dim] (got {tuple(first.shape)})")
    if any(t.shape != first.shape or t.dtype != first.dtype or t.device != first.device or not t.is_contiguous()
           for t in tensors):
        raise ValueError("centered_rows: the layers' caches must be contiguous and share shape, dtype and device")
    _, heads, tokens, head_dim = first.shape
    width = len(tensors) * heads * head_dim
    if not 0 <= start <= end <= tokens:
        raise ValueError(f"centered_rows: need 0 <= start <= end <= {tokens} (got {start}, {end})")

    def need(t, name, ok_shape, want):
        if (t is None or t.dtype != torch.float32 or t.device != first.device or not t.is_contiguous()
                or not ok_shape(tuple(t.shape))):
            got = "None" if t is None else f"{t.dtype} {tuple(t.shape)} on {t.device}"
            raise ValueError(f"centered_rows: {name} must be a contiguous float32 tensor {want} on {first.device} "
                             f"(got {got})")

    if (cos is None) != (sin is None):
        raise ValueError("centered_rows: give both cos and sin (keys) or neither (values)")
    if cos is not None:
        for t, name in ((cos, "cos"), (sin, "sin")):
            need(t, name, lambda sh: len(sh) == 2 and sh[0] >= end and sh[1] == head_dim,
                 f"[>= {end} positions, {head_dim}]")
    need(mean, "mean", lambda sh: sh == (width,), f"[{width}]")
    need(out, "out", lambda sh: sh == (end - start, width), f"[{end - start}, {width}]")
    ptrs = torch.tensor([ptr(t) for t in tensors], dtype=torch.int64).to(first.device)
    _check(lib().dkv_centered_rows(c_vp(ptr(ptrs)), c_i32(_DTYPE[first.dtype]), c_i32(len(tensors)), c_i32(heads),
                                   c_i32(tokens), c_i32(head_dim), c_vp(ptr(cos)), c_vp(ptr(sin)), c_vp(ptr(mean)),
                                   c_i32(start), c_i32(end), c_vp(ptr(out)), c_vp(stream_handle())),
           "dkv_centered_rows")


def quantize8(coef, codes, low, span, errors=None) -> None:
    """coef f32 [n, 64G] -> codes u8 [n, G, 64], low/span f16 bits [n, G], errors f32 [n, G, 9] or None."""
    n, groups = codes.shape[0], codes.shape[1]
    _check(lib().dkv_quantize8(c_vp(ptr(coef)), c_i32(n), c_i32(groups), c_vp(ptr(codes)), c_vp(ptr(low)),
                               c_vp(ptr(span)), c_vp(ptr(errors)), c_vp(stream_handle())), "dkv_quantize8")


def dequantize_codes(codes, low, span, planes, out) -> None:
    n, groups = codes.shape[0], codes.shape[1]
    _check(lib().dkv_dequantize_codes(c_vp(ptr(codes)), c_vp(ptr(low)), c_vp(ptr(span)), c_vp(ptr(planes)),
                                      c_i32(planes.shape[0]), c_i32(n), c_i32(groups), c_vp(ptr(out)),
                                      c_vp(stream_handle())), "dkv_dequantize_codes")


def prepare_key_basis(basis, layers, kv_heads, head_dim, rank, out) -> None:
    _check(lib().dkv_prepare_key_basis(c_vp(ptr(basis)), c_i32(layers), c_i32(kv_heads), c_i32(head_dim),
                                       c_i32(rank), c_vp(ptr(out)), c_vp(stream_handle())), "dkv_prepare_key_basis")


def prepare_value_basis(basis, layers, kv_heads, head_dim, rank, out) -> None:
    _check(lib().dkv_prepare_value_basis(c_vp(ptr(basis)), c_i32(layers), c_i32(kv_heads), c_i32(head_dim),
                                         c_i32(rank), c_vp(ptr(out)), c_vp(stream_handle())),
           "dkv_prepare_value_basis")


def attend_workspace_bytes(args: AttendArgs) -> int:
    n = lib().dkv_attend_workspace_bytes(ctypes.byref(args))
    if n == 0:
        _check(-2, "dkv_attend_workspace_bytes")
    return n


def attend_prepare(args: AttendArgs, workspace: torch.Tensor, plane_cap: int = 8, values: bool = True) -> None:
    """K1 into the workspace: every token's key codes decoded (to ``plane_cap`` planes) for K2, and
    the value codes for K3 unless ``values`` is False (question scoring reads keys only)."""
    if not values:
        args = AttendArgs.from_buffer_copy(args)
        args.value = Stream()  # no value blob: the library decodes the keys alone
    _check(lib().dkv_attend_prepare(ctypes.byref(args), c_i32(plane_cap), c_vp(ptr(workspace)),
                                    c_sz(workspace.numel()), c_vp(stream_handle())), "dkv_attend_prepare")


def attend_layer(args: AttendArgs, workspace: torch.Tensor) -> None:
    _check(lib().dkv_attend_layer(ctypes.byref(args), c_vp(ptr(workspace)), c_sz(workspace.numel()),
                                  c_vp(stream_handle())), "dkv_attend_layer")


def attend_layer_noalloc(args: AttendArgs) -> None:
    """K1 decode + one layer with the library's static workspace (no allocation anywhere, for
    callers that cannot allocate).  Contexts whose workspace exceeds NOALLOC_MAX_BYTES are refused;
    calls that overlap on one GPU share that workspace and race."""
    _check(lib().dkv_attend_layer_noalloc(ctypes.byref(args), c_vp(stream_handle())), "dkv_attend_layer_noalloc")


def attend_scores(args: AttendArgs, workspace: torch.Tensor) -> None:
    _check(lib().dkv_attend_scores(ctypes.byref(args), c_vp(ptr(workspace)), c_sz(workspace.numel()),
                                   c_vp(stream_handle())), "dkv_attend_scores")


def attend_values(args: AttendArgs, workspace: torch.Tensor) -> None:
    _check(lib().dkv_attend_values(ctypes.byref(args), c_vp(ptr(workspace)), c_sz(workspace.numel()),
                                   c_vp(stream_handle())), "dkv_attend_values")


def score_workspace_bytes(args: AttendArgs) -> int:
    n = lib().dkv_score_workspace_bytes(ctypes.byref(args))
    if n == 0:
        _check(-2, "dkv_score_workspace_bytes")
    return n


def score_begin(importance: torch.Tensor) -> None:
    _check(lib().dkv_score_begin(c_vp(ptr(importance)), c_i32(importance.numel()), c_vp(stream_handle())),
           "dkv_score_begin")


def score_layer(args: AttendArgs, key_question: torch.Tensor, importance: torch.Tensor,
                workspace: torch.Tensor) -> None:
    _check(lib().dkv_score_layer(ctypes.byref(args), c_vp(ptr(key_question)), c_vp(ptr(importance)),
                                 c_vp(ptr(workspace)), c_sz(workspace.numel()), c_vp(stream_handle())),
           "dkv_score_layer")


def topk(scores: torch.Tensor, k: int, out: torch.Tensor) -> None:
    _check(lib().dkv_topk(c_vp(ptr(scores)), c_i32(scores.numel()), c_i32(k), c_vp(ptr(out)), c_vp(None), c_sz(0),
                          c_vp(stream_handle())), "dkv_topk")


def refine_rows(stream: Stream, n: int, cold, cold_tok_off, rows, refined_base_off: int, blob, tok_off, pieces,
                owner, version: int, fetched) -> None:
    """K4c over any token list on the device (dkv_refine_rows): ``fetched`` [2] int64, zero on entry,
    gets the reference's byte count and the out-of-range flag."""
    k = rows.numel()
    refined_ptr = ptr(blob) + refined_base_off
    _check(lib().dkv_refine_rows(ctypes.byref(stream), c_i32(n), c_vp(ptr(cold)), c_vp(ptr(cold_tok_off)),
                                 c_vp(ptr(rows)), c_i32(k), c_vp(refined_ptr), c_i64(refined_base_off),
                                 c_vp(ptr(tok_off)), c_vp(ptr(pieces)), c_vp(ptr(owner)), c_i32(version),
                                 c_vp(ptr(fetched)), c_vp(stream_handle())), "dkv_refine_rows")


def gather_cold(stream: Stream, cold, cold_tok_off, idx, refined_base_off: int, blob, tok_off, pieces) -> None:
    k = idx.numel()
    refined_ptr = ptr(blob) + refined_base_off
    _check(lib().dkv_gather_cold(ctypes.byref(stream), c_vp(ptr(cold)), c_vp(ptr(cold_tok_off)), c_vp(ptr(idx)),
                                 c_i32(k), c_vp(refined_ptr), c_i64(refined_base_off), c_vp(ptr(tok_off)),
                                 c_vp(ptr(pieces)), c_vp(stream_handle())), "dkv_gather_cold")
