"""The C-ABI library loads, exports every entry point include/dimmerkv.h declares, and its
argument validation fails with the reference's exception types before touching a GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import dkv_hip

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> list[str]:
    text = (ROOT / "include" / "dimmerkv.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_python_exports():
    assert set(declared_symbols()) == set(dkv_hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = dkv_hip.lib()
    missing = [name for name in declared_symbols() if not hasattr(lib, name)]
    assert not missing, missing
    assert lib.dkv_abi_version() == dkv_hip.ABI_VERSION


def test_validation_errors_map_to_reference_exceptions():
    lib = dkv_hip.lib()
    order = dkv_hip.Order(0, 0, None, None, None, None)
    rc = lib.dkv_pack_planes(None, None, None, None, ctypes.c_int32(4), order, None, None, None, None, None)
    assert rc == -2  # DKV_ESHAPE: bad order checked before anything runs
    assert b"bad order" in lib.dkv_last_error()
    with pytest.raises(ValueError):
        dkv_hip._check(rc, "dkv_pack_planes")
    rc = lib.dkv_topk(None, ctypes.c_int32(10), ctypes.c_int32(3), None, None, ctypes.c_size_t(0), None)
    assert rc == -1  # DKV_EINVAL: null pointer
    rc = lib.dkv_dequantize_codes(ctypes.c_void_p(8), ctypes.c_void_p(8), ctypes.c_void_p(8), ctypes.c_void_p(8),
                                  ctypes.c_int32(3), ctypes.c_int32(5), ctypes.c_int32(2), ctypes.c_void_p(8), None)
    assert rc == -2  # planes_rows must be 1 or n
    # centred token-matrix rows: cos without sin, rows outside the tokens (checked before any launch)
    vp = ctypes.c_void_p(8)
    rc = lib.dkv_centered_rows(vp, ctypes.c_int32(1), ctypes.c_int32(2), ctypes.c_int32(8), ctypes.c_int32(16),
                               ctypes.c_int32(64), vp, None, vp, ctypes.c_int32(0), ctypes.c_int32(16), vp, None)
    assert rc == -1 and b"cos and sin" in lib.dkv_last_error()
    rc = lib.dkv_centered_rows(vp, ctypes.c_int32(1), ctypes.c_int32(2), ctypes.c_int32(8), ctypes.c_int32(16),
                               ctypes.c_int32(64), None, None, vp, ctypes.c_int32(4), ctypes.c_int32(17), vp, None)
    assert rc == -2 and b"outside" in lib.dkv_last_error()
    with pytest.raises(AssertionError):
        dkv_hip._check(-5, "budget")
    with pytest.raises(RuntimeError):
        dkv_hip._check(-4, "launch")


def test_attend_argument_checks():
    lib = dkv_hip.lib()
    a = dkv_hip.AttendArgs()
    assert lib.dkv_attend_workspace_bytes(ctypes.byref(a)) == 0  # invalid -> 0 and an error message
    assert b"dkv_attend_workspace_bytes" in lib.dkv_last_error()
    assert lib.dkv_attend_layer(ctypes.byref(a), None, ctypes.c_size_t(0), None) in (-1, -2)


def test_cpu_tensors_are_refused():
    import torch

    with pytest.raises(ValueError, match="GPU"):
        dkv_hip.ptr(torch.zeros(3))


def test_centered_rows_refuses_wrong_tables_on_the_host():
    """dkv_centered_rows reads cos/sin as float32 [positions][head_dim] and mean as [L*H*D], and
    writes [end - start][L*H*D] floats: the binding refuses anything else before the kernel could
    read or write out of bounds (the half-width attention RoPE table, a short output, an fp16 mean)."""
    import torch

    layers, heads, tokens, dim = 2, 4, 40, 64
    caches = [torch.zeros(1, heads, tokens, dim, dtype=torch.float16) for _ in range(layers)]
    cos = torch.ones(tokens, dim)
    mean = torch.zeros(layers * heads * dim)
    out = torch.empty(30, layers * heads * dim)
    cases = [
        (dict(cos=cos[:, :dim // 2].contiguous(), sin=cos[:, :dim // 2].contiguous()), "cos must be"),
        (dict(cos=cos[:20], sin=cos[:20]), "cos must be"),
        (dict(sin=None), "give both cos and sin"),
        (dict(mean=mean.half()), "mean must be"),
        (dict(mean=mean[:-1]), "mean must be"),
        (dict(out=out[:-1]), "out must be"),
        (dict(out=out.t()), "out must be"),
        (dict(end=tokens + 1), "start <= end"),
    ]
    for change, message in cases:
        kw = dict(cos=cos, sin=cos, mean=mean, start=5, end=35, out=out)
        kw.update(change)
        if "end" in change:
            kw["out"] = torch.empty(kw["end"] - 5, layers * heads * dim)
        with pytest.raises(ValueError, match=message):
            dkv_hip.centered_rows(caches, kw["cos"], kw["sin"], kw["mean"], kw["start"], kw["end"], kw["out"])
    with pytest.raises(ValueError, match="caches must be"):
        dkv_hip.centered_rows([caches[0], caches[1][:, :2]], cos, cos, mean, 5, 35, out)
    # well-formed host tensors get past the checks and are refused as host memory
    with pytest.raises(ValueError, match="GPU"):
        dkv_hip.centered_rows(caches, cos, cos, mean, 5, 35, out)


def test_noalloc_refuses_contexts_beyond_its_static_workspace():
    """A 3B-shaped context of 100,000 compressed tokens needs far more than the static workspace:
    refused by the host-side checks, before any device work."""
    lib = dkv_hip.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check comes first
    order = dkv_hip.Order(32, 256, fake, fake, fake, fake)
    stream = dkv_hip.Stream(fake, fake, fake, order, dkv_hip.DKV_FMT_PLANES, dkv_hip.Ladder())
    cu_host = (ctypes.c_int32 * 2)(0, 100_000)
    a = dkv_hip.AttendArgs()
    a.batch, a.q_len, a.layers, a.layer, a.kv_heads, a.head_dim, a.q_heads, a.rank = 1, 1, 28, 0, 8, 128, 24, 2048
    a.scaling = 128 ** -0.5
    a.key, a.value = stream, stream
    a.cu_seqlens = a.positions = a.key_basis = a.value_basis = a.mean_k = a.mean_v = 256
    a.rope_cos = a.rope_sin = a.query = a.out = 256
    a.rope_rows = 100_001
    a.cu_seqlens_host = ctypes.cast(cu_host, ctypes.c_void_p).value
    assert lib.dkv_attend_workspace_bytes(ctypes.byref(a)) > dkv_hip.NOALLOC_MAX_BYTES
    rc = lib.dkv_attend_layer_noalloc(ctypes.byref(a), None)
    assert rc == -3  # DKV_EWORKSPACE
    assert b"static maximum" in lib.dkv_last_error()


def test_prepare_refuses_stream_tables_beyond_the_decode_lds_column():
    """The decode kernels stage one group's column of the stream table in LDS; a ladder with more
    rungs than that column holds is refused before any launch."""
    lib = dkv_hip.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: refused before any device work
    ladder = dkv_hip.Ladder(32, 5000, fake, fake, fake)
    stream = dkv_hip.Stream(fake, fake, fake, dkv_hip.Order(), dkv_hip.DKV_FMT_LADDER, ladder)
    cu_host = (ctypes.c_int32 * 2)(0, 1000)
    a = dkv_hip.AttendArgs()
    a.batch, a.q_len, a.layers, a.layer, a.kv_heads, a.head_dim, a.q_heads, a.rank = 1, 1, 28, 0, 8, 128, 24, 2048
    a.scaling = 128 ** -0.5
    a.key, a.value = stream, stream
    a.cu_seqlens = a.positions = a.key_basis = a.value_basis = a.mean_k = a.mean_v = 256
    a.rope_cos = a.rope_sin = a.query = a.out = 256
    a.rope_rows = 1001
    a.cu_seqlens_host = ctypes.cast(cu_host, ctypes.c_void_p).value
    need = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
    assert need > 0
    rc = lib.dkv_attend_prepare(ctypes.byref(a), ctypes.c_int32(8), fake, ctypes.c_size_t(need), None)
    assert rc == -2 and b"table has 5000 rows" in lib.dkv_last_error()


def test_layer_refuses_bad_exact_dtype_and_misaligned_exact_tokens():
    """exact_dtype must be DKV_F32, DKV_F16 or DKV_BF16, and the exact keys / values aligned for the
    kernels' four-element loads (16 bytes for f32, 8 for the 16-bit types): refused on the host before
    any device work."""
    lib = dkv_hip.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: refused before any device work
    order = dkv_hip.Order(32, 256, fake, fake, fake, fake)
    stream = dkv_hip.Stream(fake, fake, fake, order, dkv_hip.DKV_FMT_PLANES, dkv_hip.Ladder())
    cu_host = (ctypes.c_int32 * 2)(0, 1000)
    ex_host = (ctypes.c_int32 * 2)(0, 37)
    a = dkv_hip.AttendArgs()
    a.batch, a.q_len, a.layers, a.layer, a.kv_heads, a.head_dim, a.q_heads, a.rank = 1, 1, 28, 0, 8, 128, 24, 2048
    a.scaling = 128 ** -0.5
    a.key, a.value = stream, stream
    a.cu_seqlens = a.positions = a.key_basis = a.value_basis = a.mean_k = a.mean_v = 256
    a.rope_cos = a.rope_sin = a.query = a.out = 256
    a.rope_rows = 1001
    a.cu_seqlens_host = ctypes.cast(cu_host, ctypes.c_void_p).value
    a.cu_exact, a.cu_exact_host = 256, ctypes.cast(ex_host, ctypes.c_void_p).value
    a.key_exact = a.value_exact = 512
    a.exact_dtype = 7
    assert lib.dkv_attend_layer(ctypes.byref(a), None, ctypes.c_size_t(0), None) == -1  # DKV_EINVAL
    assert b"exact_dtype 7" in lib.dkv_last_error()
    a.exact_dtype, a.key_exact = 0, 520  # f32 needs 16-byte alignment
    assert lib.dkv_attend_layer(ctypes.byref(a), None, ctypes.c_size_t(0), None) == -1
    assert b"16-byte aligned" in lib.dkv_last_error()
    a.exact_dtype, a.value_exact = 1, 514  # f16 needs 8
    assert lib.dkv_attend_layer(ctypes.byref(a), None, ctypes.c_size_t(0), None) == -1
    assert b"8-byte aligned" in lib.dkv_last_error()
