"""ctypes wrapper of the C byte oracle kvbytes.c (TEST INFRASTRUCTURE ONLY).

Every function takes CPU torch tensors and works on their bytes in place, so a test can run the
oracle on a CPU copy of exactly the pool the GPU kernel wrote and compare the two byte for byte.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"


class OCache(ctypes.Structure):
    _fields_ = [
        ("base", ctypes.c_void_p),
        ("num_pages", ctypes.c_int64),
        ("block", ctypes.c_int64),
        ("hkv", ctypes.c_int64),
        ("d", ctypes.c_int64),
        ("s_page", ctypes.c_int64),
        ("s_kv", ctypes.c_int64),
        ("s_row", ctypes.c_int64),
        ("s_head", ctypes.c_int64),
        ("elem_size", ctypes.c_int32),
        ("scale", ctypes.c_void_p),
    ]


_LIB: ctypes.CDLL | None = None


def build() -> Path:
    """make -C oracle (gcc)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIBRARY


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists() or LIBRARY.stat().st_mtime < (HERE / "kvbytes.c").stat().st_mtime:
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        p = ctypes.POINTER(OCache)
        lib.oracle_e4m3_encode.restype = ctypes.c_uint8
        lib.oracle_e4m3_encode.argtypes = [ctypes.c_float]
        lib.oracle_e4m3_decode.restype = ctypes.c_float
        lib.oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        lib.oracle_fp8_quantize.restype = ctypes.c_uint8
        lib.oracle_fp8_quantize.argtypes = [ctypes.c_float, ctypes.c_float]
        lib.oracle_e4m3_encode_array.argtypes = [vp, vp, i64]
        lib.oracle_e4m3_decode_array.argtypes = [vp, vp, i64]
        lib.oracle_kv_append_bytes.argtypes = [p, vp, vp, i64, i64, i64, i64, vp, i64]
        lib.oracle_kv_gather.argtypes = [p, vp, i64, i64, i64, vp, vp]
        lib.oracle_copy_blocks.argtypes = [p, vp, vp, i64]
        lib.oracle_kv_append_fp8.argtypes = [p, vp, vp, i64, i64, i64, i64, vp, i64, vp]
        _LIB = lib
    return _LIB


def _cache(kv_member: torch.Tensor, kv_scale: torch.Tensor | None = None) -> OCache:
    assert kv_member.device.type == "cpu" and kv_member.stride(-1) == 1
    pages, _, block, heads, dim = kv_member.shape
    s_page, s_kv, s_row, s_head, _ = kv_member.stride()
    scale = None
    if kv_scale is not None:
        assert kv_scale.dtype == torch.float32 and kv_scale.is_contiguous()
        scale = kv_scale.data_ptr()
    return OCache(kv_member.data_ptr(), pages, block, heads, dim, s_page, s_kv, s_row, s_head,
                  kv_member.element_size(), scale)


def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    """f32 -> e4m3fn bytes (uint8), round to nearest even."""
    x = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8)
    load().oracle_e4m3_encode_array(x.data_ptr(), out.data_ptr(), x.numel())
    return out


def e4m3_decode(q: torch.Tensor) -> torch.Tensor:
    q = q.contiguous().view(torch.uint8)
    out = torch.empty(q.shape, dtype=torch.float32)
    load().oracle_e4m3_decode_array(q.data_ptr(), out.data_ptr(), q.numel())
    return out


def fp8_quantize(x: float, reciprocal: float) -> int:
    """x quantized against a page scale s through its reciprocal r = 1 / s (0: s == 0)."""
    return int(load().oracle_fp8_quantize(x, reciprocal))


def kv_append(kv_member: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Same-dtype append, bytes copied (write_kv with k, v already in the cache dtype)."""
    assert k.dtype == kv_member.dtype == v.dtype
    k, v = k.contiguous(), v.contiguous()
    cache = _cache(kv_member)
    slots = slot_mapping.to(torch.int32).contiguous()
    load().oracle_kv_append_bytes(ctypes.byref(cache), k.data_ptr(), v.data_ptr(), k.stride(0),
                                  k.stride(1), v.stride(0), v.stride(1), slots.data_ptr(),
                                  k.shape[0])


def kv_gather(kv_member: torch.Tensor, block_table: torch.Tensor, width: int
              ) -> tuple[torch.Tensor, torch.Tensor]:
    pages, _, block, heads, dim = kv_member.shape
    table = block_table.to(torch.int32).contiguous()
    out_k = torch.empty(table.shape[0], width * block, heads, dim, dtype=kv_member.dtype)
    out_v = torch.empty_like(out_k)
    cache = _cache(kv_member)
    load().oracle_kv_gather(ctypes.byref(cache), table.data_ptr(), table.stride(0), table.shape[0],
                            width, out_k.data_ptr(), out_v.data_ptr())
    return out_k, out_v


def copy_blocks(kv_member: torch.Tensor, src: torch.Tensor, dst: torch.Tensor,
                kv_scale: torch.Tensor | None = None) -> None:
    s, d = src.to(torch.int32).contiguous(), dst.to(torch.int32).contiguous()
    cache = _cache(kv_member, kv_scale)
    load().oracle_copy_blocks(ctypes.byref(cache), s.data_ptr(), d.data_ptr(), s.numel())


def kv_append_fp8(kv_member: torch.Tensor, kv_scale: torch.Tensor, k: torch.Tensor,
                  v: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """The quantize-on-append rule on a CPU fp8 member (bytes) and its f32 scales, in place."""
    assert kv_member.dtype == torch.float8_e4m3fn
    k32, v32 = k.to(torch.float32).contiguous(), v.to(torch.float32).contiguous()
    cache = _cache(kv_member, kv_scale)
    slots = slot_mapping.to(torch.int32).contiguous()
    scratch = torch.empty(max(1, slots.numel()), dtype=torch.uint8)
    load().oracle_kv_append_fp8(ctypes.byref(cache), k32.data_ptr(), v32.data_ptr(),
                                k32.stride(0), k32.stride(1), v32.stride(0), v32.stride(1),
                                slots.data_ptr(), slots.numel(), scratch.data_ptr())
