"""MI355X (gfx950) quantized-matmul hot path of the MiniCPM-V 4.6 engine.

Python host mirror of the reference's C++ operator surface
(src/csrc/include/minicpmv/ops.h:95-126, quantized_weight.h:11-28) over the
C-ABI in include/mcv_quant.h.  torch supplies device memory and streams only;
every operator runs a hand-written HIP kernel from lib/libmcv_quant.so and
fails loudly (McvError) when that library is missing or the device is not a
gfx950.  There is no CPU fallback.

The directory name is not a Python identifier; load it with ``load()`` from
``__graft_entry__`` or ``importlib`` (see tests/conftest.py).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libmcv_quant.so"
GROUP = 128
SLAB = 64

MCV_F32, MCV_F16 = 0, 1
W8_KN, W8_NK, W8_TILED = 0, 1, 2
SRC_F16, SRC_BF16 = 0, 1

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_vp = ctypes.c_void_p


class McvError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero status (`status`, one of
    the mcv_status codes; None for an error raised in Python)."""

    status: Optional[int] = None


MCV_ERR_UNSUPPORTED = 4


_LIB: Optional[ctypes.CDLL] = None


class _W4Part(ctypes.Structure):
    """mcv_w4a16_part (include/mcv_quant.h)."""
    _fields_ = [("qw", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("zeros", ctypes.c_void_p),
                ("zero_bias", ctypes.c_int), ("N", ctypes.c_int64), ("out", ctypes.c_void_p)]

# name -> (restype, argtypes) for every entry point of include/mcv_quant.h
_SIGS = {
    "mcv_last_error": (ctypes.c_char_p, []),
    "mcv_version": (ctypes.c_char_p, []),
    "mcv_w4a16_packed_weight_bytes": (_c_i64, [_c_i64, _c_i64]),
    "mcv_w4a16_packed_scale_bytes": (_c_i64, [_c_i64, _c_i64]),
    "mcv_w4a16_packed_zero_bytes": (_c_i64, [_c_i64, _c_i64]),
    "mcv_w4a16_pack_awq": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp]),
    "mcv_w4a16_pack_gptq": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp]),
    "mcv_w4a16_dequant_gptq_host": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "mcv_w4a16_quantize_host": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_int]),
    "mcv_w4a16_quantize_nk_host": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int]),
    "mcv_w4a16_unpack_host": (_c_int, [_vp, _vp, _vp, _c_int, _c_i64, _c_i64, _vp, _vp, _vp]),
    "mcv_w4a16_gemm": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp]),
    "mcv_w4a16_gemm_ws": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp, _c_i64, _vp]),
    "mcv_w4a16_gemm_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "mcv_w4a16_gemm_kernel_name": (ctypes.c_char_p, [_c_i64, _c_i64, _c_i64, _c_int]),
    "mcv_w8a8_gemm_kernel_name": (ctypes.c_char_p, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "mcv_w4a16_gemm_sk_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_int, _c_int, _c_int]),
    "mcv_w4a16_gemm_sk": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int,
                                   _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _c_i64, _vp]),
    "mcv_w4a16_gemv": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp]),
    "mcv_w4a16_gemm_mfma": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp]),
    "mcv_w4a16_dequant": (_c_int, [_vp, _vp, _vp, _c_int, _c_i64, _c_i64, _vp, _vp, _vp]),
    "mcv_w4a16_gate_up_silu": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _c_int, _vp,
                                        _vp]),
    "mcv_w4a16_gemv_multi": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_int, _vp]),
    "mcv_w4a16_mlp_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "mcv_w4a16_mlp": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _c_int,
                               _vp, _vp, _vp, _vp]),
    "mcv_w4a16_gemv_tiled_i8": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
    "mcv_lm_head_workspace_bytes": (_c_i64, [_c_i64]),
    "mcv_lm_head_slabs_per_workgroup": (_c_i64, [_c_i64]),
    "mcv_w4a16_lm_head_argmax": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp,
                                          _vp]),
    "mcv_lm_head_noalloc_max_vocab": (_c_i64, []),
    "mcv_testing_lm_head_skew_poll": (None, [_c_int]),
    "mcv_w4a16_lm_head_argmax_noalloc": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp, _vp,
                                                  _vp]),
    "mcv_lm_head_slots_bytes": (_c_i64, []),
    "mcv_w4a16_lm_head_argmax_slots": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp,
                                                ctypes.c_uint32, _vp]),
    "mcv_lm_head_slots_token": (_c_i64, [_vp, ctypes.c_uint32]),
    "mcv_w4a16_gemv_argmax_partials": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_int, _vp, _vp, _vp]),
    "mcv_argmax_reduce_keys": (_c_int, [_vp, _c_i64, _vp, _vp]),
    "mcv_w8a8_quantize_act": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
    "mcv_w8a8_gemm_i32": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp, _vp]),
    "mcv_w8a8_dequant": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_i64, _c_i64, _vp, _vp]),
    "mcv_w8a8_gemm_f16": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp, _c_int, _vp, _vp]),
    "mcv_w8a8_gemm_lds": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int,
                                   _c_int, _c_int, _vp]),
    "mcv_w8a8_gemv_argmax_partials": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_int, _vp, _vp,
                                               _vp]),
    "mcv_w8a8_lm_head_slabs_per_workgroup": (_c_i64, [_c_i64]),
    "mcv_w8a8_lm_head_argmax": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp,
                                         _vp]),
    "mcv_w8a8_quantize_weight_host": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_int, _vp, _vp]),
    "mcv_w8a8_tiled_bytes": (_c_i64, [_c_i64, _c_i64]),
    "mcv_w8a8_gate_up_silu": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _c_int, _vp,
                                       _vp]),
    "mcv_w8a8_pack_tiled_host": (_c_int, [_vp, _c_i64, _c_i64, _vp]),
    "mcv_w8a8_mlp_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "mcv_w8a8_mlp": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp]),
    "mcv_w8a8_quantize_weight_nk_host": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_int, _vp, _vp]),
    "mcv_w8a8_quantize_weight_nk_pad_host": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp, _vp]),
    "mcv_w8a8_pack_tiled_nk_host": (_c_int, [_vp, _c_i64, _c_i64, _vp]),
    "mcv_silu_mul": (_c_int, [_vp, _vp, _vp, _c_i64, _vp]),
    "mcv_argmax_f16": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp]),
    "mcv_rms_norm": (_c_int, [_vp, _vp, _c_i64, _c_i64, ctypes.c_double, _vp, _vp]),
    "mcv_rms_norm_w8a8_quantize": (_c_int, [_vp, _vp, _c_i64, _c_i64, ctypes.c_double, _vp, _vp, _vp, _vp, _vp]),
}


def lib() -> ctypes.CDLL:
    """The loaded C-ABI library; raises McvError if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise McvError(f"HIP library not built: {LIB_PATH} is missing (run __graft_entry__.build())")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc != 0:
        e = McvError(f"{what} failed (status {rc}): {lib().mcv_last_error().decode()}")
        e.status = rc
        raise e


def _np_ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "host arrays must be C-contiguous"
    return a.ctypes.data


# --------------------------------------------------------------------------- #
# host-side packing / quantisation (numpy in, numpy out)                       #
# --------------------------------------------------------------------------- #
def packed_sizes(K: int, N: int) -> tuple[int, int, int]:
    L = lib()
    return (L.mcv_w4a16_packed_weight_bytes(K, N), L.mcv_w4a16_packed_scale_bytes(K, N),
            L.mcv_w4a16_packed_zero_bytes(K, N))


def _alloc_packed(K: int, N: int):
    wb, sb, zb = packed_sizes(K, N)
    if wb == 0:
        raise McvError(f"bad W4A16 shape K={K} N={N} (K must be a positive multiple of 128)")
    return np.empty(wb, np.uint8), np.empty(sb // 2, np.uint16), np.empty(zb // 4, np.uint32)


def pack_awq(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray):
    """AutoAWQ gemm tensors -> slab-64 (qw bytes, scales [G][Npad] u16, zeros [G][Npad/8] u32)."""
    qweight = np.ascontiguousarray(qweight, np.int32)
    qzeros = np.ascontiguousarray(qzeros, np.int32)
    scales = np.ascontiguousarray(scales).view(np.uint16)
    K, N = qweight.shape[0], qweight.shape[1] * 8
    qw, sc, zr = _alloc_packed(K, N)
    _check(lib().mcv_w4a16_pack_awq(_np_ptr(qweight), _np_ptr(qzeros), _np_ptr(scales), K, N, _np_ptr(qw),
                                    _np_ptr(sc), _np_ptr(zr)), "mcv_w4a16_pack_awq")
    return qw, sc, zr


def pack_gptq(qweight: np.ndarray, qzeros: np.ndarray, g_idx: Optional[np.ndarray], scales: np.ndarray):
    """GPTQ v1 tensors -> slab-64 (zero_bias 1)."""
    qweight = np.ascontiguousarray(qweight, np.int32)
    qzeros = np.ascontiguousarray(qzeros, np.int32)
    scales = np.ascontiguousarray(scales).view(np.uint16)
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    groups = scales.shape[0]
    gp = 0
    if g_idx is not None:
        g_idx = np.ascontiguousarray(g_idx, np.int32)
        gp = _np_ptr(g_idx)
    qw, sc, zr = _alloc_packed(K, N)
    _check(lib().mcv_w4a16_pack_gptq(_np_ptr(qweight), _np_ptr(qzeros), gp, _np_ptr(scales), K, N, groups,
                                     _np_ptr(qw), _np_ptr(sc), _np_ptr(zr)), "mcv_w4a16_pack_gptq")
    return qw, sc, zr


def dequant_gptq(qweight: np.ndarray, qzeros: np.ndarray, g_idx: Optional[np.ndarray], scales: np.ndarray):
    """GPTQ v1 tensors -> the dense fp16 weight [K][N] (u16 bits), RNE((q -
    zero[g_idx[k]]) * scale[k/128]): for act-order weights pack_gptq refuses."""
    qweight = np.ascontiguousarray(qweight, np.int32)
    qzeros = np.ascontiguousarray(qzeros, np.int32)
    scales = np.ascontiguousarray(scales).view(np.uint16)
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    gp = 0
    if g_idx is not None:
        g_idx = np.ascontiguousarray(g_idx, np.int32)
        gp = _np_ptr(g_idx)
    w = np.empty((K, N), np.uint16)
    _check(lib().mcv_w4a16_dequant_gptq_host(_np_ptr(qweight), _np_ptr(qzeros), gp, _np_ptr(scales), K, N,
                                             scales.shape[0], _np_ptr(w)), "mcv_w4a16_dequant_gptq_host")
    return w


def unpack(qw: np.ndarray, scales: np.ndarray, zeros: np.ndarray, zero_bias: int, K: int, N: int):
    """slab-64 -> (q [K][N] u8, effective zero [G][N] u8, scales [G][N] u16)."""
    q = np.empty((K, N), np.uint8)
    z = np.empty((K // GROUP, N), np.uint8)
    s = np.empty((K // GROUP, N), np.uint16)
    _check(lib().mcv_w4a16_unpack_host(_np_ptr(np.ascontiguousarray(qw)), _np_ptr(np.ascontiguousarray(scales)),
                                       _np_ptr(np.ascontiguousarray(zeros)), zero_bias, K, N, _np_ptr(q), _np_ptr(z),
                                       _np_ptr(s)), "mcv_w4a16_unpack_host")
    return q, z, s


def quantize_int4(w_kn_f16: np.ndarray, nthreads: int = 0):
    """Build-defined synthetic int4 quantiser -> AutoAWQ (qweight, qzeros, scales u16)."""
    w = np.ascontiguousarray(w_kn_f16).view(np.uint16)
    K, N = w.shape
    qweight = np.empty((K, N // 8), np.int32)
    qzeros = np.empty((K // GROUP, N // 8), np.int32)
    scales = np.empty((K // GROUP, N), np.uint16)
    _check(lib().mcv_w4a16_quantize_host(_np_ptr(w), K, N, _np_ptr(qweight), _np_ptr(qzeros), _np_ptr(scales),
                                         nthreads), "mcv_w4a16_quantize_host")
    return qweight, qzeros, scales


def quantize_int4_embedding(emb_vk: np.ndarray, N: int, src_dtype: int = 0, nthreads: int = 0):
    """The synthetic int4 quantiser over a tied embedding [V, H] (fp16 or bf16
    bits) as the lm_head's [H, N] projection, columns from V on zero ->
    AutoAWQ (qweight, qzeros, scales u16)."""
    w = np.ascontiguousarray(emb_vk).view(np.uint16)
    V, K = w.shape
    qweight = np.empty((K, N // 8), np.int32)
    qzeros = np.empty((K // GROUP, N // 8), np.int32)
    scales = np.empty((K // GROUP, N), np.uint16)
    _check(lib().mcv_w4a16_quantize_nk_host(_np_ptr(w), src_dtype, K, V, N, _np_ptr(qweight), _np_ptr(qzeros),
                                            _np_ptr(scales), nthreads), "mcv_w4a16_quantize_nk_host")
    return qweight, qzeros, scales


def w8a8_tiled_bytes(K: int, N: int) -> int:
    return lib().mcv_w8a8_tiled_bytes(K, N)


def pack_w8a8_tiled(q_kn: np.ndarray) -> np.ndarray:
    """int8 [K, N] (the reference's w_int8 layout) -> MCV_W8_TILED bytes."""
    q_kn = np.ascontiguousarray(q_kn, np.int8)
    K, N = q_kn.shape
    out = np.empty(w8a8_tiled_bytes(K, N), np.int8)
    _check(lib().mcv_w8a8_pack_tiled_host(_np_ptr(q_kn), K, N, _np_ptr(out)), "mcv_w8a8_pack_tiled_host")
    return out


def quantize_w8a8_weight_host(w_kn_f16: np.ndarray, layout: int = W8_KN):
    """Per-channel int8 weight quantiser (quantized_weight.cpp:231-268) -> (q, scale f32 [N], scale f16 bits [N])."""
    w = np.ascontiguousarray(w_kn_f16).view(np.uint16)
    K, N = w.shape
    if layout == W8_TILED:
        q = np.empty(w8a8_tiled_bytes(K, N), np.int8)
    else:
        q = np.empty((K, N) if layout == W8_KN else (N, K), np.int8)
    s32 = np.empty(N, np.float32)
    s16 = np.empty(N, np.uint16)
    _check(lib().mcv_w8a8_quantize_weight_host(_np_ptr(w), K, N, _np_ptr(q), layout, _np_ptr(s32), _np_ptr(s16)),
           "mcv_w8a8_quantize_weight_host")
    return q, s32, s16


def pack_w8a8_tiled_nk(q_nk: np.ndarray) -> np.ndarray:
    """int8 [N, K] (a pre-quantised checkpoint tensor) -> MCV_W8_TILED bytes."""
    q_nk = np.ascontiguousarray(q_nk, np.int8)
    N, K = q_nk.shape
    out = np.empty(w8a8_tiled_bytes(K, N), np.int8)
    _check(lib().mcv_w8a8_pack_tiled_nk_host(_np_ptr(q_nk), K, N, _np_ptr(out)), "mcv_w8a8_pack_tiled_nk_host")
    return out


def quantize_w8a8_weight_nk_host(w_nk: np.ndarray, src_dtype: int = SRC_F16, layout: int = W8_TILED):
    """The same quantiser straight from a checkpoint's [N, K] fp16 / bf16 bits
    (the reference's bf16 load + host transpose + quantize_dense_weight_w8a8,
    language_model.cpp:84-105, quantized_weight.cpp:231-268) -> (q, s32, s16)."""
    w = np.ascontiguousarray(w_nk).view(np.uint16)
    N, K = w.shape
    if layout == W8_TILED:
        q = np.empty(w8a8_tiled_bytes(K, N), np.int8)
    else:
        q = np.empty((K, N) if layout == W8_KN else (N, K), np.int8)
    s32 = np.empty(N, np.float32)
    s16 = np.empty(N, np.uint16)
    _check(lib().mcv_w8a8_quantize_weight_nk_host(_np_ptr(w), src_dtype, K, N, _np_ptr(q), layout, _np_ptr(s32),
                                                  _np_ptr(s16)), "mcv_w8a8_quantize_weight_nk_host")
    return q, s32, s16


def quantize_w8a8_embedding(emb_vk: np.ndarray, N: int, src_dtype: int = SRC_F16, layout: int = W8_TILED):
    """The per-channel quantiser over a tied embedding [V, H] as the lm_head's
    [H, N] projection, channels from V on zero (the reference's zero-padded
    chunks, language_model.cpp:238-270) -> (q, s32, s16)."""
    w = np.ascontiguousarray(emb_vk).view(np.uint16)
    V, K = w.shape
    if layout == W8_TILED:
        q = np.empty(w8a8_tiled_bytes(K, N), np.int8)
    else:
        q = np.empty((K, N) if layout == W8_KN else (N, K), np.int8)
    s32 = np.empty(N, np.float32)
    s16 = np.empty(N, np.uint16)
    _check(lib().mcv_w8a8_quantize_weight_nk_pad_host(_np_ptr(w), src_dtype, K, V, N, _np_ptr(q), layout,
                                                      _np_ptr(s32), _np_ptr(s16)), "mcv_w8a8_quantize_weight_nk_pad_host")
    return q, s32, s16


# --------------------------------------------------------------------------- #
# device side (torch tensors as memory)                                        #
# --------------------------------------------------------------------------- #
def _torch():
    import torch
    return torch


def _stream(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _dev(t) -> int:
    return int(t.data_ptr())


@dataclass
class W4A16QuantizedWeight:
    """Device W4A16 weight in the slab-64 layout.

    Mirrors W4A16QuantizedWeight (src/csrc/include/minicpmv/quantized_weight.h:11-17)
    with the zero-points kept on the device (`zeros`, `zero_bias`) instead of
    being folded into an int8 (q - z) tensor.
    """

    qweight: "object"   # torch.uint8 [packed bytes]
    scales: "object"    # torch.int16 [G][Npad] (fp16 bits)
    zeros: "object"     # torch.int32 [G][Npad/8]
    K: int
    N: int
    zero_bias: int = 0
    group_size: int = GROUP
    # torch.float16 [K, N], set instead of the slab tensors for a GPTQ
    # act-order weight whose 128-row blocks span more than 16 levels (the
    # exact dequantised values; matmul_w4a16 runs it as a dense fp16 GEMM,
    # every fused W4A16 entry point refuses it)
    dense: "object" = None

    @classmethod
    def from_packed(cls, qw, sc, zr, K, N, zero_bias=0, device="cuda"):
        torch = _torch()
        return cls(torch.from_numpy(qw).to(device), torch.from_numpy(sc.view(np.int16)).to(device),
                   torch.from_numpy(zr.view(np.int32)).to(device), K, N, zero_bias)

    @classmethod
    def from_awq(cls, qweight, qzeros, scales, device="cuda"):
        qweight = np.asarray(qweight)
        K, N = qweight.shape[0], qweight.shape[1] * 8
        return cls.from_packed(*pack_awq(qweight, qzeros, scales), K, N, 0, device)

    @classmethod
    def from_gptq(cls, qweight, qzeros, g_idx, scales, device="cuda"):
        qweight = np.asarray(qweight)
        K, N = qweight.shape[0] * 8, qweight.shape[1]
        try:
            return cls.from_packed(*pack_gptq(qweight, qzeros, g_idx, scales), K, N, 1, device)
        except McvError as e:
            if e.status != MCV_ERR_UNSUPPORTED:
                raise
        torch = _torch()
        w = dequant_gptq(qweight, qzeros, g_idx, scales)
        return cls(None, None, None, K, N, 1, dense=torch.from_numpy(w.view(np.int16)).to(device).view(torch.float16))

    def ptrs(self):
        if self.dense is not None:
            raise McvError("this GPTQ act-order weight is kept dense (its 128-row blocks span more than 16 "
                           "levels); only matmul_w4a16 takes it")
        return _dev(self.qweight), _dev(self.scales), _dev(self.zeros)


def load_w4a16_quantized_weight(tensors: dict, base: str, device="cuda") -> W4A16QuantizedWeight:
    """Mirror of load_w4a16_quantized_weight (quantized_weight.cpp:212-228): GPTQ when
    `base.g_idx` exists, AutoAWQ otherwise.  `tensors` maps names to numpy arrays
    (e.g. from safetensors.numpy.load_file)."""
    qweight, qzeros, scales = tensors[base + ".qweight"], tensors[base + ".qzeros"], tensors[base + ".scales"]
    if base + ".g_idx" in tensors:
        return W4A16QuantizedWeight.from_gptq(qweight, qzeros, tensors[base + ".g_idx"], scales, device)
    return W4A16QuantizedWeight.from_awq(qweight, qzeros, scales, device)


def has_w4a16_quantized_weight(tensors: dict, base: str) -> bool:
    """quantized_weight.cpp:206-210."""
    return all(base + s in tensors for s in (".qweight", ".qzeros", ".scales"))


def _w4_call(fn_name: str, x, w: W4A16QuantizedWeight, out, stream):
    torch = _torch()
    if x.dtype != torch.float16 or x.dim() != 2 or x.shape[1] != w.K or not x.is_contiguous():
        raise McvError(f"{fn_name}: x must be contiguous fp16 [M, {w.K}]")
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, w.N), dtype=torch.float16, device=x.device)
    if out.dtype != torch.float16 or tuple(out.shape) != (M, w.N) or not out.is_contiguous():
        raise McvError(f"{fn_name}: out must be contiguous fp16 [{M}, {w.N}]")
    q, s, z = w.ptrs()
    _check(getattr(lib(), fn_name)(_dev(x), M, w.K, w.N, q, s, z, w.zero_bias, _dev(out), _stream(stream)), fn_name)
    return out


_GEMM_WS: dict = {}


def gemm_workspace(nbytes: int, device, stream=None):
    """The K-split workspace of the W4A16 GEMM for calls on one stream: kept
    per (device, stream), zero-filled when (re)allocated -- its tile counters
    must start at zero, and every call leaves them zero -- and grown only when
    a shape needs more, so steady-state calls allocate nothing.  Calls on one
    stream are ordered, so they may share it; two streams never do."""
    torch = _torch()
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(stream))
    ws = _GEMM_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _GEMM_WS[key] = ws
    return ws


def matmul_w4a16(x, w: W4A16QuantizedWeight, out=None, stream=None):
    """out[M, N] = x[M, K] . dequant(w), any M (ops.h:104-108 generalised).
    Where the MFMA GEMM splits K across workgroups (few rows, long K) it takes
    the per-stream workspace of gemm_workspace()."""
    torch = _torch()
    if x.dtype != torch.float16 or x.dim() != 2 or x.shape[1] != w.K or not x.is_contiguous():
        raise McvError(f"matmul_w4a16: x must be contiguous fp16 [M, {w.K}]")
    if w.dense is not None:                  # act-order weight kept dense: the vendor's fp16 GEMM
        if out is None:
            out = torch.empty((x.shape[0], w.N), dtype=torch.float16, device=x.device)
        if stream is None:
            torch.matmul(x, w.dense, out=out)
        else:
            with torch.cuda.stream(stream):
                torch.matmul(x, w.dense, out=out)
        return out
    nb = int(lib().mcv_w4a16_gemm_workspace_bytes(x.shape[0], w.K, w.N))
    if nb == 0:
        return _w4_call("mcv_w4a16_gemm", x, w, out, stream)
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, w.N), dtype=torch.float16, device=x.device)
    if out.dtype != torch.float16 or tuple(out.shape) != (M, w.N) or not out.is_contiguous():
        raise McvError(f"matmul_w4a16: out must be contiguous fp16 [{M}, {w.N}]")
    ws = gemm_workspace(nb, x.device, stream)
    q, s, z = w.ptrs()
    _check(lib().mcv_w4a16_gemm_ws(_dev(x), M, w.K, w.N, q, s, z, w.zero_bias, _dev(out), _dev(ws), ws.numel(),
                                   _stream(stream)), "matmul_w4a16")
    return out


def matmul_w4a16_gemv(x, w, out=None, stream=None):
    return _w4_call("mcv_w4a16_gemv", x, w, out, stream)


def matmul_w4a16_multi(x, weights, outs=None, stream=None):
    """Up to four projections of the same x [M, K] in one launch (q/k/v or
    qkv + z at decode, decoder_layer.cpp:970-972, 1108-1110); returns the outputs."""
    torch = _torch()
    if x.dtype != torch.float16 or x.dim() != 2 or not x.is_contiguous():
        raise McvError("matmul_w4a16_multi x must be contiguous fp16 [M, K]")
    M, K = x.shape
    if outs is None:
        outs = [torch.empty((M, w.N), dtype=torch.float16, device=x.device) for w in weights]
    if len(outs) != len(weights) or not 1 <= len(weights) <= 4:
        raise McvError("matmul_w4a16_multi takes 1..4 weights and as many outputs")
    parts = (_W4Part * len(weights))()
    for i, (w, o) in enumerate(zip(weights, outs)):
        if w.K != K or tuple(o.shape) != (M, w.N) or o.dtype != torch.float16:
            raise McvError(f"matmul_w4a16_multi part {i}: weight K or output shape mismatch")
        q, sc, z = w.ptrs()
        parts[i] = _W4Part(q, sc, z, w.zero_bias, w.N, _dev(o))
    _check(lib().mcv_w4a16_gemv_multi(_dev(x), M, K, ctypes.cast(parts, ctypes.c_void_p), len(weights), _stream(stream)),
           "matmul_w4a16_multi")
    return outs


def matmul_w4a16_mfma(x, w, out=None, stream=None):
    return _w4_call("mcv_w4a16_gemm_mfma", x, w, out, stream)


def mlp_gate_up_silu_w4a16(x, w_gate: W4A16QuantizedWeight, w_up: W4A16QuantizedWeight, out=None, stream=None):
    """act[M, N] = silu(x . gate) * (x . up), one launch; bit-identical to two
    matmul_w4a16 calls and silu_mul (decoder_layer.cpp:1029-1046)."""
    torch = _torch()
    if x.dtype != torch.float16 or x.dim() != 2 or x.shape[1] != w_gate.K or not x.is_contiguous():
        raise McvError(f"mlp_gate_up_silu: x must be contiguous fp16 [M, {w_gate.K}]")
    if (w_up.K, w_up.N) != (w_gate.K, w_gate.N):
        raise McvError("mlp_gate_up_silu: gate and up weights must have the same shape")
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, w_gate.N), dtype=torch.float16, device=x.device)
    if out.dtype != torch.float16 or tuple(out.shape) != (M, w_gate.N) or not out.is_contiguous():
        raise McvError(f"mlp_gate_up_silu: out must be contiguous fp16 [{M}, {w_gate.N}]")
    qg, sg, zg = w_gate.ptrs()
    qu, su, zu = w_up.ptrs()
    _check(lib().mcv_w4a16_gate_up_silu(_dev(x), M, w_gate.K, w_gate.N, qg, sg, zg, w_gate.zero_bias, qu, su, zu,
                                        w_up.zero_bias, _dev(out), _stream(stream)), "mcv_w4a16_gate_up_silu")
    return out


class DecodeMlpW4A16:
    """The whole decode MLP block, M = 1: out[H] = (silu(x . gate) * (x . up)) . down
    (decoder_layer.cpp:1029-1046), bit-identical to mlp_gate_up_silu_w4a16
    followed by matmul_w4a16 -- in one launch (mcv_w4a16_mlp) where the shape
    allows, else those two launches (one_launch turns False).  Owns the
    workspace through which the act row passes inside the kernel; calls on one
    object must not overlap (one stream)."""

    ERROR_WORD = 0             # u32 index of the give-up flag in the workspace
    _ERR_SHAPE = 2

    def __init__(self, gate: W4A16QuantizedWeight, up: W4A16QuantizedWeight, down: W4A16QuantizedWeight):
        torch = _torch()
        if (up.K, up.N) != (gate.K, gate.N) or (down.K, down.N) != (gate.N, gate.K):
            raise McvError(f"decode MLP: gate/up must be [H, I] and down [I, H]; got gate {gate.K}x{gate.N}, "
                           f"up {up.K}x{up.N}, down {down.K}x{down.N}")
        self.gate, self.up, self.down = gate, up, down
        self.H, self.I = gate.K, gate.N
        dev = gate.qweight.device
        nbytes = lib().mcv_w4a16_mlp_workspace_bytes(self.H, self.I)
        self.one_launch = nbytes > 0
        self.workspace = torch.zeros(max(nbytes, 4) // 4, dtype=torch.int32, device=dev)
        self.act = torch.empty((1, self.I), dtype=torch.float16, device=dev)

    def _args(self, x, out, stream):
        torch = _torch()
        if x.dtype != torch.float16 or x.numel() != self.H or not x.is_contiguous():
            raise McvError(f"decode MLP: x must be contiguous fp16 [1, {self.H}]")
        if out.dtype != torch.float16 or out.numel() != self.H or not out.is_contiguous():
            raise McvError(f"decode MLP: out must be contiguous fp16 [1, {self.H}]")
        g, u, d = self.gate, self.up, self.down
        return ((_dev(x), self.H, self.I) + g.ptrs() + (g.zero_bias,) + u.ptrs() + (u.zero_bias,) + d.ptrs()
                + (d.zero_bias, _dev(out), _dev(self.workspace), None, _stream(stream)))

    def _two_launches(self, x, out, stream):
        mlp_gate_up_silu_w4a16(x.view(1, self.H), self.gate, self.up, self.act, stream)
        matmul_w4a16(self.act, self.down, out.view(1, self.H), stream)

    def __call__(self, x, out=None, stream=None):
        torch = _torch()
        if out is None:
            out = torch.empty((1, self.H), dtype=torch.float16, device=x.device)
        args = self._args(x, out, stream)
        if self.one_launch:
            rc = lib().mcv_w4a16_mlp(*args)
            if rc != self._ERR_SHAPE:
                _check(rc, "mcv_w4a16_mlp")
                return out
            self.one_launch = False            # this shape or device cannot hold the one-launch grid
        self._two_launches(x, out, stream)
        return out

    def bind(self, x, out, stream=None):
        """A zero-argument launcher over fixed buffers (arguments resolved once)."""
        self(x, out, stream)                   # settles one_launch
        if not self.one_launch:
            return lambda: self._two_launches(x, out, stream)
        fn, args = lib().mcv_w4a16_mlp, self._args(x, out, stream)

        def launch():
            _check(fn(*args), "mcv_w4a16_mlp")
        return launch

    def act_wait_gave_up(self) -> bool:
        """True if a wait for another workgroup's words in any earlier call
        timed out (synchronises)."""
        return bool(int(self.workspace[self.ERROR_WORD].item()))


def w4a16_dequant(w: W4A16QuantizedWeight, f16=True, i8=False, stream=None):
    torch = _torch()
    wf = torch.empty((w.K, w.N), dtype=torch.float16, device=w.qweight.device) if f16 else None
    w8 = torch.empty((w.K, w.N), dtype=torch.int8, device=w.qweight.device) if i8 else None
    q, s, z = w.ptrs()
    _check(lib().mcv_w4a16_dequant(q, s, z, w.zero_bias, w.K, w.N, _dev(wf) if wf is not None else 0,
                                   _dev(w8) if w8 is not None else 0, _stream(stream)), "mcv_w4a16_dequant")
    return wf, w8


def matmul_w4a16_tiled(x, w_int8, scales, out, stream=None):
    """The reference's 4-argument matmul_w4a16 (ops.cpp:1030-1095): int8 (q - z)
    tile-packed by pack_w4a16_weight, fp16 scales [K/128, N], M = 1."""
    torch = _torch()
    if x.dtype != torch.float16 or x.dim() != 2 or x.shape[0] != 1:
        raise McvError("matmul_w4a16 x must be [1, K]")
    if w_int8.dtype != torch.int8 or w_int8.dim() != 2:
        raise McvError("matmul_w4a16 w must be [packed_rows, tile_len]")
    K, N = x.shape[1], scales.shape[1]
    if tuple(scales.shape) != (K // GROUP, N) or tuple(out.shape) != (1, N):
        raise McvError("matmul_w4a16 scales must be [K/128, N] and out [1, N]")
    _check(lib().mcv_w4a16_gemv_tiled_i8(_dev(x), K, N, w_int8.shape[1], w_int8.shape[0], _dev(w_int8), _dev(scales),
                                         _dev(out), _stream(stream)), "matmul_w4a16")
    return out


class LmHeadW4A16:
    """Greedy lm_head over a W4A16 weight [K, >= vocab] with the argmax fused
    into the GEMV (replaces lm_head_greedy's 16 chunk matmuls + host scan,
    src/csrc/lib/language_model.cpp:412-482).  Owns its workspaces.

    Three routes to the same token: launch() writes it on the device (the
    call-tagged key words the last workgroup reads); launch_slots() + read_slots_token() -- what
    __call__ uses, since it returns the token to the host anyway -- leave
    call-tagged slot maxima that the host folds after its copy;
    launch_partials() + reduce_partials() use a second kernel."""

    TAG_MAX = 0xFFFFFF
    N_SLOTS, SLOT_STRIDE = 64, 16

    def __init__(self, w: W4A16QuantizedWeight, vocab: int):
        torch = _torch()
        if vocab > w.N:
            raise McvError(f"vocab {vocab} exceeds weight width {w.N}")
        self.w, self.vocab = w, vocab
        dev = w.qweight.device
        # zero-filled once; the fused calls keep its generation word and tagged keys consistent
        self.workspace = torch.zeros(lib().mcv_lm_head_workspace_bytes(vocab), dtype=torch.uint8, device=dev)
        self.slots = torch.zeros(lib().mcv_lm_head_slots_bytes() // 8, dtype=torch.int64, device=dev)
        self.tag = 0
        self._slots_stream = None                     # stream of the last slots launch (None: current)
        self.keys = torch.empty(-(-vocab // SLAB), dtype=torch.int64, device=dev)
        self.token = torch.zeros(1, dtype=torch.int64, device=dev)

    def _check_io(self, x, logits):
        torch = _torch()
        if x.dtype != torch.float16 or x.numel() != self.w.K or not x.is_contiguous():
            raise McvError(f"lm_head x must be contiguous fp16 [1, {self.w.K}]")
        if logits is not None and (logits.dtype != torch.float16 or logits.numel() != self.vocab):
            raise McvError(f"lm_head logits must be fp16 [{self.vocab}]")

    def launch(self, x, logits=None, stream=None):
        """Stream-ordered: fills self.token (and logits if given); no sync."""
        self._check_io(x, logits)
        q, s, z = self.w.ptrs()
        _check(lib().mcv_w4a16_lm_head_argmax(_dev(x), self.w.K, self.w.N, self.vocab, q, s, z, self.w.zero_bias,
                                              _dev(logits) if logits is not None else 0, _dev(self.token),
                                              _dev(self.workspace), None, _stream(stream)), "mcv_w4a16_lm_head_argmax")
        return self.token

    def _next_tag(self, stream) -> int:
        """Tags must grow call by call; at the wrap the slots are zero-filled
        again, on the launch stream so the fill is ordered with the calls."""
        if self.tag >= self.TAG_MAX:
            torch = _torch()
            with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
                self.slots.zero_()
            self.tag = 0
        self.tag += 1
        self._slots_stream = stream
        return self.tag

    def launch_slots(self, x, logits=None, stream=None) -> int:
        """Stream-ordered: leaves this call's tagged maxima in self.slots; returns the tag."""
        self._check_io(x, logits)
        self._next_tag(stream)
        q, s, z = self.w.ptrs()
        _check(lib().mcv_w4a16_lm_head_argmax_slots(_dev(x), self.w.K, self.w.N, self.vocab, q, s, z,
                                                    self.w.zero_bias, _dev(logits) if logits is not None else 0,
                                                    _dev(self.slots), self.tag, _stream(stream)),
               "mcv_w4a16_lm_head_argmax_slots")
        return self.tag

    def bind(self, x, logits=None, stream=None, route: str = "tree"):
        """A zero-argument launcher over fixed buffers, checked and resolved
        once, for decode loops that re-launch the lm_head every token (about
        4 us of host time per call).  route "tree": each call does launch();
        "slots": each call does launch_slots() and returns the tag."""
        self._check_io(x, logits)
        q, s, z = self.w.ptrs()
        head = (_dev(x), self.w.K, self.w.N, self.vocab, q, s, z, self.w.zero_bias,
                _dev(logits) if logits is not None else 0)
        st = _stream(stream)
        if route == "tree":
            fn, args = lib().mcv_w4a16_lm_head_argmax, head + (_dev(self.token), _dev(self.workspace), None, st)

            def launch():
                _check(fn(*args), "mcv_w4a16_lm_head_argmax")
                return self.token
            return launch
        if route != "slots":
            raise McvError(f"unknown lm_head route {route!r}")
        fn, slots = lib().mcv_w4a16_lm_head_argmax_slots, _dev(self.slots)

        def launch_slots():
            tag = self._next_tag(stream)
            _check(fn(*head, slots, tag, st), "mcv_w4a16_lm_head_argmax_slots")
            return tag
        return launch_slots

    def read_slots_token(self, tag: int) -> int:
        """The token of call `tag` from the slots (waits for the stream the
        slots were last launched on, then copies them to the host)."""
        if self._slots_stream is not None:
            self._slots_stream.synchronize()
        host = np.ascontiguousarray(self.slots.cpu().numpy())      # synchronising copy
        return int(lib().mcv_lm_head_slots_token(_np_ptr(host), tag))

    def launch_partials(self, x, logits=None, stream=None):
        """First stage only: the GEMV writing logits and per-slab argmax keys."""
        q, s, z = self.w.ptrs()
        _check(lib().mcv_w4a16_gemv_argmax_partials(_dev(x), self.w.K, self.w.N, self.vocab, q, s, z,
                                                    self.w.zero_bias, _dev(logits) if logits is not None else 0,
                                                    _dev(self.keys), _stream(stream)),
               "mcv_w4a16_gemv_argmax_partials")

    def reduce_partials(self, stream=None):
        _check(lib().mcv_argmax_reduce_keys(_dev(self.keys), self.keys.numel(), _dev(self.token),
                                            _stream(stream)), "mcv_argmax_reduce_keys")
        return self.token

    def __call__(self, x, logits=None) -> int:
        return self.read_slots_token(self.launch_slots(x, logits))


# ----------------------------------------------------------------- W8A8 ----- #
@dataclass
class W8A8QuantizedWeight:
    """Mirrors W8A8QuantizedWeight (quantized_weight.h:19-24) plus the fp32 scale."""

    w_int8: "object"       # torch.int8, [K, N] (W8_KN), [N, K] (W8_NK) or flat MFMA tiles (W8_TILED)
    w_scale: "object"      # torch.float16 [N] (truncating encode, the reference's stored form)
    w_scale_f32: "object"  # torch.float32 [N]
    K: int
    N: int
    layout: int = W8_TILED


def quantize_dense_weight_w8a8(weight_kn, layout: int = W8_TILED) -> W8A8QuantizedWeight:
    """quantized_weight.cpp:231-268 without the device round trip: fp16 [K, N] -> int8 + scales."""
    torch = _torch()
    w_np = weight_kn.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16) \
        if hasattr(weight_kn, "detach") else np.asarray(weight_kn).view(np.uint16)
    K, N = w_np.shape
    q, s32, s16 = quantize_w8a8_weight_host(w_np, layout)
    # numpy arrays carry .device == "cpu" (a string) in numpy 2: only a torch
    # CUDA tensor names its device
    dev = weight_kn.device if getattr(getattr(weight_kn, "device", None), "type", None) == "cuda" else "cuda"
    return W8A8QuantizedWeight(torch.from_numpy(q).to(dev), torch.from_numpy(s16.view(np.int16)).to(dev).view(torch.float16),
                               torch.from_numpy(s32).to(dev), K, N, layout)


_NO_F32 = object()     # w8a8_quantize(x_scale=_NO_F32): write only the fp16 scale


def w8a8_quantize(x, x_int8=None, x_scale=None, x_scale_f16=None, stream=None):
    """Per-row activation quant (ops.cpp:1135-1171 generalised to M rows).
    Returns (x_int8 [M, K], x_scale fp32 [M] or None, x_scale_f16 [M] or None);
    the fp16 scale is the RNE encoding of the fp32 one, the reference's stored
    form.  x_scale=_NO_F32 skips the fp32 scale (x_scale_f16 is then required)."""
    torch = _torch()
    if x.dtype != torch.float16 or x.dim() != 2 or not x.is_contiguous():
        raise McvError("w8a8_quantize x must be contiguous fp16 [M, K]")
    M, K = x.shape
    if x_int8 is None:
        x_int8 = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if x_scale is _NO_F32:
        x_scale = None
        if x_scale_f16 is None:
            raise McvError("w8a8_quantize: needs an fp32 or an fp16 scale output")
    elif x_scale is None:
        x_scale = torch.empty(M, dtype=torch.float32, device=x.device)
    _check(lib().mcv_w8a8_quantize_act(_dev(x), M, K, _dev(x_int8), _dev(x_scale) if x_scale is not None else 0,
                                       _dev(x_scale_f16) if x_scale_f16 is not None else 0, _stream(stream)),
           "w8a8_quantize")
    return x_int8, x_scale, x_scale_f16


def matmul_w8a8_i32(x_int8, w_int8, out=None, layout: int = W8_KN, stream=None, N: int = 0):
    """acc[M, N] int32 = x_int8 . w (ops.cpp:1097-1133 generalised to M rows).
    `w_int8` may also be a W8A8QuantizedWeight (its layout and N are used)."""
    torch = _torch()
    M, K = x_int8.shape
    if isinstance(w_int8, W8A8QuantizedWeight):
        layout, N, w_int8 = w_int8.layout, w_int8.N, w_int8.w_int8
    elif layout == W8_TILED:
        if N <= 0:
            raise McvError("matmul_w8a8_i32: N is required for a tiled weight tensor")
    else:
        N = w_int8.shape[1] if layout == W8_KN else w_int8.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=x_int8.device)
    _check(lib().mcv_w8a8_gemm_i32(_dev(x_int8), M, K, N, _dev(w_int8), layout, _dev(out), _stream(stream)),
           "matmul_w8a8_i32")
    return out


def _scale_dtype(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return MCV_F32
    if t.dtype == torch.float16:
        return MCV_F16
    raise McvError(f"scale dtype must be fp32 or fp16, got {t.dtype}")


def w8a8_dequant(acc, x_scale, w_scale, out=None, stream=None):
    """out = fp16 RNE((acc * w_scale[n]) * x_scale[m]) (ops.cpp:1173-1210)."""
    torch = _torch()
    M, N = acc.shape
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=acc.device)
    _check(lib().mcv_w8a8_dequant(_dev(acc), _dev(x_scale), _scale_dtype(x_scale), _dev(w_scale), _scale_dtype(w_scale),
                                  M, N, _dev(out), _stream(stream)), "w8a8_dequant")
    return out


def matmul_w8a8(x_int8, x_scale, w: W8A8QuantizedWeight, out=None, use_f32_scale=True, stream=None):
    """Fused int8 GEMM + dequant epilogue; bit-identical to matmul_w8a8_i32 + w8a8_dequant."""
    torch = _torch()
    M, K = x_int8.shape
    if out is None:
        out = torch.empty((M, w.N), dtype=torch.float16, device=x_int8.device)
    ws = w.w_scale_f32 if use_f32_scale else w.w_scale
    _check(lib().mcv_w8a8_gemm_f16(_dev(x_int8), _dev(x_scale), _scale_dtype(x_scale), M, K, w.N, _dev(w.w_int8),
                                   w.layout, _dev(ws), _scale_dtype(ws), _dev(out), _stream(stream)), "matmul_w8a8")
    return out


def lm_head_argmax_w8a8(x_int8, x_scale, w: W8A8QuantizedWeight, vocab: int, logits=None, keys=None, token=None,
                        use_f32_scale=False, stream=None):
    """The W8A8 lm_head on the device (language_model.cpp:434-480): the fused
    GEMV over the first `vocab` columns (logits bit-identical to matmul_w8a8,
    written when `logits` is given) with one argmax key per 64-column slab,
    then their reduction.  Returns the int64 [1] token on the device.  Scales
    as matmul_w8a8: the weight's fp16 w_scale unless use_f32_scale."""
    torch = _torch()
    if w.layout != W8_TILED:
        raise McvError("lm_head_argmax_w8a8 needs an MCV_W8_TILED weight")
    if x_int8.dtype != torch.int8 or x_int8.numel() != w.K or not x_int8.is_contiguous():
        raise McvError("lm_head_argmax_w8a8 x must be contiguous int8 [1, K]")
    nslab = -(-vocab // SLAB)
    if keys is None:
        keys = torch.empty(nslab, dtype=torch.int64, device=x_int8.device)
    if token is None:
        token = torch.empty(1, dtype=torch.int64, device=x_int8.device)
    if keys.numel() < nslab or token.numel() < 1:
        raise McvError(f"lm_head_argmax_w8a8: keys need {nslab} int64 and token one")
    ws = w.w_scale_f32 if use_f32_scale else w.w_scale
    _check(lib().mcv_w8a8_gemv_argmax_partials(_dev(x_int8), _dev(x_scale), _scale_dtype(x_scale), w.K, w.N, vocab,
                                               _dev(w.w_int8), _dev(ws), _scale_dtype(ws),
                                               _dev(logits) if logits is not None else None, _dev(keys),
                                               _stream(stream)), "mcv_w8a8_gemv_argmax_partials")
    _check(lib().mcv_argmax_reduce_keys(_dev(keys), nslab, _dev(token), _stream(stream)), "mcv_argmax_reduce_keys")
    return token


def lm_head_workspace_bytes(vocab: int) -> int:
    """Bytes of the device-token lm_head workspace for `vocab` columns (0: unsupported)."""
    return int(lib().mcv_lm_head_workspace_bytes(vocab))


def lm_head_argmax_w8a8_fused(x, w: W8A8QuantizedWeight, vocab: int, workspace, logits=None, token=None,
                              use_f32_scale=False, status=None, stream=None):
    """The whole W8A8 lm_head step in one launch (mcv_w8a8_lm_head_argmax):
    x fp16 [1, K] quantised on the device, the fused GEMV over the first
    `vocab` columns (logits written when given) and the argmax as an int64
    [1] token on the device -- bit-identical to w8a8_quantize +
    lm_head_argmax_w8a8.  Scales: the fp16 x_scale and the weight's fp16
    w_scale (the reference's), or fp32 both with use_f32_scale.  `workspace`
    is a zero-filled uint8 tensor of lm_head_workspace_bytes(vocab) bytes
    that later calls reuse (the W4A16 lm_head's workspace format)."""
    torch = _torch()
    if w.layout != W8_TILED:
        raise McvError("lm_head_argmax_w8a8_fused needs an MCV_W8_TILED weight")
    if x.dtype != torch.float16 or x.numel() != w.K or not x.is_contiguous():
        raise McvError("lm_head_argmax_w8a8_fused x must be contiguous fp16 [1, K]")
    if token is None:
        token = torch.empty(1, dtype=torch.int64, device=x.device)
    ws = w.w_scale_f32 if use_f32_scale else w.w_scale
    _check(lib().mcv_w8a8_lm_head_argmax(_dev(x), w.K, w.N, vocab, _dev(w.w_int8), _dev(ws), _scale_dtype(ws),
                                         MCV_F32 if use_f32_scale else MCV_F16,
                                         _dev(logits) if logits is not None else None, _dev(token),
                                         _dev(workspace), _dev(status) if status is not None else None,
                                         _stream(stream)), "mcv_w8a8_lm_head_argmax")
    return token


class DecodeMlpW8A8:
    """The whole W8A8 decode MLP block, M = 1, in one launch from the normed
    fp16 row: out[H] = deq(quant(silu(deq(quant(x) . gate)) * deq(quant(x) . up)) . down)
    (decoder_layer.cpp:1022-1046), bit-identical to w8a8_quantize,
    mlp_gate_up_silu_w8a8, w8a8_quantize and matmul_w8a8 with the same
    scales; those four launches where the one-launch grid does not fit
    (one_launch turns False).  precision "reference" (default): the fp16
    activation scale and the truncated fp16 weight scale in every epilogue, as
    the reference's dispatcher stores and reads them (decoder_layer.cpp:216-237);
    "f32": fp32 scales throughout (BASELINE config 5's precision).  Weights
    must be MCV_W8_TILED.  Calls on one object must not overlap."""

    ERROR_WORD = 0
    _ERR_SHAPE = 2

    def __init__(self, gate: "W8A8QuantizedWeight", up: "W8A8QuantizedWeight", down: "W8A8QuantizedWeight",
                 precision: str = "reference"):
        torch = _torch()
        if (up.K, up.N) != (gate.K, gate.N) or (down.K, down.N) != (gate.N, gate.K):
            raise McvError("decode MLP (W8A8): gate/up must be [H, I] and down [I, H]")
        if any(w.layout != W8_TILED for w in (gate, up, down)):
            raise McvError("decode MLP (W8A8): weights must be in the tiled layout")
        if precision not in ("reference", "f32"):
            raise McvError(f"decode MLP (W8A8): precision must be 'reference' or 'f32', got {precision!r}")
        self.gate, self.up, self.down = gate, up, down
        self.H, self.I = gate.K, gate.N
        self.f32 = precision == "f32"
        dev = gate.w_int8.device
        nbytes = lib().mcv_w8a8_mlp_workspace_bytes(self.H, self.I)
        self.one_launch = nbytes > 0
        self.workspace = torch.zeros(max(nbytes, 4) // 4, dtype=torch.int32, device=dev)

    def _scales(self, w):
        return w.w_scale_f32 if self.f32 else w.w_scale

    def _quant(self, x, stream):
        torch = _torch()
        if self.f32:
            xq, xs, _ = w8a8_quantize(x, stream=stream)
            return xq, xs
        s16 = torch.empty(x.shape[0], dtype=torch.float16, device=x.device)
        xq, _, s16 = w8a8_quantize(x, x_scale=_NO_F32, x_scale_f16=s16, stream=stream)
        return xq, s16

    def _four_launches(self, x, out, stream):
        xq, xs = self._quant(x.view(1, self.H), stream)
        act = mlp_gate_up_silu_w8a8(xq, xs, self.gate, self.up, use_f32_scale=self.f32, stream=stream)
        aq, asc = self._quant(act, stream)
        matmul_w8a8(aq, asc, self.down, out.view(1, self.H), use_f32_scale=self.f32, stream=stream)

    def __call__(self, x, out=None, stream=None):
        torch = _torch()
        if x.dtype != torch.float16 or x.numel() != self.H or not x.is_contiguous():
            raise McvError(f"decode MLP (W8A8): x must be contiguous fp16 [1, {self.H}]")
        if out is None:
            out = torch.empty((1, self.H), dtype=torch.float16, device=x.device)
        if out.dtype != torch.float16 or out.numel() != self.H or not out.is_contiguous():
            raise McvError(f"decode MLP (W8A8): out must be contiguous fp16 [1, {self.H}]")
        if self.one_launch:
            g, u, d = self.gate, self.up, self.down
            rc = lib().mcv_w8a8_mlp(_dev(x), self.H, self.I, _dev(g.w_int8), _dev(self._scales(g)), _dev(u.w_int8),
                                    _dev(self._scales(u)), _dev(d.w_int8), _dev(self._scales(d)),
                                    MCV_F32 if self.f32 else MCV_F16, _dev(out), _dev(self.workspace), None,
                                    _stream(stream))
            if rc != self._ERR_SHAPE:
                _check(rc, "mcv_w8a8_mlp")
                return out
            self.one_launch = False
        self._four_launches(x, out, stream)
        return out

    def wait_gave_up(self) -> bool:
        """True if a wait for another workgroup's words in any earlier call
        timed out (synchronises)."""
        return bool(int(self.workspace[self.ERROR_WORD].item()))


def mlp_gate_up_silu_w8a8(x_int8, x_scale, w_gate: W8A8QuantizedWeight, w_up: W8A8QuantizedWeight, out=None,
                          use_f32_scale=True, stream=None):
    """act = silu(gate) * up over one quantised x, tiled weights, M <= 4 (decoder_layer.cpp:1029-1046
    + silu_mul): one launch, bit-identical to two matmul_w8a8 calls and silu_mul."""
    torch = _torch()
    M, K = x_int8.shape
    if out is None:
        out = torch.empty((M, w_gate.N), dtype=torch.float16, device=x_int8.device)
    wsg = w_gate.w_scale_f32 if use_f32_scale else w_gate.w_scale
    wsu = w_up.w_scale_f32 if use_f32_scale else w_up.w_scale
    _check(lib().mcv_w8a8_gate_up_silu(_dev(x_int8), _dev(x_scale), _scale_dtype(x_scale), M, K, w_gate.N,
                                       _dev(w_gate.w_int8), _dev(wsg), _dev(w_up.w_int8), _dev(wsu), _scale_dtype(wsg),
                                       _dev(out), _stream(stream)), "mlp_gate_up_silu_w8a8")
    return out


# ------------------------------------------------------------- elementwise -- #
def silu_mul(gate, up, out=None, stream=None):
    """out = silu(gate) * up in fp32, RNE to fp16 (ops.cpp:437-456)."""
    torch = _torch()
    if gate.shape != up.shape or gate.dtype != torch.float16 or up.dtype != torch.float16:
        raise McvError("silu_mul requires fp16 tensors of one shape")
    if out is None:
        out = torch.empty_like(gate)
    _check(lib().mcv_silu_mul(_dev(gate), _dev(up), _dev(out), gate.numel(), _stream(stream)), "silu_mul")
    return out


def lm_head_slabs_per_workgroup(vocab: int) -> int:
    """Slabs of 64 columns per workgroup the lm_head launches for `vocab` columns."""
    return int(lib().mcv_lm_head_slabs_per_workgroup(int(vocab)))


def w8a8_lm_head_slabs_per_workgroup(vocab: int) -> int:
    """Slabs of 64 columns per workgroup the one-launch W8A8 lm_head launches for `vocab` columns."""
    return int(lib().mcv_w8a8_lm_head_slabs_per_workgroup(int(vocab)))


def argmax_last_dim(x, out=None, stream=None):
    """Per-row first-maximum argmax of fp16 [M, N] -> int64 [M]."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    if out is None:
        out = torch.empty(x2.shape[0], dtype=torch.int64, device=x.device)
    _check(lib().mcv_argmax_f16(_dev(x2), x2.shape[0], x2.shape[1], _dev(out), _stream(stream)), "argmax")
    return out


def rms_norm(x, gamma, eps: float, out=None, stream=None):
    """Row-wise RMSNorm of fp16 [M, H] with fp16 gamma [H] (fp32 arithmetic)."""
    torch = _torch()
    if x.dtype != torch.float16 or gamma.dtype != torch.float16 or x.shape[-1] != gamma.numel():
        raise McvError("rms_norm requires fp16 x [M, H] and gamma [H]")
    x2 = x.reshape(-1, x.shape[-1])
    if out is None:
        out = torch.empty_like(x)
    _check(lib().mcv_rms_norm(_dev(x2), _dev(gamma), x2.shape[0], x2.shape[1], float(eps), _dev(out), _stream(stream)),
           "rms_norm")
    return out


def rms_norm_w8a8_quantize(x, gamma, eps: float, normed=None, want_normed: bool = True, x_scale_f16=None,
                           stream=None):
    """RMSNorm then per-row int8 quantisation in one launch (decoder_layer.cpp:955-966,
    1022-1032); bit-identical to rms_norm + w8a8_quantize.  Returns
    (normed fp16 [M, H] or None, x_int8 [M, H], x_scale fp32 [M], x_scale_f16 or None)."""
    torch = _torch()
    if x.dtype != torch.float16 or gamma.dtype != torch.float16 or x.dim() != 2 or not x.is_contiguous() \
            or x.shape[1] != gamma.numel():
        raise McvError("rms_norm_w8a8_quantize requires contiguous fp16 x [M, H] and gamma [H]")
    M, H = x.shape
    if normed is None and want_normed:
        normed = torch.empty_like(x)
    xq = torch.empty((M, H), dtype=torch.int8, device=x.device)
    xs = torch.empty(M, dtype=torch.float32, device=x.device)
    _check(lib().mcv_rms_norm_w8a8_quantize(_dev(x), _dev(gamma), M, H, float(eps),
                                            _dev(normed) if normed is not None else 0, _dev(xq), _dev(xs),
                                            _dev(x_scale_f16) if x_scale_f16 is not None else 0, _stream(stream)),
           "rms_norm_w8a8_quantize")
    return normed, xq, xs, x_scale_f16


def version() -> str:
    return lib().mcv_version().decode()
