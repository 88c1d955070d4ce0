"""Test helpers: package loader, the CPU oracle (ctypes), seeded generators.

The oracle (oracle/mcv_oracle.c) is the checker only; nothing here is used
by the product path.
"""
from __future__ import annotations

import ctypes
import importlib.util
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "minicpm-v-4.6-orangepi_amd"
ORACLE_DIR = ROOT / "oracle"
ORACLE_SO = ORACLE_DIR / "build" / "libmcv_oracle.so"
PKG_NAME = "minicpmv_amd"


def load_pkg():
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(PKG_NAME, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available() and torch.cuda.device_count() > 0
    except Exception:
        return False


_u16p = ctypes.c_void_p
_i64 = ctypes.c_int64


class Oracle:
    """numpy-facing wrapper of oracle/build/libmcv_oracle.so."""

    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            subprocess.run(["make", "-C", str(ORACLE_DIR)], check=True, capture_output=True)
        L = ctypes.CDLL(str(path))
        vp = ctypes.c_void_p
        sig = {
            "or_h2f": (ctypes.c_float, [ctypes.c_uint16]),
            "or_h2f_ftz": (ctypes.c_float, [ctypes.c_uint16]),
            "or_f2h_trunc": (ctypes.c_uint16, [ctypes.c_float]),
            "or_f2h_rne": (ctypes.c_uint16, [ctypes.c_float]),
            "or_h2f_array": (None, [vp, _i64, vp]),
            "or_f2h_rne_array": (None, [vp, _i64, vp]),
            "or_f2h_trunc_array": (None, [vp, _i64, vp]),
            "or_bf16_to_f16_trunc_array": (None, [vp, _i64, vp]),
            "or_unpack_awq": (ctypes.c_int, [vp, vp, _i64, _i64, vp]),
            "or_unpack_gptq": (ctypes.c_int, [vp, vp, vp, _i64, _i64, _i64, vp]),
            "or_quantize_int4_awq": (ctypes.c_int, [vp, _i64, _i64, vp, vp, vp]),
            "or_w4a16_matmul": (None, [vp, vp, vp, _i64, _i64, _i64, vp, ctypes.c_int]),
            "or_w4a16_dequant_f16": (None, [vp, vp, _i64, _i64, vp]),
            "or_quantize_i8": (ctypes.c_int8, [ctypes.c_float, ctypes.c_float]),
            "or_w8a8_quantize_weight": (None, [vp, _i64, _i64, vp, vp, vp]),
            "or_w8a8_quantize_act": (None, [vp, _i64, _i64, vp, vp, vp]),
            "or_gemm_i32": (None, [vp, vp, _i64, _i64, _i64, vp, ctypes.c_int]),
            "or_w8a8_dequant": (None, [vp, vp, vp, _i64, _i64, vp]),
            "or_silu_mul": (None, [vp, vp, _i64, vp]),
            "or_argmax_f16": (_i64, [vp, _i64]),
            "or_rms_norm": (None, [vp, vp, _i64, _i64, ctypes.c_float, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        self.L = L

    @staticmethod
    def _p(a):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data

    def h2f(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.L.or_h2f_array(self._p(h), h.size, self._p(out))
        return out

    def f2h_rne(self, f):
        f = np.ascontiguousarray(f, np.float32)
        out = np.empty(f.shape, np.uint16)
        self.L.or_f2h_rne_array(self._p(f), f.size, self._p(out))
        return out

    def f2h_trunc(self, f):
        f = np.ascontiguousarray(f, np.float32)
        out = np.empty(f.shape, np.uint16)
        self.L.or_f2h_trunc_array(self._p(f), f.size, self._p(out))
        return out

    def bf16_to_f16_trunc(self, bf):
        bf = np.ascontiguousarray(bf, np.uint16)
        out = np.empty(bf.shape, np.uint16)
        self.L.or_bf16_to_f16_trunc_array(self._p(bf), bf.size, self._p(out))
        return out

    def unpack_awq(self, qweight, qzeros):
        qweight = np.ascontiguousarray(qweight, np.int32)
        qzeros = np.ascontiguousarray(qzeros, np.int32)
        K, N = qweight.shape[0], qweight.shape[1] * 8
        out = np.empty((K, N), np.int8)
        rc = self.L.or_unpack_awq(self._p(qweight), self._p(qzeros), K, N, self._p(out))
        assert rc == 0, rc
        return out

    def unpack_gptq(self, qweight, qzeros, g_idx, groups):
        qweight = np.ascontiguousarray(qweight, np.int32)
        qzeros = np.ascontiguousarray(qzeros, np.int32)
        g_idx = np.ascontiguousarray(g_idx, np.int32)
        K, N = qweight.shape[0] * 8, qweight.shape[1]
        out = np.empty((K, N), np.int8)
        rc = self.L.or_unpack_gptq(self._p(qweight), self._p(qzeros), self._p(g_idx), K, N, groups, self._p(out))
        return out if rc == 0 else rc

    def quantize_int4_awq(self, w_kn_u16):
        w = np.ascontiguousarray(w_kn_u16, np.uint16)
        K, N = w.shape
        qweight = np.empty((K, N // 8), np.int32)
        qzeros = np.empty((K // 128, N // 8), np.int32)
        scales = np.empty((K // 128, N), np.uint16)
        rc = self.L.or_quantize_int4_awq(self._p(w), K, N, self._p(qweight), self._p(qzeros), self._p(scales))
        assert rc == 0, rc
        return qweight, qzeros, scales

    def w4a16_matmul(self, x_u16, w8, scales_u16, nthreads=0):
        x = np.ascontiguousarray(x_u16, np.uint16)
        w8 = np.ascontiguousarray(w8, np.int8)
        s = np.ascontiguousarray(scales_u16, np.uint16)
        M, K = x.shape
        N = w8.shape[1]
        out = np.empty((M, N), np.float32)
        self.L.or_w4a16_matmul(self._p(x), self._p(w8), self._p(s), M, K, N, self._p(out), nthreads)
        return out

    def w4a16_dequant_f16(self, w8, scales_u16):
        w8 = np.ascontiguousarray(w8, np.int8)
        s = np.ascontiguousarray(scales_u16, np.uint16)
        K, N = w8.shape
        out = np.empty((K, N), np.uint16)
        self.L.or_w4a16_dequant_f16(self._p(w8), self._p(s), K, N, self._p(out))
        return out

    def quantize_i8(self, v, inv):
        return int(self.L.or_quantize_i8(ctypes.c_float(v), ctypes.c_float(inv)))

    def w8a8_quantize_weight(self, w_kn_u16):
        w = np.ascontiguousarray(w_kn_u16, np.uint16)
        K, N = w.shape
        q = np.empty((K, N), np.int8)
        s32 = np.empty(N, np.float32)
        s16 = np.empty(N, np.uint16)
        self.L.or_w8a8_quantize_weight(self._p(w), K, N, self._p(q), self._p(s32), self._p(s16))
        return q, s32, s16

    def w8a8_quantize_act(self, x_u16):
        x = np.ascontiguousarray(x_u16, np.uint16)
        M, K = x.shape
        q = np.empty((M, K), np.int8)
        s32 = np.empty(M, np.float32)
        s16 = np.empty(M, np.uint16)
        self.L.or_w8a8_quantize_act(self._p(x), M, K, self._p(q), self._p(s32), self._p(s16))
        return q, s32, s16

    def gemm_i32(self, x_i8, w_kn_i8, nthreads=0):
        x = np.ascontiguousarray(x_i8, np.int8)
        w = np.ascontiguousarray(w_kn_i8, np.int8)
        M, K = x.shape
        N = w.shape[1]
        out = np.empty((M, N), np.int32)
        self.L.or_gemm_i32(self._p(x), self._p(w), M, K, N, self._p(out), nthreads)
        return out

    def w8a8_dequant(self, acc, xs_f32, ws_f32):
        acc = np.ascontiguousarray(acc, np.int32)
        xs = np.ascontiguousarray(xs_f32, np.float32)
        ws = np.ascontiguousarray(ws_f32, np.float32)
        M, N = acc.shape
        out = np.empty((M, N), np.uint16)
        self.L.or_w8a8_dequant(self._p(acc), self._p(xs), self._p(ws), M, N, self._p(out))
        return out

    def silu_mul(self, g_u16, u_u16):
        g = np.ascontiguousarray(g_u16, np.uint16)
        u = np.ascontiguousarray(u_u16, np.uint16)
        out = np.empty(g.shape, np.uint16)
        self.L.or_silu_mul(self._p(g), self._p(u), g.size, self._p(out))
        return out

    def argmax_f16(self, logits_u16):
        x = np.ascontiguousarray(logits_u16, np.uint16)
        return int(self.L.or_argmax_f16(self._p(x), x.size))


    def rms_norm(self, x_u16, gamma_u16, eps):
        x = np.ascontiguousarray(x_u16, np.uint16)
        g = np.ascontiguousarray(gamma_u16, np.uint16)
        M, H = x.shape
        out = np.empty((M, H), np.uint16)
        self.L.or_rms_norm(self._p(x), self._p(g), M, H, float(eps), self._p(out))
        return out


_ORACLE = None


def load_oracle() -> Oracle:
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE


# ------------------------------------------------------------ generators --
def f16_normal(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    """fp16 bits of N(0, std) samples, rounded RNE by numpy's float16 cast."""
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16).view(np.uint16)


def synth_w4a16(rng: np.random.Generator, K: int, N: int, std: float = 0.02):
    """fp16 weights ~N(0, std) [K][N] quantised by the build-defined int4
    quantiser (oracle restatement) into AutoAWQ tensors.  N % 8 == 0."""
    o = load_oracle()
    w = f16_normal(rng, (K, N), std)
    qweight, qzeros, scales = o.quantize_int4_awq(w)
    return w, qweight, qzeros, scales


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def too_wide_gptq(rng, K, N):
    """GPTQ tensors whose act-order g_idx makes every 128-row block draw rows
    from a zero-1 group and a zero-16 group: values up to 31 levels apart."""
    G = K // 128
    qn = rng.integers(0, 16, (K, N)).astype(np.uint32)
    qweight = np.zeros((K // 8, N), np.uint32)
    for i in range(8):
        qweight |= qn[i::8] << (4 * i)
    zn = np.where(np.arange(G)[:, None] % 2 == 0, 0, 15) * np.ones((G, N), np.uint32)   # stored zeros 0 / 15
    qzeros = np.zeros((G, N // 8), np.uint32)
    for sl in range(8):
        qzeros |= zn[:, sl::8].astype(np.uint32) << (4 * sl)
    g_idx = (np.arange(K) % 2).astype(np.int32)
    return qweight.view(np.int32), qzeros.view(np.int32), g_idx
