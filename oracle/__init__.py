"""CPU oracle for the quantized frozen-base LoRA linear — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline). The product path (``loractl_amd``) never imports it.

This module is a thin numpy front end over ``lrq_oracle.c`` (built into
``liblrq_oracle.so`` by ``oracle/Makefile``); each function names the
reference behaviour it restates. See the header of ``lrq_oracle.c`` for the
per-function citations and for which test pins which function.

Parity status: every function here is pinned by a reference golden, a
reference fixture pair, a closed-form invariant or a brute-force check
(``tests/test_oracle.py``). Nothing is "parity unpinned" except two
behaviours the reference itself leaves open and this build defines:
rounding of exact .5 ties (half away from zero, Rust ``f32::round``) and the
all-zero block (scale 0, q 0).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblrq_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile ``liblrq_oracle.so`` with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        L.lrq_o_f32_to_bf16.restype = ctypes.c_uint16
        L.lrq_o_f32_to_bf16.argtypes = [ctypes.c_float]
        L.lrq_o_round_bf16.argtypes = [_f32p, _u16p, _i64]
        L.lrq_o_quantize.restype = ctypes.c_int
        L.lrq_o_quantize.argtypes = [_f32p, _i64, _i64, _i64, ctypes.c_int, _i8p, _f32p]
        L.lrq_o_dequant_q.argtypes = [_i8p, _f32p, _i64, _i64, _i64, _f32p]
        L.lrq_o_pack_int4.argtypes = [_i8p, _i64, _i64, _u8p]
        L.lrq_o_unpack_int4.argtypes = [_u8p, _i64, _i64, _i8p]
        L.lrq_o_dequant_int4.argtypes = [_u8p, _f32p, _i64, _i64, _i64, _f32p]
        L.lrq_o_dequant_chunk_rows.restype = _i64
        L.lrq_o_dequant_chunk_rows.argtypes = [_i64, _i64, ctypes.c_uint64, _i64p, _i64]
        L.lrq_o_fp8_decode.restype = ctypes.c_float
        L.lrq_o_fp8_decode.argtypes = [ctypes.c_uint8]
        L.lrq_o_fp8_encode.restype = ctypes.c_uint8
        L.lrq_o_fp8_encode.argtypes = [ctypes.c_float]
        L.lrq_o_fp8_quantize.argtypes = [_f32p, _i64, _i64, ctypes.c_int, _u8p, _f32p]
        L.lrq_o_fp8_dequant.argtypes = [_u8p, _i64, _i64, _f32p, _i64, _f32p]
        vp = ctypes.c_void_p
        L.lrq_o_linear_fwd.argtypes = [vp, vp, vp, vp, vp, ctypes.c_double, _i64, _i64, _i64, _i64, vp, vp]
        L.lrq_o_linear_bwd.argtypes = [vp, vp, vp, vp, ctypes.c_double, vp, _i64, _i64, _i64, _i64, vp, vp, vp]
        L.lrq_o_cpu_dequant_int4.restype = ctypes.c_int
        L.lrq_o_cpu_dequant_int4.argtypes = [vp, vp, _i64, _i64, _i64, vp]
        L.lrq_o_cpu_dequant_int8.restype = ctypes.c_int
        L.lrq_o_cpu_dequant_int8.argtypes = [vp, vp, _i64, _i64, _i64, vp]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- bf16
def bf16_bits(x) -> np.ndarray:
    """f32 -> bf16 bit patterns (uint16), round-to-nearest-even."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().lrq_o_round_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_round(x) -> np.ndarray:
    """Round f32 values to the nearest bf16 and return them as f32."""
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def bf16_from_bits(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- int quant
def quantize(w, group: int, qmax: int):
    """Block-symmetric quantization (quant.rs:47-82). Returns (q int8 [N,K], scales f32 [N,K/g])."""
    w = _c(w, np.float32)
    N, K = w.shape
    if K % group:
        raise ValueError(f"linear weight [{N}, {K}]: the input dim must be a multiple of the quant block ({group})")
    q = np.empty((N, K), np.int8)
    s = np.empty((N, K // group), np.float32)
    rc = lib().lrq_o_quantize(w, N, K, group, qmax, q, s)
    assert rc == 0
    return q, s


def dequant_q(q, scales, group: int) -> np.ndarray:
    q = _c(q, np.int8)
    s = _c(scales, np.float32)
    N, K = q.shape
    out = np.empty((N, K), np.float32)
    lib().lrq_o_dequant_q(q, s, N, K, group, out)
    return out


def pack_int4(q) -> np.ndarray:
    q = _c(q, np.int8)
    N, K = q.shape
    out = np.empty((N, K // 2), np.uint8)
    lib().lrq_o_pack_int4(q, N, K, out)
    return out


def unpack_int4(packed, K: int) -> np.ndarray:
    p = _c(packed, np.uint8)
    N = p.shape[0]
    out = np.empty((N, K), np.int8)
    lib().lrq_o_unpack_int4(p, N, K, out)
    return out


def dequant_int4(packed, scales, K: int, group: int) -> np.ndarray:
    p = _c(packed, np.uint8)
    s = _c(scales, np.float32)
    N = p.shape[0]
    out = np.empty((N, K), np.float32)
    lib().lrq_o_dequant_int4(p, s, N, K, group, out)
    return out


def quantize_int4_packed(w, group: int):
    """w f32 [N,K] -> (packed u8 [N,K/2], scales f32 [N,K/g])."""
    q, s = quantize(w, group, 7)
    return pack_int4(q), s


def dequant_chunk_rows(d_out: int, d_in: int, chunk_bytes: int) -> list[int]:
    buf = np.zeros(max(1, d_out), np.int64)
    n = lib().lrq_o_dequant_chunk_rows(d_out, d_in, chunk_bytes, buf, buf.size)
    return [int(v) for v in buf[:n]]


# ---------------------------------------------------------------- fp8
def fp8_lut() -> np.ndarray:
    return np.array([lib().lrq_o_fp8_decode(b) for b in range(256)], np.float32)


def fp8_encode(x) -> np.ndarray:
    x = np.asarray(x, np.float32)
    f = np.vectorize(lambda v: lib().lrq_o_fp8_encode(float(v)), otypes=[np.uint8])
    return f(x) if x.size else x.astype(np.uint8)


def fp8_quantize(w, per_channel: bool):
    w = _c(w, np.float32)
    N, K = w.shape
    b = np.empty((N, K), np.uint8)
    s = np.empty((N if per_channel else 1,), np.float32)
    lib().lrq_o_fp8_quantize(w, N, K, int(per_channel), b, s)
    return b, s


def fp8_dequant(bytes_, scales) -> np.ndarray:
    b = _c(bytes_, np.uint8)
    s = _c(np.atleast_1d(scales), np.float32).reshape(-1)
    N, K = b.shape
    out = np.empty((N, K), np.float32)
    lib().lrq_o_fp8_dequant(b, N, K, s, s.size, out)
    return out


# ---------------------------------------------------------------- linear
def linear_fwd(X, Wdq, A=None, B=None, s: float = 1.0, bias=None):
    """Y = X Wdq^T + s (X A) B (+ bias), f64 accumulation. Returns (Y, T=s X A)."""
    X = _c(X, np.float32)
    W = _c(Wdq, np.float32)
    M, K = X.shape
    N = W.shape[0]
    r = 0 if A is None else A.shape[1]
    A = None if A is None else _c(A, np.float32)
    B = None if B is None else _c(B, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    Y = np.empty((M, N), np.float32)
    T = np.empty((M, max(r, 1)), np.float32)
    lib().lrq_o_linear_fwd(_ptr(X), _ptr(W), _ptr(A), _ptr(B), _ptr(bias), float(s), M, N, K, r,
                           _ptr(Y), _ptr(T) if r else None)
    return Y, (T if r else None)


def linear_bwd(X, Wdq, A, B, s: float, dY):
    """Returns (dX [M,K], dA [K,r], dB [r,N]) of linear_fwd, f64 accumulation."""
    X = _c(X, np.float32)
    W = _c(Wdq, np.float32)
    dY = _c(dY, np.float32)
    M, K = X.shape
    N = W.shape[0]
    r = 0 if A is None else A.shape[1]
    A = None if A is None else _c(A, np.float32)
    B = None if B is None else _c(B, np.float32)
    dX = np.empty((M, K), np.float32)
    dA = np.empty((K, max(r, 1)), np.float32)
    dB = np.empty((max(r, 1), N), np.float32)
    lib().lrq_o_linear_bwd(_ptr(X), _ptr(W), _ptr(A), _ptr(B), float(s), _ptr(dY), M, N, K, r,
                           _ptr(dX), _ptr(dA) if r else None, _ptr(dB) if r else None)
    return dX, (dA if r else None), (dB if r else None)


def rel_deviation(ours, reference) -> float:
    """Peak-normalized max deviation (crates/loractl-core/src/accuracy.rs:107-131)."""
    a = np.asarray(ours, np.float64).reshape(-1)
    b = np.asarray(reference, np.float64).reshape(-1)
    if a.size == 0 or a.size != b.size or not (np.isfinite(a).all() and np.isfinite(b).all()):
        return float("inf")
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-12))


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-300))


# ---------------------------------------------------------------- cpu baseline
def blas_info() -> str:
    """The BLAS numpy's f32 GEMMs run on, and its thread count."""
    try:
        import threadpoolctl

        for d in threadpoolctl.threadpool_info():
            if d.get("user_api") == "blas":
                return f"{d.get('internal_api')} {d.get('version')} ({d.get('architecture')}), " \
                       f"{d.get('num_threads')} threads"
    except Exception:  # noqa: BLE001 - informational only
        pass
    return "numpy BLAS"


def blas_threads() -> int:
    try:
        import threadpoolctl

        for d in threadpoolctl.threadpool_info():
            if d.get("user_api") == "blas":
                return int(d.get("num_threads") or 1)
    except Exception:  # noqa: BLE001 - informational only
        pass
    return 1


class CpuFwdInt4:
    """The reference's CPU forward in f32, burn-ndarray's way
    (quant.rs:175-176, :232-233; lora.rs:199-203): dequantize the whole
    weight to an f32 [N, K] (lrq_o_cpu_dequant_int4, OpenMP), then f32 GEMMs
    Y = X Wdq^T, T = s X A, Y += T B in numpy's cache-blocked SGEMM (the
    stand-in for burn-ndarray's matrixmultiply/gemm crates)."""

    def __init__(self, packed, scales, group, X, A, B, s):
        self.packed = _c(packed, np.uint8)
        self.scales = _c(scales, np.float32)
        self.g = group
        self.X = _c(X, np.float32)
        self.A = _c(A, np.float32)
        self.B = _c(B, np.float32)
        self.s = np.float32(s)
        self.M, self.K = self.X.shape
        self.N = self.B.shape[1]
        self.Wdq = np.empty((self.N, self.K), np.float32)

    def dequant(self) -> int:
        return lib().lrq_o_cpu_dequant_int4(_ptr(self.packed), _ptr(self.scales), self.g, self.N, self.K,
                                            _ptr(self.Wdq))

    def forward(self) -> int:
        """One forward; returns the threads of the dequant (the GEMMs use
        ``blas_threads()``)."""
        th = self.dequant()
        self.Y = self.X @ self.Wdq.T
        self.T = (self.X @ self.A) * self.s
        self.Y += self.T @ self.B
        return th

    def run(self) -> int:
        return self.forward()


class CpuStepInt4(CpuFwdInt4):
    """One forward + backward, the reference's CPU way: the forward above,
    then a second f32 dequant of the whole weight (the reference's backward
    re-dequantizes, quant.rs:250-251) and the f32 GEMMs dX = dY Wdq,
    U = s dY B^T, dX += U A^T, dA = X^T U, dB = T^T dY (the autodiff of the
    two LoRA Linears)."""

    def __init__(self, packed, scales, group, X, A, B, s, dY):
        super().__init__(packed, scales, group, X, A, B, s)
        self.dY = _c(dY, np.float32)

    def run(self) -> int:
        th = self.forward()
        self.dequant()
        self.dX = self.dY @ self.Wdq
        self.U = (self.dY @ self.B.T) * self.s
        self.dX += self.U @ self.A.T
        self.dA = self.X.T @ self.U
        self.dB = self.T.T @ self.dY
        return th


class CpuStepInt8(CpuStepInt4):
    """The same step over an int8 (Q8S) weight: q int8 [N, K] and scales
    [N, K/g], dequantized to f32 on every forward and every backward
    (lrq_o_cpu_dequant_int8, OpenMP)."""

    def __init__(self, q, scales, group, X, A, B, s, dY):
        super().__init__(np.zeros((1, 1), np.uint8), scales, group, X, A, B, s, dY)
        self.q = _c(q, np.int8)

    def dequant(self) -> int:
        return lib().lrq_o_cpu_dequant_int8(_ptr(self.q), _ptr(self.scales), self.g, self.N, self.K,
                                            _ptr(self.Wdq))


class CpuStepF32(CpuStepInt4):
    """One forward + backward over a Plain f32 weight [N, K] (an fp8
    checkpoint decoded once at load, fp8.rs:306-318, and kept full
    precision): the same f32 GEMMs, no per-pass dequantization."""

    def __init__(self, W, X, A, B, s, dY):
        W = _c(W, np.float32)
        N, K = W.shape
        super().__init__(np.zeros((N, K // 2), np.uint8), np.zeros((N, 1), np.float32), K, X, A, B, s, dY)
        self.Wdq = W

    def dequant(self) -> int:
        return 1
