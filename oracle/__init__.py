"""CPU oracle of the quantized matmul path -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over oracle/libqref.so (oracle/qref.c, a C restatement of the reference's CPU path). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this package; the product never does.

Pinning (each function is checked by something other than a retyped formula; tests/test_oracle_*.py):
  fp16_to_f32 / f32_to_fp16   exhaustive / randomized against numpy's IEEE half conversion
  decode_sb (4 types)         independent numpy encoders built from the GGML block structs (round trips of chosen
                              fields), closed forms (all-equal nibbles -> the published IQ4_NL values, zero scales),
                              codebook invariants, golden fixtures under tests/golden/
  quantize_act                special cases that separate the plausible variants (half-way ties -> even, v*(127/amax)
                              vs v/(amax/127), zero blocks, +-amax -> +-127), absum = brute-force sums
  blockdot (int sums)         brute-force int64 sums of decoded quants x int8 activations
  blockdot (f32)              double-precision dequantized reference, and the f32 reference matmul
  matmul_f32                  numpy float64 matmul of the dequantized rows
  moe_route                   textbook stable-sort top-k and softmax over the selection (tests/test_route.cpp recipe)
  moe_forward                 a numpy pipeline built from the pinned pieces (route, blockdot, quantize_act)
  rmsnorm_quant / swiglu_quant / add_norm_quant
                              closed forms (constant rows, zero rows, t = 0, silu/gelu limits and identities), float64
                              references of the norms, and the pinned quantizer on the returned f32 values
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqref.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        srcs = [os.path.join(HERE, f) for f in ("qref.c", "qref.h", "iq_tables.inc")]
        if not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < max(os.path.getmtime(s) for s in srcs):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        P, I = ctypes.c_void_p, ctypes.c_int
        _lib.qref_fp16_to_f32.restype = ctypes.c_float
        _lib.qref_fp16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.qref_f32_to_fp16.restype = ctypes.c_uint16
        _lib.qref_f32_to_fp16.argtypes = [ctypes.c_float]
        _lib.qref_sb_bytes.argtypes = [I]
        _lib.qref_decode_sb.argtypes = [I, P, P]
        _lib.qref_dequant_row.argtypes = [I, P, I, P]
        _lib.qref_quantize_act.argtypes = [P, I, I, I, I, P, P, P]
        _lib.qref_quantize_act.restype = None
        _lib.qref_blockdot.argtypes = [I, P, I, I, P, P, P, I, I, P, I, P, P, I, I]
        _lib.qref_matmul_f32.argtypes = [I, P, I, I, P, I, P, I]
        _lib.qref_moe_route.argtypes = [P, I, I, I, I, P, P, P]
        _lib.qref_moe_route.restype = None
        _lib.qref_moe_forward.argtypes = [I, P, I, P, I, P, I, I, I, P, I, I, I, P, P, I, P, I, I]
        _lib.qref_moe_route_ex.argtypes = [P, I, I, I, I, P, P, P, P]
        _lib.qref_moe_route_ex.restype = None
        _lib.qref_moe_forward_ex.argtypes = [I, P, I, P, I, P, I, I, I, P, I, I, I, P, P, I, P, P, I, I, P, I, I]
        Fl = ctypes.c_float
        _lib.qref_rmsnorm_quant.argtypes = [P, I, P, I, I, I, Fl, P, P, P, P]
        _lib.qref_rmsnorm_quant.restype = None
        _lib.qref_swiglu_quant.argtypes = [P, I, I, I, I, I, I, P, P, P, P]
        _lib.qref_swiglu_quant.restype = None
        _lib.qref_add_norm_quant.argtypes = [P, P, P, I, Fl, Fl, P, I, I, P, P, P, P]
        _lib.qref_add_norm_quant.restype = None
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


class SB(ctypes.Structure):
    _fields_ = [("d", ctypes.c_float), ("dmin", ctypes.c_float), ("d8", ctypes.c_float * 8),
                ("sc", ctypes.c_int * 8), ("mn", ctypes.c_int * 8), ("q", ctypes.c_int16 * 256),
                ("sc16", ctypes.c_int * 16), ("mn16", ctypes.c_int * 16)]


def fp16_to_f32(h):
    L = lib()
    return np.array([L.qref_fp16_to_f32(int(v)) for v in np.asarray(h, dtype=np.uint16).ravel()], dtype=np.float32)


def f32_to_fp16(x):
    L = lib()
    return np.array([L.qref_f32_to_fp16(float(v)) for v in np.asarray(x, dtype=np.float32).ravel()], dtype=np.uint16)


def sb_bytes(qtype):
    return lib().qref_sb_bytes(qtype)


def decode_sb(qtype, sb):
    """One superblock's bytes -> dict(d, dmin, d8[8], sc[8], mn[8], q[256])."""
    sb = np.ascontiguousarray(sb, dtype=np.uint8)
    o = SB()
    if lib().qref_decode_sb(qtype, _p(sb), ctypes.byref(o)):
        raise ValueError(f"decode_sb: type {qtype}")
    return {"d": o.d, "dmin": o.dmin, "d8": np.array(o.d8[:], np.float32), "sc": np.array(o.sc[:], np.int64),
            "mn": np.array(o.mn[:], np.int64), "q": np.array(o.q[:], np.int64), "sc16": np.array(o.sc16[:], np.int64),
            "mn16": np.array(o.mn16[:], np.int64)}


def dequant_rows(qtype, W, K):
    """uint8 [N, row_bytes] -> float32 [N, K]"""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    N = W.shape[0]
    out = np.empty((N, K), dtype=np.float32)
    rb = W.shape[1]
    for n in range(N):
        row = W[n]
        if lib().qref_dequant_row(qtype, _p(row), K, ctypes.c_void_p(out.ctypes.data + 4 * K * n)):
            raise ValueError("dequant_row failed")
    assert rb == W.shape[1]
    return out


def quantize_act(x, M_stride=None, act32=True):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    Ms = M if M_stride is None else M_stride
    B = 32 if act32 else 256
    aq = np.empty((Ms, K), dtype=np.int8)
    asc = np.empty((K // B, Ms), dtype=np.float32)
    absum = np.empty((K // 16, Ms), dtype=np.int16)
    lib().qref_quantize_act(_p(x), M, K, Ms, 1 if act32 else 0, _p(aq), _p(asc), _p(absum))
    return aq, asc, absum


def blockdot(qtype, W, K, aq, asc, absum, M=None, blocksums=False, col_stride=1, nthreads=0):
    """int8 block-dot product -> C f32 [M, N] (+ isum, msum int32 [M, N, K/32] with blocksums)."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    N = W.shape[0]
    Ms = aq.shape[0]
    M = Ms if M is None else M
    aq = np.ascontiguousarray(aq)
    asc = np.ascontiguousarray(asc, dtype=np.float32)
    absum = None if absum is None else np.ascontiguousarray(absum, dtype=np.int16)
    C = np.zeros((M, N), dtype=np.float32)
    isum = np.zeros((M, N, K // 32), dtype=np.int32) if blocksums else None
    msum = np.zeros((M, N, K // 32), dtype=np.int32) if blocksums else None
    if lib().qref_blockdot(qtype, _p(W), N, K, _p(aq), _p(asc), _p(absum), M, Ms, _p(C), N, _p(isum), _p(msum),
                           col_stride, nthreads):
        raise ValueError("blockdot failed")
    return (C, isum, msum) if blocksums else C


def blockdot256(qtype, W, K, aq, asc256, absum, M=None, col_stride=1, nthreads=0):
    """The product with per-256 activation scales (the reference's act32 = false GEMM, zero/kernels/gemm.cl:413-447:
    per superblock res += asc * (d * sum_b sc*isum) - asc * (dmin * sum_b mn*bsum)). Every 32-block of a
    superblock carries the superblock's scale, so in qref_blockdot's double accumulation the per-block form
    sum_b asc * d * (sc*isum) equals the reference's superblock form exactly; this expands asc [K/256][M_stride] to
    the per-32 layout and calls it."""
    asc32 = np.repeat(np.ascontiguousarray(asc256, dtype=np.float32), 8, axis=0)
    return blockdot(qtype, W, K, aq, asc32, absum, M=M, col_stride=col_stride, nthreads=nthreads)


def matmul_f32(qtype, W, K, X, nthreads=0):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32)
    N, M = W.shape[0], X.shape[0]
    Y = np.empty((M, N), dtype=np.float32)
    if lib().qref_matmul_f32(qtype, _p(W), N, K, _p(X), M, _p(Y), nthreads):
        raise ValueError("matmul_f32 failed")
    return Y


def moe_route(logits, NU, NE=None, escale=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, ldl = logits.shape
    NE = ldl if NE is None else NE
    ids = np.empty((T, NU), dtype=np.int32)
    wts = np.empty((T, NU), dtype=np.float32)
    counts = np.empty((NE,), dtype=np.int32)
    esc = None if escale is None else np.ascontiguousarray(escale, dtype=np.float32)
    lib().qref_moe_route_ex(_p(logits), ldl, T, NE, NU, _p(esc), _p(ids), _p(wts),
                            _p(counts))
    return ids, wts, counts


def moe_forward(tg, Wg, tu, Wu, td, Wd, NE, E, F, logits, NU, aq, asc, x=None, accumulate=False, nthreads=0,
                escale=None, sh=None, sh_gated=True):
    """The MoE FFN of qref_moe_forward_ex: logits [T, ldl] (ldl > NE when a gated shared expert is given),
    escale [NE] or None, sh [T, E] (the shared expert's output) or None."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T = logits.shape[0]
    out = np.zeros((T, E), dtype=np.float32) if x is None else np.ascontiguousarray(x, dtype=np.float32).copy()
    aq = np.ascontiguousarray(aq)
    asc = np.ascontiguousarray(asc, dtype=np.float32)
    Wg, Wu, Wd = (np.ascontiguousarray(w, dtype=np.uint8) for w in (Wg, Wu, Wd))
    esc = None if escale is None else np.ascontiguousarray(escale, dtype=np.float32)
    shv = None if sh is None else np.ascontiguousarray(sh, dtype=np.float32)
    if lib().qref_moe_forward_ex(tg, _p(Wg), tu, _p(Wu), td, _p(Wd), NE, E, F, _p(logits), logits.shape[1], T, NU,
                                 _p(aq), _p(asc), aq.shape[0], _p(esc),
                                 _p(shv), E, 1 if sh_gated else 0, _p(out),
                                 1 if accumulate else 0, nthreads):
        raise ValueError("moe_forward failed")
    return out


def _acts(Ms, K):
    return (np.zeros((Ms, K), dtype=np.int8), np.zeros((K // 32, Ms), dtype=np.float32),
            np.zeros((K // 16, Ms), dtype=np.int16), np.zeros((Ms, K), dtype=np.float32))


def rmsnorm_quant(x, w, eps, M_stride=None):
    """x f32 [M, K] (row stride K), w [K] -> (aq, asc, absum, h) (zero rows M..M_stride-1)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = x.shape
    Ms = M if M_stride is None else M_stride
    aq, asc, absum, h = _acts(Ms, K)
    lib().qref_rmsnorm_quant(_p(x), K, _p(w), K, M, Ms, float(eps), _p(aq), _p(asc), _p(absum), _p(h))
    return aq, asc, absum, h


def swiglu_quant(gu, F, fused=False, gelu=False, M_stride=None):
    """gu f32 [M, 2F] ([gate | up]) or [M, F] with fused -> (aq, asc, absum, h)."""
    gu = np.ascontiguousarray(gu, dtype=np.float32)
    M, ldg = gu.shape
    Ms = M if M_stride is None else M_stride
    aq, asc, absum, h = _acts(Ms, F)
    lib().qref_swiglu_quant(_p(gu), ldg, F, M, Ms, int(fused), int(gelu), _p(aq), _p(asc), _p(absum), _p(h))
    return aq, asc, absum, h


def add_norm_quant(x, t, w, eps, s, w2=None, M_stride=None):
    """Returns (x_new, aq, asc, absum, h); x is not modified."""
    xn = np.ascontiguousarray(x, dtype=np.float32).copy()
    t = np.ascontiguousarray(t, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    w2 = None if w2 is None else np.ascontiguousarray(w2, dtype=np.float32)
    M, K = xn.shape
    Ms = M if M_stride is None else M_stride
    aq, asc, absum, h = _acts(Ms, K)
    lib().qref_add_norm_quant(_p(xn), _p(t), _p(w), K, float(eps), float(s), _p(w2), M, Ms, _p(aq), _p(asc),
                              _p(absum), _p(h))
    return xn, aq, asc, absum, h
