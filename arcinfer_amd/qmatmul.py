"""ctypes binding of libqmatmul.so (include/qmatmul.h) and torch-tensor conveniences.

The library is the product: this module only passes device pointers and sizes through the C ABI. It raises
QMatmulError for any non-zero status, and refuses to run when the library is not built (there is no fallback).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqmatmul.so")

QM_OK = 0
STATUS_NAMES = {0: "QM_OK", 1: "QM_ERR_ARG", 2: "QM_ERR_SHAPE", 3: "QM_ERR_TYPE", 4: "QM_ERR_HIP",
                5: "QM_ERR_NOMEM", 6: "QM_ERR_WORKSPACE"}

# every function include/qmatmul.h declares: (name, restype, argtypes)
_c = ctypes
_P = _c.c_void_p
_I = _c.c_int
_Z = _c.c_size_t
SIGNATURES = [
    ("qmatmul_init", _I, []),
    ("qmatmul_last_error", _c.c_char_p, []),
    ("qmatmul_sb_bytes", _Z, [_I]),
    ("qmatmul_weight_bytes", _Z, [_I, _I, _I]),
    ("qmatmul_prepare_weight", _I, [_I, _P, _I, _I, _I, _P, _c.POINTER(_P)]),
    ("qmatmul_release_weight", _I, [_P]),
    ("qmatmul_weight_info", _I, [_P, _c.POINTER(_I), _c.POINTER(_I), _c.POINTER(_I)]),
    ("qmatmul_quantize_act", _I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_quantize_act_ex", _I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_gemv", _I, [_P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P]),
    ("qmatmul_gemm", _I, [_P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P]),
    ("qmatmul_gemm_ex", _I, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _P]),
    ("qmatmul_gemm_noalloc", _I, [_P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P]),
    ("qmatmul_gemm_workspace_size", _Z, [_P, _I]),
    ("qmatmul_gemm_ws", _I, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _P, _Z, _P]),
    ("qmatmul_moe_workspace_size", _Z, [_I, _I, _I, _I, _I]),
    ("qmatmul_moe_route", _I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_moe_grouped", _I, [_P, _P, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P, _I, _P, _Z, _P]),
    ("qmatmul_moe_grouped_ex", _I, [_P, _P, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P, _P, _I, _I, _P, _I, _P, _Z, _P]),
    ("qmatmul_moe_ws_layout", _I, [_I, _I, _I, _I, _I, _P]),
    ("qmatmul_gemv_blocksums", _I, [_P, _P, _P, _I, _I, _P, _P, _P]),
    ("qmatmul_gemm_blocksums", _I, [_P, _P, _I, _I, _P, _P]),
    ("qmatmul_rmsnorm_quant", _I, [_P, _I, _P, _I, _I, _I, _c.c_float, _P, _P, _P, _P, _I, _P]),
    ("qmatmul_swiglu_quant", _I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_add_norm_quant", _I, [_P, _P, _P, _I, _c.c_float, _c.c_float, _P, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_rmsnorm_quant_ex", _I, [_P, _I, _P, _I, _I, _I, _c.c_float, _I, _P, _P, _P, _P, _I, _P]),
    ("qmatmul_swiglu_quant_ex", _I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_add_norm_quant_ex", _I, [_P, _P, _P, _I, _c.c_float, _c.c_float, _P, _I, _I, _I, _P, _P, _P, _P]),
    ("qmatmul_gguf_open", _I, [_c.c_char_p, _c.POINTER(_P)]),
    ("qmatmul_gguf_close", _I, [_P]),
    ("qmatmul_gguf_tensor_count", _I, [_P, _c.POINTER(_I)]),
    ("qmatmul_gguf_find_tensor", _I, [_P, _c.c_char_p, _c.POINTER(_I)]),
    ("qmatmul_gguf_tensor_info", _I, [_P, _I, _c.POINTER(_c.c_char_p), _c.POINTER(_I), _c.POINTER(_I),
                                      _c.POINTER(_c.c_uint64), _c.POINTER(_P), _c.POINTER(_c.c_uint64)]),
    ("qmatmul_gguf_get_int", _I, [_P, _c.c_char_p, _c.POINTER(_c.c_int64)]),
    ("qmatmul_gguf_get_float", _I, [_P, _c.c_char_p, _c.POINTER(_c.c_double)]),
    ("qmatmul_gguf_get_str", _I, [_P, _c.c_char_p, _c.POINTER(_c.c_char_p)]),
]


class QMatmulError(RuntimeError):
    def __init__(self, fn, status, msg):
        super().__init__(f"{fn}: {STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class MoeWsLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in
                ("ids", "wts", "counts", "cursor", "tstart", "tiles", "stok", "swt", "inv", "hq", "hsc", "y",
                 "hf", "total")] + [("slots", ctypes.c_int), ("max_tiles", ctypes.c_int), ("tile_rows", ctypes.c_int)]


_lib = None


def load_library(path=LIB_PATH):
    """Loads libqmatmul.so (built in-tree by arcinfer_amd.build); raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python -m arcinfer_amd.build` (there is no fallback path)")
    # One HIP runtime per process: torch ships its own libamdhip64.so.7 and loads it under another file name, so
    # it must be loaded first; the library's libamdhip64.so.7 dependency then binds to that copy (by soname)
    # instead of bringing in /opt/rocm's as a second runtime that would not know torch's memory and streams.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, res, args in SIGNATURES:
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def _call(name, *args):
    lib = load_library()
    st = getattr(lib, name)(*args)
    if st != QM_OK:
        raise QMatmulError(name, st, lib.qmatmul_last_error().decode())
    return st


# ---- torch helpers ------------------------------------------------------------------------------------------------
def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(stream)
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class QWeight:
    """A prepared weight (qm_weight*) from GGUF bytes: a uint8 tensor (device or CPU) or a numpy array. K is the raw
    row length; Q8_0 / Q4_0 / IQ4_NL / Q2_0 rows of K % 256 != 0 are padded with zero blocks, and self.K is then the
    prepared (padded) length, self.K_raw the given one."""

    def __init__(self, qtype, raw, rows, K, stream=None):
        import numpy as np
        import torch
        self.qtype, self.rows, self.K = int(qtype), int(rows), int(K)
        self.K_raw = self.K
        h = ctypes.c_void_p()
        if isinstance(raw, np.ndarray):
            raw = np.ascontiguousarray(raw)
            _call("qmatmul_prepare_weight", self.qtype, ctypes.c_void_p(raw.ctypes.data), 0, self.rows, self.K,
                  _stream(stream), ctypes.byref(h))
        else:
            assert isinstance(raw, torch.Tensor) and raw.is_contiguous()
            _call("qmatmul_prepare_weight", self.qtype, _ptr(raw), 1 if raw.is_cuda else 0, self.rows, self.K,
                  _stream(stream), ctypes.byref(h))
        self.handle = h
        k = ctypes.c_int()
        _call("qmatmul_weight_info", h, None, None, ctypes.byref(k))
        self.K = k.value

    @property
    def nbytes(self):
        return load_library().qmatmul_weight_bytes(self.qtype, self.rows, self.K)

    def release(self):
        if self.handle:
            _call("qmatmul_release_weight", self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.qmatmul_release_weight(self.handle)
                self.handle = None
        except Exception:
            pass


def quantize_act(x, M_stride=None, stream=None, act32=True):
    """x f32 [M, K] (cuda) -> (aq int8 [M_stride, K], asc f32 [K/32, M_stride], absum int16 [K/16, M_stride]);
    act32=False: per-256 scales, asc [K/256, M_stride] (qmatmul_quantize_act_ex)."""
    M, K = x.shape
    Ms = M if M_stride is None else M_stride
    aq, asc, absum = _out_acts(Ms, K, x.device, act32)
    if act32:
        _call("qmatmul_quantize_act", _ptr(x), x.stride(0), M, Ms, K, _ptr(aq), _ptr(asc), _ptr(absum), _stream(stream))
    else:
        _call("qmatmul_quantize_act_ex", _ptr(x), x.stride(0), M, Ms, K, 0, _ptr(aq), _ptr(asc), _ptr(absum),
              _stream(stream))
    return aq, asc, absum


def gemv(w, aq, asc, absum, T=1, C=None, ldc=None, c_off=0, accumulate=0, stream=None):
    import torch
    Ms = aq.shape[0]
    if C is None:
        C = torch.empty((T, w.rows), dtype=torch.float32, device=aq.device)
        ldc = w.rows
    _call("qmatmul_gemv", w.handle, _ptr(aq), _ptr(asc), _ptr(absum), Ms, T, _ptr(C),
          w.rows if ldc is None else ldc, c_off, accumulate, _stream(stream))
    return C


def gemm(w, aq, asc, absum, M=None, C=None, ldc=None, c_off=0, accumulate=0, stream=None, noalloc=False, act32=True):
    """qmatmul_gemm (noalloc=True: qmatmul_gemm_noalloc, the entry point that allocates no device memory;
    act32=False: qmatmul_gemm_ex with per-256 activation scales)."""
    import torch
    Ms = aq.shape[0]
    M = Ms if M is None else M
    if C is None:
        C = torch.empty((M, w.rows), dtype=torch.float32, device=aq.device)
        ldc = w.rows
    if not act32:
        if noalloc:
            raise ValueError("qmatmul_gemm_noalloc takes per-32 activation scales only")
        _call("qmatmul_gemm_ex", w.handle, _ptr(aq), _ptr(asc), _ptr(absum), M, Ms, 0, _ptr(C),
              w.rows if ldc is None else ldc, c_off, accumulate, _stream(stream))
        return C
    _call("qmatmul_gemm_noalloc" if noalloc else "qmatmul_gemm", w.handle, _ptr(aq), _ptr(asc), _ptr(absum), M, Ms, _ptr(C),
          w.rows if ldc is None else ldc, c_off, accumulate, _stream(stream))
    return C


def gemm_workspace_size(w, M):
    return load_library().qmatmul_gemm_workspace_size(w.handle, M)


def gemm_ws(w, aq, asc, absum, ws, M=None, C=None, ldc=None, c_off=0, accumulate=0, stream=None, act32=True):
    """qmatmul_gemm_ws: the prompt GEMM with a caller-owned workspace ws (a uint8 device tensor, or None when
    gemm_workspace_size(w, M) is 0)."""
    import torch
    Ms = aq.shape[0]
    M = Ms if M is None else M
    if C is None:
        C = torch.empty((M, w.rows), dtype=torch.float32, device=aq.device)
        ldc = w.rows
    _call("qmatmul_gemm_ws", w.handle, _ptr(aq), _ptr(asc), _ptr(absum), M, Ms, int(act32), _ptr(C),
          w.rows if ldc is None else ldc, c_off, accumulate, _ptr(ws), 0 if ws is None else ws.numel(),
          _stream(stream))
    return C


def gemv_blocksums(w, aq, absum, T=1, stream=None):
    import torch
    nb = w.K // 32
    isum = torch.empty((T, w.rows, nb), dtype=torch.int32, device=aq.device)
    msum = torch.empty((T, w.rows, nb), dtype=torch.int32, device=aq.device) if w.qtype in (12, 13, 10) else None
    _call("qmatmul_gemv_blocksums", w.handle, _ptr(aq), _ptr(absum), aq.shape[0], T, _ptr(isum), _ptr(msum),
          _stream(stream))
    return isum, msum


def gemm_blocksums(w, aq, M=None, stream=None):
    import torch
    M = aq.shape[0] if M is None else M
    isum = torch.empty((M, w.rows, w.K // 32), dtype=torch.int32, device=aq.device)
    _call("qmatmul_gemm_blocksums", w.handle, _ptr(aq), M, aq.shape[0], _ptr(isum), _stream(stream))
    return isum


def moe_route(logits, NU, NE=None, stream=None):
    import torch
    T, ldl = logits.shape
    NE = ldl if NE is None else NE
    ids = torch.empty((T, NU), dtype=torch.int32, device=logits.device)
    wts = torch.empty((T, NU), dtype=torch.float32, device=logits.device)
    counts = torch.empty((NE,), dtype=torch.int32, device=logits.device)
    _call("qmatmul_moe_route", _ptr(logits), ldl, T, NE, NU, _ptr(ids), _ptr(wts), _ptr(counts), _stream(stream))
    return ids, wts, counts


def moe_ws_layout(T, NE, NU, E, F):
    L = MoeWsLayout()
    _call("qmatmul_moe_ws_layout", T, NE, NU, E, F, ctypes.byref(L))
    return L


def moe_workspace(T, NE, NU, E, F, device="cuda"):
    import torch
    n = load_library().qmatmul_moe_workspace_size(T, NE, NU, E, F)
    return torch.empty((n,), dtype=torch.uint8, device=device)


def moe_grouped(gate, up, down, NE, logits, NU, aq, asc, x, ws, T=None, accumulate=0, stream=None, escale=None,
                sh=None, sh_gated=True):
    """qmatmul_moe_grouped, or qmatmul_moe_grouped_ex when escale [NE] or a shared expert's output sh [T, E] is
    given (sh_gated: gate it with sigmoid(logits[t, NE]), logits then having NE + 1 columns)."""
    T = logits.shape[0] if T is None else T
    if escale is None and sh is None:
        _call("qmatmul_moe_grouped", gate.handle, up.handle, down.handle, NE, _ptr(logits), logits.stride(0), T, NU,
              _ptr(aq), _ptr(asc), aq.shape[0], _ptr(x), accumulate, _ptr(ws), ws.numel(), _stream(stream))
    else:
        _call("qmatmul_moe_grouped_ex", gate.handle, up.handle, down.handle, NE, _ptr(logits), logits.stride(0), T,
              NU, _ptr(aq), _ptr(asc), aq.shape[0], _ptr(escale), _ptr(sh), 0 if sh is None else sh.stride(0),
              1 if sh_gated else 0, _ptr(x), accumulate, _ptr(ws), ws.numel(), _stream(stream))
    return x


def _out_acts(Ms, K, dev, act32=True):
    import torch
    return (torch.empty((Ms, K), dtype=torch.int8, device=dev),
            torch.empty((K // (32 if act32 else 256), Ms), dtype=torch.float32, device=dev),
            torch.empty((K // 16, Ms), dtype=torch.int16, device=dev))


def rmsnorm_quant(x, w, eps, M_stride=None, want_h=False, stream=None, act32=True):
    """x f32 [M, K] (cuda), w [K] -> (aq, asc, absum, h or None); act32=False: per-256 scales."""
    import torch
    M, K = x.shape
    Ms = M if M_stride is None else M_stride
    aq, asc, absum = _out_acts(Ms, K, x.device, act32)
    h = torch.empty((Ms, K), dtype=torch.float32, device=x.device) if want_h else None
    _call("qmatmul_rmsnorm_quant_ex", _ptr(x), x.stride(0), _ptr(w), K, M, Ms, float(eps), int(act32), _ptr(aq),
          _ptr(asc), _ptr(absum), _ptr(h), K, _stream(stream))
    return aq, asc, absum, h


def swiglu_quant(gu, F, fused=False, gelu=False, M_stride=None, stream=None, act32=True):
    M = gu.shape[0]
    Ms = M if M_stride is None else M_stride
    aq, asc, absum = _out_acts(Ms, F, gu.device, act32)
    _call("qmatmul_swiglu_quant_ex", _ptr(gu), gu.stride(0), F, M, Ms, int(fused), int(gelu), int(act32), _ptr(aq),
          _ptr(asc), _ptr(absum), _stream(stream))
    return aq, asc, absum


def add_norm_quant(x, t, w, eps, s, w2=None, M_stride=None, stream=None, act32=True):
    """Updates x in place; returns (aq, asc, absum)."""
    M, K = x.shape
    Ms = M if M_stride is None else M_stride
    aq, asc, absum = _out_acts(Ms, K, x.device, act32)
    _call("qmatmul_add_norm_quant_ex", _ptr(x), _ptr(t), _ptr(w), K, float(eps), float(s), _ptr(w2), M, Ms,
          int(act32), _ptr(aq), _ptr(asc), _ptr(absum), _stream(stream))
    return aq, asc, absum


class GgufTensor:
    def __init__(self, name, qtype, dims, data, nbytes):
        self.name, self.qtype, self.dims, self.data, self.nbytes = name, qtype, dims, data, nbytes

    @property
    def K(self):
        return self.dims[0]

    @property
    def rows(self):
        r = 1
        for d in self.dims[1:]:
            r *= d
        return r

    def numpy(self):
        """The tensor's bytes as a uint8 numpy view of the mapping (valid while the file is open)."""
        import numpy as np
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.nbytes).from_address(self.data))


class GgufFile:
    """A mapped GGUF file (qmatmul_gguf_*): tensors by name, metadata by key."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _call("qmatmul_gguf_open", os.fsencode(path), ctypes.byref(h))
        self.handle = h

    def __len__(self):
        n = ctypes.c_int()
        _call("qmatmul_gguf_tensor_count", self.handle, ctypes.byref(n))
        return n.value

    def tensor(self, key):
        i = key
        if isinstance(key, str):
            idx = ctypes.c_int()
            _call("qmatmul_gguf_find_tensor", self.handle, key.encode(), ctypes.byref(idx))
            i = idx.value
        name, t, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_uint64 * 8)()
        data, nb = ctypes.c_void_p(), ctypes.c_uint64()
        _call("qmatmul_gguf_tensor_info", self.handle, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd), dims,
              ctypes.byref(data), ctypes.byref(nb))
        return GgufTensor(name.value.decode(), t.value, [int(d) for d in dims[:nd.value]], data.value or 0, nb.value)

    def get_int(self, key):
        v = ctypes.c_int64()
        _call("qmatmul_gguf_get_int", self.handle, key.encode(), ctypes.byref(v))
        return v.value

    def get_float(self, key):
        v = ctypes.c_double()
        _call("qmatmul_gguf_get_float", self.handle, key.encode(), ctypes.byref(v))
        return v.value

    def get_str(self, key):
        v = ctypes.c_char_p()
        _call("qmatmul_gguf_get_str", self.handle, key.encode(), ctypes.byref(v))
        return v.value.decode()

    def close(self):
        if self.handle:
            _call("qmatmul_gguf_close", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
