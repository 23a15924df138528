"""ctypes bindings of the C oracle (liborc.so) and of the reference CPU build (_ref/libsepal_ref.so), numpy in and out.

Test infrastructure only. Every function here forwards to a C function whose header names the reference file:line it
restates (oracle/sepal_oracle.h) or to the reference's own compiled code (oracle/ref_harness.cpp).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_PATH = os.path.join(HERE, "liborc.so")
REF_PATH = os.path.join(HERE, "_ref", "libsepal_ref.so")

STORE, ADD, SWIGLU = 0, 1, 2

_orc = None
_ref = None


def build(quiet: bool = True) -> None:
    """Compiles liborc.so (and _ref when the reference sources are present) with make."""
    out = subprocess.run(["make", "-C", HERE, "-j8"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def lib():
    global _orc
    if _orc is None:
        if not os.path.exists(ORC_PATH):
            build()
        L = C.CDLL(ORC_PATH)
        sz, vp, f32, i32, d = C.c_size_t, C.c_void_p, C.c_float, C.c_int, C.c_double
        L.orc_quantize_group_r1.argtypes = [vp, sz, sz, sz, vp, sz, vp, sz]
        L.orc_quantize_block_r2.argtypes = [vp, sz, sz, sz, sz, vp, sz, vp, sz]
        L.orc_group_sums.argtypes = [vp, sz, vp, sz, sz, sz, sz, vp]
        L.orc_gemm_q8.argtypes = [vp, sz, vp, sz, sz, vp, sz, vp, sz, vp, sz, sz, sz, sz, i32]
        L.orc_gemm_q8y.argtypes = [vp, sz, vp, vp, sz, vp, vp, sz, sz, sz, sz, i32]
        L.orc_gemm_w8g.argtypes = [vp, sz, vp, sz, vp, sz, vp, sz, sz, sz, sz, i32]
        L.orc_rmsnorm_rows.argtypes = [vp, sz, vp, sz, sz, sz, vp, d]
        L.orc_exp_cephes.argtypes = [f32]
        L.orc_exp_cephes.restype = f32
        L.orc_silu_cephes.argtypes = [f32]
        L.orc_silu_cephes.restype = f32
        L.orc_swiglu_libm.argtypes = [f32, f32]
        L.orc_swiglu_libm.restype = f32
        L.orc_gate_up_source.argtypes = [sz, sz]
        L.orc_gate_up_source.restype = sz
        L.orc_s8_quantize_rows.argtypes = [vp, sz, vp, sz, sz, vp, sz, vp]
        L.orc_gemm_s8.argtypes = [vp, sz, vp, vp, sz, vp, vp, sz, sz, sz, sz]
        _orc = L
    return _orc


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            raise FileNotFoundError(REF_PATH + " (build with `make -C oracle` where the reference sources exist)")
        L = C.CDLL(REF_PATH)
        sz, vp, i32, d, u = C.c_size_t, C.c_void_p, C.c_int, C.c_double, C.c_uint
        L.ref_last_error.restype = C.c_char_p
        L.ref_i8_variant_is_z.restype = i32
        L.ref_default_threads.restype = u
        L.ref_pack_weight_i8.argtypes = [vp, sz, sz, vp, vp, vp]
        L.ref_pack_acts_i8.argtypes = [vp, sz, sz, vp, vp]
        L.ref_gemm_i8.argtypes = [vp, sz, vp, sz, sz, vp, i32, u]
        L.ref_gemm_i8_swiglu.argtypes = [vp, sz, vp, vp, sz, sz, vp, u]
        L.ref_rmsnorm.argtypes = [vp, sz, sz, vp, d, vp]
        L.ref_gemm_i8y.argtypes = [vp, sz, vp, sz, sz, vp, i32, u]
        L.ref_gemm_i8y_swiglu.argtypes = [vp, sz, vp, vp, sz, sz, vp, u]
        L.ref_pack_weight_i8y.argtypes = [vp, sz, sz, vp, vp]
        L.ref_time_mlp_block.argtypes = [vp, sz, vp, vp, vp, sz, sz, u, i32, C.POINTER(d), C.POINTER(d), C.POINTER(u)]
        _ref = L
    return _ref


def _chk(rc):
    if rc != 0:
        raise RuntimeError("reference: " + ref().ref_last_error().decode())


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i8(a):
    return np.ascontiguousarray(a, dtype=np.int8)


# ---- oracle ----------------------------------------------------------------------------------------------------------

def quantize_group_r1(w):
    w = _f32(w)
    rows, k = w.shape
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, k // 128), np.float32)
    lib().orc_quantize_group_r1(_p(w), k, rows, k, _p(q), k, _p(s), k // 128)
    return q, s


def quantize_block_r2(x, block=128):
    x = _f32(x)
    rows, k = x.shape
    nb = -(-k // block)
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, nb), np.float32)
    lib().orc_quantize_block_r2(_p(x), k, rows, k, block, _p(q), k, _p(s), nb)
    return q, s


def gate_up_order(inter):
    """Source-row index of every packed row of the 64-row gate/up interleave (gate rows first, then up rows)."""
    L = lib()
    return np.array([L.orc_gate_up_source(p, inter) for p in range(2 * inter)], dtype=np.int64)


def interleave_gate_up(gate, up):
    inter = gate.shape[0]
    return np.concatenate([gate, up], axis=0)[gate_up_order(inter)]


def group_sums(xq, wq):
    xq, wq = _i8(xq), _i8(wq)
    t, k = xq.shape
    n = wq.shape[0]
    g = -(-k // 128)
    out = np.zeros((g, t, n), np.int32)
    lib().orc_group_sums(_p(xq), k, _p(wq), k, t, n, k, _p(out))
    return out


def gemm_q8(xq, xs, wq, ws, epilogue=STORE, act_block=128, y=None):
    xq, wq, xs, ws = _i8(xq), _i8(wq), _f32(xs), _f32(ws)
    t, k = xq.shape
    n = wq.shape[0]
    ncols = n // 2 if epilogue == SWIGLU else n
    y = np.zeros((t, ncols), np.float32) if y is None else _f32(y).copy()
    lib().orc_gemm_q8(_p(xq), k, _p(xs), xs.shape[1], act_block, _p(wq), k, _p(ws), ws.shape[1], _p(y), ncols, t, n, k,
                      epilogue)
    return y


def s8_quantize_rows(x, smooth=None):
    """GPU int8 path's per-row quantizer (127 / amax rule, zero rows scale 0): int8 q and scales [rows]."""
    x = _f32(x)
    rows, cols = x.shape
    q = np.zeros((rows, cols), np.int8)
    s = np.zeros(rows, np.float32)
    sm = None if smooth is None else _f32(smooth)
    lib().orc_s8_quantize_rows(_p(x), cols, None if sm is None else _p(sm), rows, cols, _p(q), cols, _p(s))
    return q, s


def gemm_s8(xq, sx, wq, sw):
    """y = ((float)S * sx[t]) * sw[n] with S the exact integer sum, float32 [T, N]."""
    xq, wq = _i8(xq), _i8(wq)
    t, k = xq.shape
    n = wq.shape[0]
    y = np.zeros((t, n), np.float32)
    lib().orc_gemm_s8(_p(xq), k, _p(_f32(sx)), _p(wq), k, _p(_f32(sw)), _p(y), n, t, n, k)
    return y


def gemm_w8g(x, q, s, epilogue=STORE, y=None):
    x, q, s = _f32(x), _i8(q), _f32(s)
    t, k = x.shape
    n = q.shape[0]
    ncols = n // 2 if epilogue == SWIGLU else n
    y = np.zeros((t, ncols), np.float32) if y is None else _f32(y).copy()
    lib().orc_gemm_w8g(_p(x), k, _p(q), k, _p(s), s.shape[1], _p(y), ncols, t, n, k, epilogue)
    return y


def gemm_q8y(xq, xs, wq, ws, epilogue=STORE, y=None):
    """kernel_i8_y: xs [t] per row, ws [n] per feature, one int32 sum over k."""
    xq, wq, xs, ws = _i8(xq), _i8(wq), _f32(xs).reshape(-1), _f32(ws).reshape(-1)
    t, k = xq.shape
    n = wq.shape[0]
    ncols = n // 2 if epilogue == SWIGLU else n
    y = np.zeros((t, ncols), np.float32) if y is None else _f32(y).copy()
    lib().orc_gemm_q8y(_p(xq), k, _p(xs), _p(wq), k, _p(ws), _p(y), ncols, t, n, k, epilogue)
    return y


def rmsnorm_rows(x, eps=1e-6, w1=None):
    x = _f32(x)
    rows, cols = x.shape
    y = np.zeros_like(x)
    w = _f32(w1) if w1 is not None else None
    lib().orc_rmsnorm_rows(_p(x), cols, _p(y), cols, rows, cols, _p(w) if w is not None else None, eps)
    return y


def exp_cephes(v):
    L = lib()
    return np.array([L.orc_exp_cephes(float(a)) for a in np.ravel(v)], np.float32)


def silu_cephes(v):
    L = lib()
    return np.array([L.orc_silu_cephes(float(a)) for a in np.ravel(v)], np.float32)


def bf16_round(x):
    """float32 -> bfloat16 (nearest even) -> float32, vectorised (runner/src/cpu/gemm.cpp:73-78)."""
    b = _f32(x).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32)
    r = np.where(nan, (b >> 16) | 0x40, r).astype(np.uint32)
    return (r << 16).view(np.float32)


# ---- the compiled reference --------------------------------------------------------------------------------------------

def ref_pack_weight_i8(w):
    w = _f32(w)
    n, k = w.shape
    kb = -(-k // 128)
    q = np.zeros((n, k), np.int8)
    s = np.zeros((n, kb), np.float32)
    corr = np.zeros((n, kb), np.int32)
    _chk(ref().ref_pack_weight_i8(_p(w), n, k, _p(q), _p(s), _p(corr)))
    return q, s, corr


def ref_pack_acts_i8(x):
    x = _f32(x)
    rows, k = x.shape
    kb = -(-k // 128)
    q = np.zeros((rows, k), np.int8)
    s = np.zeros((rows, kb), np.float32)
    _chk(ref().ref_pack_acts_i8(_p(x), rows, k, _p(q), _p(s)))
    return q, s


def ref_gemm_i8(x, w, y=None, threads=4):
    x, w = _f32(x), _f32(w)
    rows, k = x.shape
    n = w.shape[0]
    acc = y is not None
    y = np.zeros((rows, n), np.float32) if y is None else _f32(y).copy()
    _chk(ref().ref_gemm_i8(_p(x), rows, _p(w), n, k, _p(y), int(acc), threads))
    return y


def ref_gemm_i8_swiglu(x, gate, up, threads=4):
    x, gate, up = _f32(x), _f32(gate), _f32(up)
    rows, k = x.shape
    n = gate.shape[0]
    y = np.zeros((rows, n), np.float32)
    _chk(ref().ref_gemm_i8_swiglu(_p(x), rows, _p(gate), _p(up), n, k, _p(y), threads))
    return y


def ref_gemm_i8y(x, w, y=None, threads=4):
    """The reference's AVX2 int8 path (I8_Y) on x [rows, k] and w [n, k]."""
    x, w = _f32(x), _f32(w)
    rows, k = x.shape
    n = w.shape[0]
    acc = y is not None
    y = np.zeros((rows, n), np.float32) if y is None else _f32(y).copy()
    _chk(ref().ref_gemm_i8y(_p(x), rows, _p(w), n, k, _p(y), int(acc), threads))
    return y


def ref_gemm_i8y_swiglu(x, gate, up, threads=4):
    x, gate, up = _f32(x), _f32(gate), _f32(up)
    rows, k = x.shape
    n = gate.shape[0]
    y = np.zeros((rows, n), np.float32)
    _chk(ref().ref_gemm_i8y_swiglu(_p(x), rows, _p(gate), _p(up), n, k, _p(y), threads))
    return y


def ref_pack_weight_i8y(w):
    w = _f32(w)
    n, k = w.shape
    q = np.zeros((n, k), np.int8)
    s = np.zeros(n, np.float32)
    _chk(ref().ref_pack_weight_i8y(_p(w), n, k, _p(q), _p(s)))
    return q, s


def ref_rmsnorm(x, eps=1e-6, w1=None):
    x = _f32(x)
    rows, cols = x.shape
    w = _f32(w1) if w1 is not None else np.ones(cols, np.float32)
    y = np.zeros_like(x)
    _chk(ref().ref_rmsnorm(_p(x), rows, cols, _p(w), eps, _p(y)))
    return y


def ref_time_mlp_block(x, gate, up, down, threads=0, reps=7):
    """Median seconds of one reference cpu-q8 MLP block call (pack_acts + gemm_packed x2), and of its packing alone."""
    x, gate, up, down = _f32(x), _f32(gate), _f32(up), _f32(down)
    rows, hidden = x.shape
    inter = gate.shape[0]
    tot, pk, th = C.c_double(), C.c_double(), C.c_uint()
    _chk(ref().ref_time_mlp_block(_p(x), rows, _p(gate), _p(up), _p(down), hidden, inter, threads, reps,
                                  C.byref(tot), C.byref(pk), C.byref(th)))
    return tot.value, pk.value, th.value
