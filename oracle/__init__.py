"""CPU oracle for spanqr's orth(X) (kcholf): the checker for the MI355X library.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and
only to check or time the CPU restatement; the product (spanqr_amd, orth.py) never imports it.

kcholf_oracle.c (loaded below through ctypes) restates candidates/kcholqr.py:92-112 (kcholqr_f) and
candidates/kbig.py:69-95 (borth, the r > 512 branch of orth.py:18-19) bit-exactly: it fixes the order of every
floating-point operation, and the HIP kernels follow the same order, so GPU results are compared bit for bit.

Arrays are numpy, row-major, float32 unless stated.
"""
import contextlib
import ctypes
import os
import subprocess

import numpy as np

TB = 64
CB = 32
BK = 32
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_kcholf.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p


def build():
    """compile the C oracle in place (gcc; no GPU needed)"""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _bind(L):
    c_int, c_long, c_float = ctypes.c_int, ctypes.c_long, ctypes.c_float
    L.spqo_amax.argtypes = [_f32p, c_long, c_int, c_int]
    L.spqo_amax.restype = c_float
    L.spqo_pow2_scale.argtypes = [c_float]
    L.spqo_pow2_scale.restype = c_float
    L.spqo_rsqrt.argtypes = [c_float]
    L.spqo_rsqrt.restype = c_float
    L.spqo_dust.argtypes = [c_int, c_int, _f32p]
    L.spqo_gram_splits.argtypes = [c_int, c_int]
    L.spqo_gram_splits.restype = c_int
    L.spqo_gram.argtypes = [_f32p, c_long, c_int, c_int, c_float, c_int, c_int, c_int, _f32p, _vp]
    L.spqo_norm.argtypes = [_f64p, c_int]
    L.spqo_norm.restype = c_float
    L.spqo_shift.argtypes = [_f32p, c_int, c_float, c_float, c_float]
    L.spqo_shift.restype = c_float
    L.spqo_diag_factor.argtypes = [_f32p, c_long, c_float, _f32p, c_long, _f32p]
    L.spqo_chol.argtypes = [_f32p, c_int, c_float, _f32p, _f32p]
    L.spqo_trsm.argtypes = [_f32p, c_long, c_int, c_int, c_float, c_int, _vp, c_float, _f32p, _f32p, _f32p, c_long]
    L.spqo_ns_D.argtypes = [_f32p, c_int, _f32p]
    L.spqo_ns_apply.argtypes = [_f32p, c_long, c_int, c_int, _f32p, _f32p, c_long]
    L.spqo_orth.argtypes = [_f32p, c_long, c_int, c_int, c_int, c_float, c_float, c_float, c_int, _f32p, c_long,
                            _vp, _vp, _vp, _vp, _vp]
    L.spqo_orth_dust.argtypes = [_f32p, c_long, c_int, c_int, c_int, c_float, c_float, c_float, c_int, _vp, c_long,
                                 _f32p, c_long]
    L.spqo_split_rows.argtypes = [c_int, c_int]
    L.spqo_split_rows.restype = c_int
    L.spqo_gram_short.argtypes = [c_int, c_int]
    L.spqo_gram_short.restype = c_int
    L.spqo_gram_short_rows.argtypes = [c_int]
    L.spqo_gram_short_rows.restype = c_int
    L.spqo_npart_count.argtypes = [c_int, c_int]
    L.spqo_npart_count.restype = c_int
    L.spqo_gram_rows.argtypes = [c_int, c_int]
    L.spqo_gram_rows.restype = c_int
    L.spqo_xgram.argtypes = [_vp, c_long, c_int, c_int, _vp, c_long, c_int, c_int, _f32p]
    L.spqo_project.argtypes = [_vp, c_long, c_int, c_int, _vp, c_long, c_int, c_int, _f32p, c_long]
    L.spqo_borth.argtypes = [_f32p, c_long, c_int, c_int, c_int, c_int, c_float, c_float, c_float, c_int, _f32p,
                             c_long]
    L.spqo_rsqrt64.argtypes = [ctypes.c_double]
    L.spqo_rsqrt64.restype = ctypes.c_double
    L.spqo_diag_factor64.argtypes = [_f64p, c_long, ctypes.c_double, _f64p, c_long, _f64p]
    L.spqo_chol64.argtypes = [_f64p, c_int, ctypes.c_double, _f64p, _f64p, _f32p, _f32p]
    return L


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = _bind(ctypes.CDLL(_LIB_PATH))
    return _lib


@contextlib.contextmanager
def planted(n, workdir):
    """inside the block, every function of this module runs a copy of the oracle built with planted defect n
    (kcholf_oracle.c, PLANTED(n)); for the tests that show the oracle's checks catch such mistakes"""
    global _lib
    path = os.path.join(str(workdir), f"liboracle_plant{n}.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", _HERE, f"PLANT={n}", f"OUT={path}"], check=True)
    saved = lib()
    _lib = _bind(ctypes.CDLL(path))
    try:
        yield
    finally:
        _lib = saved


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- scale (kcholqr.py:29-30, :102) ----

def amax(X):
    X = _c32(X)
    return np.float32(lib().spqo_amax(X, X.shape[1], X.shape[0], X.shape[1]))


def pow2_scale(m):
    return np.float32(lib().spqo_pow2_scale(float(np.float32(m))))


def rsqrt(x):
    return np.float32(lib().spqo_rsqrt(float(np.float32(x))))


# ---- dust (kcholqr.py:83-89, own generator) ----

def dust(K, r):
    Z = np.empty((K, r), np.float32)
    lib().spqo_dust(K, r, Z)
    return Z


# ---- Gram (tri.py:255-297, 324-375) ----

def gram(A, KS, kahan, s=None):
    """(G [r, r], norm partials fp64: 16 per upper 64x64 tile, or one per upper 32x32 tile for short X, the form
    gram_short(K, r) picks); s: scale on load (None: no scale)"""
    A = _c32(A)
    K, r = A.shape
    G = np.empty((r, r), np.float32)
    npart = np.empty(npart_count(K, r), np.float64)
    lib().spqo_gram(A, r, K, r, 1.0 if s is None else float(s), s is not None, int(bool(kahan)), KS, G,
                    _ptr(npart))
    return G, npart


def gram_splits(K, KS):
    return lib().spqo_gram_splits(K, KS)


def gram_short(K, r):
    """the Gram's form for X [K, r]: True for the one-launch form over 32x32 tiles (two row splits)"""
    return bool(lib().spqo_gram_short(K, r))


def gram_rows(K, r):
    """rows per Gram split for X [K, r], either form (the library's spanqr_split_rows)"""
    return lib().spqo_gram_rows(K, r)


def npart_count(K, r):
    return lib().spqo_npart_count(K, r)


def norm(npart):
    npart = np.ascontiguousarray(npart, np.float64)
    return np.float32(lib().spqo_norm(npart, npart.size))


def shift(G, nrm, alpha=1e-7, tau_rel=1e-8):
    """returns (G + shift I, tau) -- kcholqr.py:107-109"""
    G = _c32(G).copy()
    tau = lib().spqo_shift(G, G.shape[0], float(nrm), float(np.float32(alpha)), float(np.float32(tau_rel)))
    return G, np.float32(tau)


# ---- Cholesky (chol.cu:115-271) ----

def diag_factor(D, tau):
    D = _c32(D).copy()
    L = np.zeros((CB, CB), np.float32)
    Li = np.zeros((CB, CB), np.float32)
    lib().spqo_diag_factor(D, CB, float(tau), L, CB, Li)
    return L, Li


def chol(G, tau):
    """(L [r, r] lower, Li [r, 32] diagonal-tile inverses) of the clamped factorisation of G (lower tiles read)"""
    A = _c32(G).copy()
    r = A.shape[0]
    L = np.zeros((r, r), np.float32)
    Li = np.zeros((r, CB), np.float32)
    lib().spqo_chol(A, r, float(tau), L, Li)
    return L, Li


# ---- TRSM (tri.py:378-412) ----

def trsm(A, L, Li, s=None, Z=None, eps=0.0):
    """Y = A L^-T; with s and Z given, the operand is fmaf(eps, Z, s * A) (the pass-1 fused input)"""
    A = _c32(A)
    K, r = A.shape
    Y = np.empty((K, r), np.float32)
    pass1 = s is not None
    Zc = _c32(Z) if pass1 else None
    lib().spqo_trsm(A, r, K, r, float(s) if pass1 else 1.0, int(pass1), _ptr(Zc), float(np.float32(eps)),
                    _c32(L), _c32(Li), Y, r)
    return Y


# ---- Newton-Schulz (kcholqr.py:16-23) ----

def ns_D(G):
    G = _c32(G)
    D = np.empty_like(G)
    lib().spqo_ns_D(G, G.shape[0], D)
    return D


def ns_apply(Y, D):
    Y = _c32(Y)
    K, r = Y.shape
    Q = np.empty((K, r), np.float32)
    lib().spqo_ns_apply(Y, r, K, r, _c32(D), Q, r)
    return Q


# ---- whole call (kcholqr.py:92-112) ----

def orth(X, KS, eps=5e-7, alpha=1e-7, tau=1e-8, ns=2, stages=False):
    """Q = orth(X). KS: rows per Gram split (the plan's choice; a multiple of 32). With stages=True also returns
    dict(G=[3,r,r] shifted Grams, L=[3,r,r], Li=[3,r,32], Y=[3,K,r], s, nrm[3], tau[3])."""
    X = _c32(X)
    K, r = X.shape
    Q = np.empty((K, r), np.float32)
    if stages:
        Gs = np.empty((3, r, r), np.float32)
        Ls = np.empty((3, r, r), np.float32)
        Lis = np.empty((3, r, CB), np.float32)
        Ys = np.empty((3, K, r), np.float32)
        sc = np.empty(7, np.float32)
        ptrs = [_ptr(a) for a in (Gs, Ls, Lis, Ys, sc)]
    else:
        ptrs = [None] * 5
    lib().spqo_orth(X, r, K, r, KS, float(np.float32(eps)), float(np.float32(alpha)), float(np.float32(tau)), ns,
                    Q, r, *ptrs)
    if not stages:
        return Q
    return Q, dict(G=Gs, L=Ls, Li=Lis, Y=Ys, s=sc[0], nrm=sc[1::2].copy(), tau=sc[2::2].copy())


def orth_dust(X, Z, KS, eps=5e-7, alpha=1e-7, tau=1e-8, ns=2):
    """kcholqr_f with the dust Z [K, r] given (kbig.py:48-63, _kf); Z may be a column slice of a wider dust"""
    X = _c32(X)
    K, r = X.shape
    Z = np.asarray(Z, np.float32)
    assert Z.shape == (K, r) and Z.strides[1] == 4
    Q = np.empty((K, r), np.float32)
    lib().spqo_orth_dust(X, r, K, r, KS, float(np.float32(eps)), float(np.float32(alpha)), float(np.float32(tau)), ns,
                         Z.ctypes.data_as(ctypes.c_void_p), Z.strides[0] // 4, Q, r)
    return Q


# ---- column-blocked path (kbig.py:69-95) ----

BW = 256   # the borth block width orth.py:19 uses


def split_rows(K, U):
    """rows per split of a split-K product with U 64x64 output tiles (the Gram's rule; a function of (K, U) only)"""
    return lib().spqo_split_rows(K, U)


def xgram(P, C, KS):
    """T = P^T C for P [K, j], C [K, b]: fp32 chains per split of KS rows, fp64 across splits"""
    P, C = _c32(P), _c32(C)
    K, j = P.shape
    b = C.shape[1]
    assert C.shape[0] == K
    T = np.empty((j, b), np.float32)
    lib().spqo_xgram(_ptr(P), j, K, j, _ptr(C), b, b, KS, T)
    return T


def project(P, C, KS):
    """C - P (P^T C) (kbig.py:88-89)"""
    P, C = _c32(P), _c32(C)
    K, j = P.shape
    b = C.shape[1]
    Out = np.empty((K, b), np.float32)
    lib().spqo_project(_ptr(P), j, K, j, _ptr(C), b, b, KS, Out, b)
    return Out


def borth(X, b=BW, reorth=True, eps=5e-7, alpha=1e-7, tau=1e-8, ns=2):
    """Q = borth(X, b, reorth) (kbig.py:69-95), b a multiple of 32, r > b a multiple of b; the default b is the 256
    orth.py:19 passes"""
    X = _c32(X)
    K, r = X.shape
    assert b % 32 == 0 and r % b == 0 and r > b
    Q = np.empty((K, r), np.float32)
    lib().spqo_borth(X, r, K, r, b, int(bool(reorth)), float(np.float32(eps)), float(np.float32(alpha)),
                     float(np.float32(tau)), ns, Q, r)
    return Q


# ---- fp64 clamped Cholesky (kchol.py:47-57, chol.cu:278-281) ----

def rsqrt64(x):
    return float(lib().spqo_rsqrt64(float(x)))


def chol64(G, tau):
    """(L [r, r] fp64, Li [r, 32] fp64, Lf, Lif fp32 copies) of the clamped factorisation of fp64 G"""
    A = np.ascontiguousarray(G, np.float64).copy()
    r = A.shape[0]
    L = np.zeros((r, r), np.float64)
    Li = np.zeros((r, CB), np.float64)
    Lf = np.zeros((r, r), np.float32)
    Lif = np.zeros((r, CB), np.float32)
    lib().spqo_chol64(A, r, float(tau), L, Li, Lf, Lif)
    return L, Li, Lf, Lif
