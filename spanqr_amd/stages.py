"""Single stages of orth(X) on device tensors, for checking each MI355X kernel against the oracle.

Each wraps one stage entry point of include/spanqr.h and is named after the reference function it replaces:
  gram(A, ...)        tri.gram_f / tri.gram_split (candidates/tri.py:324-375, :255-297) and Y.T @ Y
  chol(G, npart, ...) the shift (kcholqr.py:107-109) + kchol.chol32 (candidates/kchol.py:35-44)
  chol32(G, tau)      kchol.chol32 itself: G already shifted, absolute pivot floor tau
  trsm(A, L, Li, ...) tri.trsm_f (candidates/tri.py:378-412)
  ns_step(Y, kahan)   one iteration of _ns_mm (candidates/kcholqr.py:16-23)
  dust(K, r)          _zdust (candidates/kcholqr.py:83-89), this project's generator
All tensors are fp32 (npart fp64) row-major on the plan's device; calls run on the current stream.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from .plan import get_plan, stream_handle

CB = 32


def _dev(t):
    return t.device


def dust_host(K, r):
    """the dust matrix as the library generates it on the host (numpy, no GPU needed)"""
    Z = np.empty((K, r), np.float32)
    _lib.check(_lib.lib().spanqr_dust_host(K, r, Z.ctypes.data_as(ctypes.c_void_p)))
    return Z


def dust(K, r, device="cuda"):
    """the plan's device copy of the dust matrix"""
    plan = get_plan(K, r, device)
    Z = torch.empty(K, r, device=device, dtype=torch.float32)
    _lib.check(_lib.lib().spanqr_plan_copy_dust(plan.handle, Z.data_ptr(), stream_handle(Z.device)))
    return Z


def scalars(K, r, device="cuda"):
    """{s, nrm0, tau0, nrm1, tau1, nrm2, tau2, barrier error} of the plan's last call (device fp32 [8])"""
    plan = get_plan(K, r, device)
    s = torch.empty(8, device=device, dtype=torch.float32)
    _lib.check(_lib.lib().spanqr_plan_copy_scalars(plan.handle, s.data_ptr(), stream_handle(s.device)))
    return s


def amax(X):
    """max|x| partials of X into the (K, r) plan (the pass-1 scale is derived from them)"""
    X = X.contiguous()
    plan = get_plan(X.shape[0], X.shape[1], _dev(X))
    _lib.check(_lib.lib().spanqr_stage_amax(plan.handle, X.data_ptr(), X.stride(0), stream_handle(X.device)))


def gram(A, kahan, use_scale=False):
    """(G [r, r], ||G||_F^2 partials fp64: 16 per upper 64x64 tile, or one per upper 32x32 tile where the plan runs
    the one-launch Gram of short X); use_scale: scale on load by the plan's pass-1 scale"""
    A = A.contiguous()
    K, r = A.shape
    plan = get_plan(K, r, _dev(A))
    G = torch.empty(r, r, device=A.device, dtype=torch.float32)
    npart = torch.empty(plan.query(_lib.Q_NORM_PARTIALS), device=A.device, dtype=torch.float64)
    _lib.check(_lib.lib().spanqr_stage_gram(plan.handle, A.data_ptr(), A.stride(0), int(bool(use_scale)),
                                            int(bool(kahan)), G.data_ptr(), npart.data_ptr(),
                                            stream_handle(A.device)))
    return G, npart


def chol(G, npart, K, alpha=1e-7, tau=1e-8):
    """(L [r, r], Li [r, 32], scal [nrm, tau, barrier error]) of G + fp32(alpha ||G||_F) I with pivot floor
    fp32(tau ||G||_F) + 1e-30; K selects the plan"""
    r = G.shape[0]
    plan = get_plan(K, r, _dev(G))
    L = torch.zeros(r, r, device=G.device, dtype=torch.float32)
    Li = torch.empty(r, CB, device=G.device, dtype=torch.float32)
    sc = torch.zeros(3, device=G.device, dtype=torch.float32)
    _lib.check(_lib.lib().spanqr_stage_chol(plan.handle, G.contiguous().data_ptr(), npart.contiguous().data_ptr(),
                                            float(alpha), float(tau), L.data_ptr(), Li.data_ptr(), sc.data_ptr(),
                                            stream_handle(G.device)))
    return L, Li, sc


def chol32(G, tau, K=None):
    """(L, Li) of the clamped Cholesky of G (already shifted) with absolute pivot floor tau (kchol.py:35-44)"""
    r = G.shape[0]
    K = r if K is None else K
    plan = get_plan(K, r, _dev(G))
    L = torch.zeros(r, r, device=G.device, dtype=torch.float32)
    Li = torch.empty(r, CB, device=G.device, dtype=torch.float32)
    _lib.check(_lib.lib().spanqr_stage_chol(plan.handle, G.contiguous().data_ptr(), None, 0.0, float(tau),
                                            L.data_ptr(), Li.data_ptr(), None, stream_handle(G.device)))
    return L, Li


def trsm(A, L, Li, pass1=False, eps=5e-7):
    """Y = A L^-T; pass1: operand fmaf(eps, Z, s * A) with the plan's dust and scale (call amax first)"""
    A = A.contiguous()
    K, r = A.shape
    plan = get_plan(K, r, _dev(A))
    Y = torch.empty(K, r, device=A.device, dtype=torch.float32)
    _lib.check(_lib.lib().spanqr_stage_trsm(plan.handle, A.data_ptr(), A.stride(0), int(bool(pass1)), float(eps),
                                            L.contiguous().data_ptr(), Li.contiguous().data_ptr(), Y.data_ptr(), r,
                                            stream_handle(A.device)))
    return Y


def ns_step(Y, kahan):
    """Y + Y fp32(I - Y^T Y) / 2"""
    Y = Y.contiguous()
    K, r = Y.shape
    plan = get_plan(K, r, _dev(Y))
    out = torch.empty_like(Y)
    _lib.check(_lib.lib().spanqr_stage_ns(plan.handle, Y.data_ptr(), Y.stride(0), int(bool(kahan)), out.data_ptr(), r,
                                          stream_handle(Y.device)))
    return out
