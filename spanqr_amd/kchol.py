"""The clamped Cholesky kernels of candidates/kchol.py on the MI355X, same arguments and results:

    chol32(G, tau) -> (L, Li)            kchol.py:35-44 -> chol_f32 (candidates/cuk/chol.cu:273-276)
    chol64(G, tau) -> (L64, Li64, Lf, Lif)   kchol.py:47-57 -> chol_f64 (candidates/cuk/chol.cu:278-281)

Enqueued on the current stream; tau may be a float or a device tensor (no host synchronisation either way,
kchol.py:24-28)."""
import ctypes
import threading

import torch

from . import _lib
from .plan import get_plan, stream_handle

TB = 32   # kchol.py:8
_plans = {}
_lock = threading.Lock()


class _Plan64:
    def __init__(self, n, device_index):
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().spanqr_chol64_plan_create(n, device_index, ctypes.byref(h)))
        self.handle = h

    def __del__(self):
        try:
            if getattr(self, "handle", None) and self.handle.value and _lib._lib is not None:
                _lib.lib().spanqr_chol64_plan_destroy(self.handle)
        except Exception:  # noqa: BLE001 (interpreter shutdown)
            pass


def _plan(n, dev):
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (n, idx, stream_handle(dev))
    with _lock:
        p = _plans.get(key)
        if p is None:
            p = _plans[key] = _Plan64(n, idx)
        return p


def _tau(tau, G):
    """the pivot floor as a 1-element device tensor of G's dtype (kchol.py:24-28)"""
    if torch.is_tensor(tau):
        return tau.reshape(1).to(device=G.device, dtype=G.dtype).contiguous()
    return torch.full((1,), float(tau), device=G.device, dtype=G.dtype)


def chol32(G, tau):
    """G [n, n] fp32 on a ROCm device (lower triangle read, not modified), n a multiple of 32 up to 1024. Returns
    (L, Li): L lower-triangular (zeros above), Li [n, 32] the inverses of L's 32 x 32 diagonal tiles. Pivots below tau
    (or NaN) are clamped to tau; no shift is added (kchol.py:35-44). Runs the fp32 factorisation of orth's passes
    (one kernel, flag-synchronised 32 x 32 tiles) on a plan for [n, n]."""
    if not isinstance(G, torch.Tensor) or G.dim() != 2 or G.shape[0] != G.shape[1]:
        raise ValueError("chol32: G must be a square 2-D tensor")
    if G.dtype != torch.float32:
        raise TypeError(f"chol32: G must be float32, got {G.dtype}")
    if G.device.type != "cuda":
        raise TypeError("chol32: G must be on a GPU (ROCm device); there is no CPU implementation")
    n = G.shape[0]
    if n % TB or not TB <= n <= 1024:
        raise ValueError(f"chol32: n = {n} must be a multiple of {TB} in [{TB}, 1024]")
    if G.stride(1) != 1:
        G = G.contiguous()
    dev = G.device
    L = torch.empty(n, n, device=dev, dtype=torch.float32)
    Li = torch.empty(n, TB, device=dev, dtype=torch.float32)
    t = _tau(tau, G)
    plan = get_plan(n, n, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().spanqr_chol32(plan.handle, G.data_ptr(), G.stride(0), t.data_ptr(), L.data_ptr(), n,
                                            Li.data_ptr(), stream_handle(dev)))
    return L, Li


def chol64(G, tau):
    """G [n, n] fp64 on a ROCm device (lower triangle read), n a multiple of 32 up to 1024. Returns (L64, Li64, Lf, Lif):
    L lower-triangular (zeros above), Li [n, 32] the inverses of L's 32 x 32 diagonal tiles, and fp32 copies of both."""
    if not isinstance(G, torch.Tensor) or G.dim() != 2 or G.shape[0] != G.shape[1]:
        raise ValueError("chol64: G must be a square 2-D tensor")
    if G.dtype != torch.float64:
        raise TypeError(f"chol64: G must be float64, got {G.dtype}")
    if G.device.type != "cuda":
        raise TypeError("chol64: G must be on a GPU (ROCm device); there is no CPU implementation")
    n = G.shape[0]
    if n % TB or n > 1024:
        raise ValueError(f"chol64: n = {n} must be a multiple of {TB} up to 1024")
    G = G.contiguous()
    dev = G.device
    L = torch.empty(n, n, device=dev, dtype=torch.float64)
    Li = torch.empty(n, TB, device=dev, dtype=torch.float64)
    Lf = torch.empty(n, n, device=dev, dtype=torch.float32)
    Lif = torch.empty(n, TB, device=dev, dtype=torch.float32)
    t = _tau(tau, G)
    p = _plan(n, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().spanqr_chol64(p.handle, G.data_ptr(), n, t.data_ptr(), L.data_ptr(), Li.data_ptr(),
                                            Lf.data_ptr(), Lif.data_ptr(), stream_handle(dev)))
    return L, Li, Lf, Lif


def status(n, device=None):
    """synchronise and raise if a bounded wait of the last fp64 factorisation of size n on this stream gave up"""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    p = _plan(n, dev)
    _lib.check(_lib.lib().spanqr_chol64_status(p.handle, stream_handle(dev)))
