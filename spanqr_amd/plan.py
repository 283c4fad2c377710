"""Plans: one native workspace per (K, r, batch, device, stream).

A plan owns the dust matrix, the Gram partials, the Cholesky factors, the solve buffers and the Cholesky's
grid-barrier counters (include/spanqr.h). The reference keeps module-level caches instead (the dust cache
candidates/kcholqr.py:26, the per-device barrier buffer candidates/kchol.py:12-18) and allocates the rest per call.
Plans are keyed by stream as well, so calls on different streams never share a workspace or a barrier.
"""
import atexit
import ctypes
import threading

import torch

from . import _lib

# At interpreter exit the process releases device memory by itself; destroying plans then would call into a HIP
# runtime (and any attached profiler) that may already be shutting down.
_SHUTTING_DOWN = [False]


@atexit.register
def _mark_shutdown():
    _SHUTTING_DOWN[0] = True


class Plan:
    def __init__(self, K, r, device_index, batch=1, borth=None):
        """borth = (b, reorth): a column-blocked plan for borth(X, b, reorth) (spanqr_plan_create_borth)"""
        self.K, self.r, self.device, self.batch = int(K), int(r), int(device_index), int(batch)
        h = ctypes.c_void_p()
        if borth is None:
            _lib.check(_lib.lib().spanqr_plan_create_batched(self.K, self.r, self.batch, self.device, ctypes.byref(h)))
        else:
            b, reorth = borth
            _lib.check(_lib.lib().spanqr_plan_create_borth(self.K, self.r, int(b), int(bool(reorth)), self.device,
                                                           ctypes.byref(h)))
        self.handle = h

    def query(self, what):
        return int(_lib.lib().spanqr_plan_query(self.handle, what))

    @property
    def splits(self):
        return self.query(_lib.Q_SPLITS)

    @property
    def split_rows(self):
        return self.query(_lib.Q_SPLIT_ROWS)

    @property
    def chol_grid(self):
        return self.query(_lib.Q_CHOL_GRID)

    @property
    def solve_rows(self):
        """rows per solve workgroup in the Cholesky's launch (0: the solve runs as its own launch)"""
        return self.query(_lib.Q_SOLVE_ROWS)

    @property
    def norm_partials(self):
        return self.query(_lib.Q_NORM_PARTIALS)

    @property
    def gram_short(self):
        """the one-launch Gram over 32x32 tiles (no separate split reduction)"""
        nt = (self.r + 63) // 64
        return self.norm_partials != 16 * nt * (nt + 1) // 2

    @property
    def chol_batch(self):
        return self.query(_lib.Q_CHOL_BATCH)

    def status(self):
        """synchronise the current stream and raise SpanqrError if a bounded Cholesky wait of the plan's last call
        gave up (that matrix's Q is NaN; spanqr_plan_status)"""
        _lib.check(_lib.lib().spanqr_plan_status(self.handle, stream_handle(self.device)))

    def close(self):
        if self.handle and not _SHUTTING_DOWN[0]:
            _lib.lib().spanqr_plan_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 (interpreter shutdown)
            pass


_PLANS = {}
_LOCK = threading.Lock()


def stream_handle(device):
    return torch.cuda.current_stream(device).cuda_stream


def get_plan(K, r, device, batch=1):
    """the cached plan for (K, r) and `batch` matrices per call on `device` and the current stream"""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (int(K), int(r), int(batch), idx, stream_handle(idx))
    with _LOCK:
        p = _PLANS.get(key)
        if p is None:
            p = Plan(K, r, idx, batch)
            _PLANS[key] = p
        return p


def get_borth_plan(K, r, b, reorth, device):
    """the cached column-blocked plan for borth(X [K, r], b, reorth) on `device` and the current stream"""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = ("borth", int(K), int(r), int(b), bool(reorth), idx, stream_handle(idx))
    with _LOCK:
        p = _PLANS.get(key)
        if p is None:
            p = Plan(K, r, idx, borth=(b, reorth))
            _PLANS[key] = p
        return p


def clear_plans():
    with _LOCK:
        for p in _PLANS.values():
            p.close()
        _PLANS.clear()
