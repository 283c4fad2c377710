"""Accuracy and robustness checks for orth(X), restated from qrbench/metrics.py (reference).

Span error (metrics.py:1-7): for every left singular direction u_i of X with sigma_i > SPAN_THRESH * sigma_1 (fp64
reference computed from the fp32 input), s_i = ||(I - Q Q^T) u_i||, and span_n = max_i s_i (sigma_i / sigma_1) / u32
("units of fp32 rounding"). A method passes when span_n <= max(SPAN_RATIO * householder's span_n, SPAN_FLOOR).

Gates: the reference's orthogonality bar is 1e-6 (metrics.py:16); this project's target is tighter, ORTH_TOL_TARGET
= 2e-7, and both are reported.
"""
from dataclasses import asdict, dataclass

import torch

U32 = 2.0 ** -24
ORTH_TOL = 1e-6           # metrics.py:16
ORTH_TOL_TARGET = 2e-7    # this project's gate
SPAN_THRESH = 1e-6        # metrics.py:17
SPAN_RATIO = 10.0         # metrics.py:18
SPAN_FLOOR = 100.0        # metrics.py:19
BAD_COL = 0.5             # metrics.py:20


def reference(X):
    """fp64 SVD of the fp32 matrix X (via QR, on the CPU): singular values S and left vectors Ud [K, r]
    (metrics.py:23-28)"""
    Xd = X.detach().double().cpu()
    Qd, Rd = torch.linalg.qr(Xd)
    Ur, S, _ = torch.linalg.svd(Rd)
    return S, Qd @ Ur


def cond_of(ref):
    S = ref[0]
    return float(S[0] / S[-1]) if S[-1] > 0 else float("inf")


@dataclass
class Result:
    ok_shape: bool = True
    contiguous: bool = True
    finite: bool = True
    bad_cols: int = 0
    orth: float = float("nan")
    span_raw: float = 0.0
    span_n: float = 0.0
    n_dirs: int = 0
    deterministic: bool = True
    sync_free: bool = True
    input_intact: bool = True
    error: str = ""

    def failures(self, span_ref=None, orth_tol=ORTH_TOL):
        """hard-requirement failures (metrics.py:46-68); span_ref: Householder's span_n on the same matrix"""
        f = []
        if self.error:
            return [f"error: {self.error}"]
        if not self.ok_shape:
            f.append("shape/dtype/device")
        if not self.finite:
            f.append("non-finite")
        if self.bad_cols:
            f.append(f"{self.bad_cols} degenerate cols")
        if not (self.orth <= orth_tol):
            f.append(f"orth {self.orth:.1e}")
        lim = max(SPAN_RATIO * span_ref, SPAN_FLOOR) if span_ref is not None else None
        if lim is not None and not (self.span_n <= lim):
            f.append(f"span {self.span_n:.3g} > {lim:.3g}")
        if not self.deterministic:
            f.append("non-deterministic")
        if not self.sync_free:
            f.append("host sync")
        if not self.input_intact:
            f.append("modified input")
        return f

    def as_dict(self):
        return asdict(self)


def evaluate(Q, X, ref):
    """checks one output Q of orth(X) (metrics.py:74-100); Q, X: torch tensors on any device"""
    r_ = Result()
    K, r = X.shape
    r_.ok_shape = tuple(Q.shape) == (K, r) and Q.dtype == torch.float32 and Q.device == X.device
    r_.contiguous = Q.is_contiguous()
    if tuple(Q.shape) != (K, r):
        r_.finite, r_.bad_cols = False, r
        return r_
    Qd = Q.detach().double().cpu()
    fin_col = torch.isfinite(Qd).all(dim=0)
    r_.finite = bool(fin_col.all())
    norms = torch.where(fin_col, Qd.norm(dim=0), torch.zeros(r, dtype=torch.float64))
    r_.bad_cols = int(((~fin_col) | (norms < BAD_COL)).sum())
    if not r_.finite:
        return r_
    r_.orth = float((Qd.T @ Qd - torch.eye(r, dtype=torch.float64)).abs().max())
    S, Ud = ref
    if S[0] > 0:
        keep = S > SPAN_THRESH * S[0]
        Uk = Ud[:, keep]
        s = (Uk - Qd @ (Qd.T @ Uk)).norm(dim=0)
        r_.n_dirs = int(keep.sum())
        if r_.n_dirs:
            r_.span_raw = float(s.max())
            r_.span_n = float((s * (S[keep] / S[0]) / U32).max())
    return r_


def bits_equal(A, B):
    """bit-for-bit (NaN == NaN, -0 != +0) -- metrics.py:103-106"""
    return A.shape == B.shape and A.dtype == B.dtype and bool(torch.equal(
        A.contiguous().view(torch.int32).cpu(), B.contiguous().view(torch.int32).cpu()))


def run_checked(fn, X, ref, check_sync=True):
    """(Result, Q): calls fn(X) three times -- warm-up, under torch's sync-debug "error" mode (a host sync raises),
    again for determinism -- then evaluates and checks that X was left intact (metrics.py:109-141). On CPU tensors
    the sync check is skipped. A crash becomes a reported error."""
    on_gpu = X.device.type == "cuda"
    X0 = X.clone()
    res = Result()
    sync = torch.cuda.synchronize if on_gpu else (lambda: None)
    try:
        fn(X)
        sync()
        if check_sync and on_gpu:
            prev = torch.cuda.get_sync_debug_mode()
            torch.cuda.set_sync_debug_mode("error")
            try:
                Q1 = fn(X)
            except RuntimeError as e:
                if "synchroniz" not in str(e).lower():
                    raise
                res.sync_free = False
                torch.cuda.set_sync_debug_mode(prev)
                Q1 = fn(X)
            finally:
                torch.cuda.set_sync_debug_mode(prev)
        else:
            Q1 = fn(X)
        Q2 = fn(X)
        sync()
    except Exception as e:  # noqa: BLE001 (a crash is a reported failure)
        if on_gpu:
            torch.cuda.set_sync_debug_mode(0)
        res.error = f"{type(e).__name__}: {str(e).splitlines()[0][:120] if str(e) else ''}"
        return res, None
    ev = evaluate(Q1, X, ref)
    ev.sync_free = res.sync_free
    ev.deterministic = bits_equal(Q1, Q2)
    ev.input_intact = bits_equal(X, X0)
    return ev, Q1


def householder(X):
    """the span comparator: fp32 Householder QR (the current TTF orth, qrbench/methods.py:47-50)"""
    return torch.linalg.qr(X)[0]
