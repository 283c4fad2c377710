"""How an orth(X) result is judged: orthogonality, span, degenerate columns, determinism, sync-freedom, input intact.

The quantities and thresholds are the reference's (qrbench/metrics.py:1-20), restated here:

* span error: for each left singular direction u_i of X with sigma_i > SPAN_THRESH sigma_1 (an fp64 reference built
  from the fp32 input), s_i = ||(I - Q Q^T) u_i||; its size-free form is span_n = max_i s_i (sigma_i / sigma_1) / u32,
  in units of fp32 rounding (metrics.py:1-7). A result passes when span_n <= max(SPAN_RATIO x Householder's span_n
  on the same X, SPAN_FLOOR);
* orthogonality: max |Q^T Q - I| <= ORTH_TOL (1e-6, metrics.py:16); this project's own target is ORTH_TOL_TARGET;
* a column whose norm is below BAD_COL or that holds a non-finite value is degenerate (metrics.py:20).

The fp64 reference (QR of X in fp64, then the SVD of its R) is the reference's construction (metrics.py:23-28).
"""
from dataclasses import asdict, dataclass

import torch

U32 = 2.0 ** -24          # fp32 unit roundoff
ORTH_TOL = 1e-6           # metrics.py:16
ORTH_TOL_TARGET = 2e-7    # this project's orthogonality target
SPAN_THRESH = 1e-6        # metrics.py:17
SPAN_RATIO = 10.0         # metrics.py:18
SPAN_FLOOR = 100.0        # metrics.py:19
BAD_COL = 0.5             # metrics.py:20


class Reference:
    """fp64 ground truth of one fp32 X [K, r]: its singular values (descending) and left singular vectors, computed on
    the CPU from a double-precision QR of X and the SVD of the R factor"""

    def __init__(self, X):
        Xd = X.detach().double().cpu()
        Qd, Rd = torch.linalg.qr(Xd)
        Ur, self.sigma, _ = torch.linalg.svd(Rd)
        self.U = Qd @ Ur

    @property
    def cond(self):
        smin = float(self.sigma[-1])
        return float(self.sigma[0]) / smin if smin > 0 else float("inf")

    def span_errors(self, Qd):
        """(max s_i, span_n, number of directions checked) for an fp64 Q"""
        top = float(self.sigma[0])
        if top <= 0:
            return 0.0, 0.0, 0
        strong = self.sigma > SPAN_THRESH * top
        n = int(strong.sum())
        if n == 0:
            return 0.0, 0.0, 0
        Us = self.U[:, strong]
        resid = (Us - Qd @ (Qd.T @ Us)).norm(dim=0)
        weighted = resid * (self.sigma[strong] / top) / U32
        return float(resid.max()), float(weighted.max()), n


def reference(X):
    return Reference(X)


@dataclass
class Report:
    """What was measured on one result; failures() turns it into the list of broken requirements"""
    shape_ok: bool = True
    contiguous: bool = True       # information only (torch.linalg.qr returns a column-major Q)
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
        """messages of the requirements this result breaks (empty: it passes). span_ref: Householder's span_n on the
        same X (the span rule is skipped without it); orth_tol: the orthogonality bar"""
        if self.error:
            return [f"error: {self.error}"]
        span_lim = None if span_ref is None else max(SPAN_RATIO * span_ref, SPAN_FLOOR)
        return [msg for broken, msg in _rules(self, span_lim, orth_tol) if broken]

    def as_dict(self):
        return asdict(self)


def _rules(rep, span_lim, orth_tol):
    """(broken?, message) for every requirement, in reporting order"""
    yield not rep.shape_ok, "shape/dtype/device"
    yield not rep.finite, "non-finite"
    yield rep.bad_cols > 0, f"{rep.bad_cols} degenerate cols"
    yield not rep.orth <= orth_tol, f"orth {rep.orth:.1e}"          # NaN counts as broken
    if span_lim is not None:
        yield not rep.span_n <= span_lim, f"span {rep.span_n:.3g} > {span_lim:.3g}"
    yield not rep.deterministic, "non-deterministic"
    yield not rep.sync_free, "host sync"
    yield not rep.input_intact, "modified input"


def assess(Q, X, ref):
    """measure one output Q of orth(X) against ref = Reference(X); Q and X may live on any device"""
    K, r = X.shape
    rep = Report(shape_ok=tuple(Q.shape) == (K, r) and Q.dtype == torch.float32 and Q.device == X.device,
                 contiguous=Q.is_contiguous())
    if tuple(Q.shape) != (K, r):
        rep.finite, rep.bad_cols = False, r
        return rep
    Qd = Q.detach().double().cpu()
    col_finite = torch.isfinite(Qd).all(dim=0)
    col_norm = Qd.nan_to_num(0.0, 0.0, 0.0).norm(dim=0)
    rep.finite = bool(col_finite.all())
    rep.bad_cols = int((~col_finite | (col_norm < BAD_COL)).sum())
    if rep.finite:
        rep.orth = float((Qd.T @ Qd - torch.eye(r, dtype=torch.float64)).abs().max())
        rep.span_raw, rep.span_n, rep.n_dirs = ref.span_errors(Qd)
    return rep


def bits_equal(A, B):
    """bit-for-bit equality (NaN equals NaN, -0 differs from +0)"""
    if A.shape != B.shape or A.dtype != B.dtype:
        return False
    return bool(torch.equal(A.contiguous().view(torch.int32).cpu(), B.contiguous().view(torch.int32).cpu()))


def _sync_checked(call):
    """(Q, sync_free): one call under torch's sync-debug "error" mode, where a host synchronisation raises; a call
    that synchronises is repeated outside the mode so that its result can still be judged"""
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        return call(), True
    except RuntimeError as e:
        if "synchroniz" not in str(e).lower():
            raise
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    return call(), False


def check_call(fn, X, ref, check_sync=True):
    """(Report, Q) for fn(X): a warm-up call, a call checked for host synchronisation (GPU tensors only), a second
    call for bitwise determinism, then assess(); X must come back bit-identical. A crash is reported as an error, not
    raised (qrbench/metrics.py:109-141 defines these checks)."""
    on_gpu = X.device.type == "cuda"
    settle = torch.cuda.synchronize if on_gpu else (lambda: None)
    X0 = X.clone()
    try:
        fn(X)
        settle()
        Q1, sync_free = _sync_checked(lambda: fn(X)) if (check_sync and on_gpu) else (fn(X), True)
        Q2 = fn(X)
        settle()
    except Exception as e:  # noqa: BLE001 (a crashing method is a reported failure)
        if on_gpu:
            torch.cuda.set_sync_debug_mode(0)
        first = str(e).splitlines()[0][:120] if str(e) else ""
        return Report(error=f"{type(e).__name__}: {first}"), None
    rep = assess(Q1, X, ref)
    rep.sync_free = sync_free
    rep.deterministic = bits_equal(Q1, Q2)
    rep.input_intact = bits_equal(X, X0)
    return rep, Q1


def householder(X):
    """the span comparator: fp32 Householder QR, torch.linalg.qr(X)[0] (the TTF orth the reference replaces,
    qrbench/methods.py:47-50)"""
    return torch.linalg.qr(X)[0]
