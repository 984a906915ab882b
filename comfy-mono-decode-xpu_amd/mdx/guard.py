"""Failure handling shared by the host hooks (comfy_mono_decode_xpu/guard.py:1-51, the same contract).

A fast path that raises (a contract check of libmdx, a HIP error at launch, an out-of-memory) is logged
once with its traceback and switched off for the rest of the process; the call that hit the error runs
the host's original code instead when no state has been modified yet, and re-raises otherwise. A user
interrupt (the host's cancel exception, or KeyboardInterrupt) is not a failure: it passes through
unchanged and switches nothing off.
"""
from __future__ import annotations

import logging
import threading

_lock = threading.Lock()
_off = {}  # piece -> reason


def off(piece):
    return piece in _off


def _is_interrupt(exc):
    if isinstance(exc, KeyboardInterrupt):
        return True
    try:
        import comfy.model_management
        return isinstance(exc, comfy.model_management.InterruptProcessingException)
    except Exception:
        return False


def failed(piece, exc, *, can_fallback=True):
    """Record a failure of `piece` and switch it off; log only its first failure. Re-raises interrupts."""
    if _is_interrupt(exc):
        raise exc
    with _lock:
        first = piece not in _off
        _off[piece] = f"{type(exc).__name__}: {exc}"
    if first:
        action = "running the host's own path" if can_fallback else "aborting this call (state was already modified)"
        logging.warning("[mdx] %s path failed and is now disabled; %s", piece, action,
                        exc_info=(type(exc), exc, exc.__traceback__))


def disabled():
    with _lock:
        return dict(_off)


def reset(piece=None):
    """Switch a piece (or every piece) back on: for tests and for a host that reloads its model."""
    with _lock:
        if piece is None:
            _off.clear()
        else:
            _off.pop(piece, None)
