"""Circuit breakers for the host hooks.

The rule a hooked piece follows when its fast path raises (the failure contract of the reference's hook
layer, comfy_mono_decode_xpu/guard.py:30-43):

* The piece trips: it stays off for the rest of the process (until `BOARD.clear`), and every later call
  goes straight to the host's own code.
* Only its first failure is logged, with the traceback; later failures of a tripped piece are counted.
* The failing call itself is answered by the host's code when the fast path had written no state yet.
  Once it has (KV rows, a recurrent state, x in place), the error propagates instead: the host's code
  would apply the same block a second time.
* An interrupt (KeyboardInterrupt, or the host's own cancel exception) is not a failure. It propagates
  unchanged and trips nothing. So does a `PassThrough` error, which a sub-path raises after it has
  tripped its own breaker.

A fast path runs under `shielded(piece, fast, host)`. It receives a `Progress` and calls
`progress.wrote()` right before its first state-modifying launch. A launch that fails does not prove that
nothing ran, so the mark goes before the launch, not after it.
"""
from __future__ import annotations

import logging
import threading

__all__ = ["BOARD", "Board", "PassThrough", "Progress", "is_interrupt", "shielded"]


class PassThrough(RuntimeError):
    """An error that propagates through `shielded` untouched, tripping nothing: a sub-path that already
    tripped its own breaker after writing state raises it."""


class Progress:
    """What a fast path has done so far: `written` once it may have modified state."""
    __slots__ = ("written",)

    def __init__(self):
        self.written = False

    def wrote(self):
        self.written = True


class _Trip:
    __slots__ = ("reason", "count")

    def __init__(self, reason):
        self.reason = reason
        self.count = 1


class Board:
    """The breakers of every hooked piece (by name). A piece with no entry is closed (fast path on)."""

    def __init__(self, log=None):
        self._lock = threading.Lock()
        self._trips: dict[str, _Trip] = {}
        self._log = log or logging.getLogger("mdx")

    def allows(self, piece: str) -> bool:
        return piece not in self._trips

    def trip(self, piece: str, exc: BaseException, *, wrote: bool = False) -> None:
        """Record a failure of `piece`; log it if it is the piece's first. An interrupt is no failure: it is
        re-raised as it is."""
        if is_interrupt(exc):
            raise exc
        reason = f"{type(exc).__name__}: {exc}"
        with self._lock:
            t = self._trips.get(piece)
            if t is None:
                self._trips[piece] = _Trip(reason)
            else:
                t.count += 1
                t.reason = reason
        if t is None:
            then = ("the call re-raises (state was already written)" if wrote
                    else "the call runs the host's own code")
            self._log.warning("[mdx] %s path failed and is switched off; %s", piece, then,
                              exc_info=(type(exc), exc, exc.__traceback__))

    def tripped(self) -> dict:
        """{piece: last failure text} of the pieces that are off."""
        with self._lock:
            return {p: t.reason for p, t in self._trips.items()}

    def failures(self, piece: str) -> int:
        with self._lock:
            t = self._trips.get(piece)
            return t.count if t else 0

    def clear(self, piece: str | None = None) -> None:
        """Switch one piece (or all) back on: for tests, or a host that reloads its model."""
        with self._lock:
            if piece is None:
                self._trips.clear()
            else:
                self._trips.pop(piece, None)


BOARD = Board()

_host_interrupts: tuple | None = None


def _interrupt_types() -> tuple:
    """KeyboardInterrupt plus the host's cancel exception when the host is importable (looked up once)."""
    global _host_interrupts
    if _host_interrupts is None:
        found = [KeyboardInterrupt]
        try:
            from comfy import model_management
            cls = getattr(model_management, "InterruptProcessingException", None)
            if isinstance(cls, type):
                found.append(cls)
        except Exception:
            pass
        _host_interrupts = tuple(found)
    return _host_interrupts


def is_interrupt(exc: BaseException) -> bool:
    return isinstance(exc, _interrupt_types())


def shielded(piece: str, fast, host, board: Board | None = None):
    """fast(progress) under the board's rule: its value, or host() when it failed before writing state."""
    board = BOARD if board is None else board
    progress = Progress()
    try:
        return fast(progress)
    except BaseException as exc:
        if is_interrupt(exc) or isinstance(exc, PassThrough) or not isinstance(exc, Exception):
            raise
        board.trip(piece, exc, wrote=progress.written)
        if progress.written:
            raise
    return host()
