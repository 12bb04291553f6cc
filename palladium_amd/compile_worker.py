"""Compiling in a helper process (opt-in: PALLADIUM_COMPILE_ISOLATED=1).

hiprtc runs the LLVM AMDGPU backend inside the calling process, so a
backend crash (an `LLVM ERROR` abort) ends that process. With isolation on,
`runtime.Kernel.load` sends the source to a long-lived child process, which
compiles it with `ph_compile_code_object` (hiprtc only: the child makes no
other HIP call), and loads the returned code object with
`ph_load_code_object`. If the child dies, sends a reply that does not
parse, or does not deliver a whole reply within PALLADIUM_COMPILE_TIMEOUT
seconds (default 900; the child is then stopped), the parent raises
`CompileError` and starts a fresh child on the next compile.

Protocol over the child's stdin and a private copy of its stdout: a request
is a 4-byte big-endian length and a JSON header {"name", "mode", "arch",
"size"} followed by `size` bytes of source; a reply is a length-prefixed
JSON header {"ok": true, "size"} followed by the code object, or {"ok":
false, "error"}. The child points its file descriptor 1 at stderr before
anything else runs, so a stray write by native code cannot corrupt a
reply; its stderr goes to a temporary file, which cannot fill up and stall
it the way an unread pipe would, and whose tail is reported if it dies.
"""

from __future__ import annotations

import json
import os
import select
import struct
import subprocess
import sys
import tempfile
import threading
import time
from typing import Any

__all__ = ["compile_isolated", "isolation_enabled"]

_HEADER_MAX = 1 << 20


def isolation_enabled() -> bool:
    return os.environ.get("PALLADIUM_COMPILE_ISOLATED", "") not in ("", "0")


def compile_timeout() -> float:
    """PALLADIUM_COMPILE_TIMEOUT in seconds (default 900), checked."""
    from palladium_amd.errors import CompileError

    raw = os.environ.get("PALLADIUM_COMPILE_TIMEOUT", "900")
    try:
        value = float(raw)
    except ValueError:
        raise CompileError(f"PALLADIUM_COMPILE_TIMEOUT={raw!r} is not a number of seconds") from None
    if not value > 0 or value != value or value == float("inf"):
        raise CompileError(f"PALLADIUM_COMPILE_TIMEOUT={raw!r} must be a positive, finite number of seconds")
    return value


def _send(stream: Any, header: dict, payload: bytes) -> None:
    h = json.dumps(header).encode()
    stream.write(struct.pack(">I", len(h)) + h + payload)
    stream.flush()


def _recv(stream: Any) -> tuple[dict, bytes] | None:
    """Blocking read of one message (the child's side)."""
    raw = stream.read(4)
    if len(raw) < 4:
        return None
    (n,) = struct.unpack(">I", raw)
    header = json.loads(stream.read(n).decode())
    size = int(header.get("size", 0))
    payload = stream.read(size) if size else b""
    return header, payload


class _ReplyError(Exception):
    """The reply was cut off, malformed or late."""


def _read_exact(fd: int, n: int, deadline: float) -> bytes:
    chunks = []
    while n:
        left = deadline - time.monotonic()
        if left <= 0:
            raise TimeoutError
        ready, _, _ = select.select([fd], [], [], left)
        if not ready:
            raise TimeoutError
        chunk = os.read(fd, min(n, 1 << 20))
        if not chunk:
            raise _ReplyError("the compiler process closed its reply stream")
        chunks.append(chunk)
        n -= len(chunk)
    return b"".join(chunks)


def _recv_by(fd: int, deadline: float) -> tuple[dict, bytes]:
    """One whole reply, or TimeoutError / _ReplyError."""
    (n,) = struct.unpack(">I", _read_exact(fd, 4, deadline))
    if n > _HEADER_MAX:
        raise _ReplyError(f"reply header of {n} bytes")
    try:
        header = json.loads(_read_exact(fd, n, deadline).decode())
        size = int(header.get("size", 0))
    except (ValueError, UnicodeDecodeError, AttributeError) as e:
        raise _ReplyError(f"malformed reply header ({e})") from None
    if size < 0:
        raise _ReplyError("negative payload size")
    return header, (_read_exact(fd, size, deadline) if size else b"")


class _Worker:
    def __init__(self) -> None:
        self.lock = threading.Lock()
        self.proc: subprocess.Popen | None = None
        self.log: Any = None

    def _start(self) -> subprocess.Popen:
        root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
        if self.log is not None:
            self.log.close()
        self.log = tempfile.TemporaryFile()
        return subprocess.Popen([sys.executable, "-m", "palladium_amd.compile_worker"], stdin=subprocess.PIPE,
                                stdout=subprocess.PIPE, stderr=self.log, env=env)

    def _log_tail(self) -> str:
        if self.log is None:
            return ""
        try:
            self.log.seek(0, os.SEEK_END)
            size = self.log.tell()
            self.log.seek(max(0, size - 16384))
            return "\n".join(self.log.read().decode(errors="replace").strip().splitlines()[-20:])
        except OSError:
            return ""

    def _discard(self, kill: bool) -> None:
        """Stop (if asked) and reap the child, close its pipes and log."""
        proc, self.proc = self.proc, None
        if proc is None:
            return
        if kill and proc.poll() is None:
            proc.kill()
        proc.wait()
        for f in (proc.stdin, proc.stdout):
            try:
                if f is not None:
                    f.close()
            except OSError:
                pass

    def compile(self, source: str, name: str, mode: int, arch: str) -> bytes:
        from palladium_amd.errors import CompileError

        timeout = compile_timeout()
        with self.lock:
            if self.proc is None or self.proc.poll() is not None:
                self._discard(kill=True)
                self.proc = self._start()
            proc = self.proc
            src = source.encode()
            try:
                _send(proc.stdin, {"name": name, "mode": int(mode), "arch": arch, "size": len(src)}, src)
                header, payload = _recv_by(proc.stdout.fileno(), time.monotonic() + timeout)
            except TimeoutError:
                self._discard(kill=True)
                raise CompileError(f"compiling {name!r} took longer than {timeout:g} s "
                                   "(PALLADIUM_COMPILE_TIMEOUT); the compiler process was stopped") from None
            except (BrokenPipeError, OSError, struct.error, _ReplyError) as e:
                self._discard(kill=True)
                tail = self._log_tail()
                raise CompileError(
                    f"the compiler process ended (exit {proc.returncode}) while compiling {name!r} "
                    f"({type(e).__name__}: {e}):\n{tail}"
                ) from None
            if not header.get("ok"):
                raise CompileError(str(header.get("error", "compile failed")))
            return payload


_worker = _Worker()


def compile_isolated(source: str, name: str, mode: int, arch: str = "gfx950") -> bytes:
    """Code object for `source`, compiled in the helper process."""
    return _worker.compile(source, name, mode, arch)


def _serve() -> None:
    # The protocol gets a private descriptor; fd 1 (and sys.stdout) now lead
    # to stderr, so nothing else the process prints can reach the parent's
    # reply stream.
    proto = os.fdopen(os.dup(1), "wb")
    os.dup2(2, 1)
    sys.stdout = sys.stderr

    from palladium_amd import runtime as rt

    stdin = sys.stdin.buffer
    while True:
        req = _recv(stdin)
        if req is None:
            return
        header, payload = req
        try:
            if os.environ.get("PALLADIUM_COMPILE_WORKER_TEST_NOISE"):
                # test hook: flood stderr and write to fd 1 before replying
                os.write(2, b"x" * int(os.environ["PALLADIUM_COMPILE_WORKER_TEST_NOISE"]))
                os.write(1, b"stray bytes on fd 1\n")
            code = rt.compile_code_object(payload.decode(), header["name"], int(header["mode"]), header["arch"])
            _send(proto, {"ok": True, "size": len(code)}, code)
        except Exception as e:  # noqa: BLE001 - every compile error goes back to the caller
            _send(proto, {"ok": False, "error": str(e)}, b"")


if __name__ == "__main__":
    _serve()
