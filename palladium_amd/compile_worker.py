"""Compiling in a helper process (opt-in: PALLADIUM_COMPILE_ISOLATED=1).

hiprtc runs the LLVM AMDGPU backend inside the calling process, so a
backend crash (an `LLVM ERROR` abort) ends that process. With isolation on,
`runtime.Kernel.load` sends the source to a long-lived child process, which
compiles it with `ph_compile_code_object` (hiprtc only: the child makes no
other HIP call), and loads the returned code object with
`ph_load_code_object`. If the child dies, or a compile outlasts
PALLADIUM_COMPILE_TIMEOUT seconds (default 900; the child is then
stopped), the parent raises `CompileError` and starts a fresh child on the
next compile.

Protocol over the child's stdin/stdout: a request is a 4-byte big-endian
length and a JSON header {"name", "mode", "arch", "size"} followed by `size`
bytes of source; a reply is a length-prefixed JSON header {"ok": true,
"size"} followed by the code object, or {"ok": false, "error"}.
"""

from __future__ import annotations

import json
import os
import select
import struct
import subprocess
import sys
import threading
from typing import Any

__all__ = ["compile_isolated", "isolation_enabled"]


def isolation_enabled() -> bool:
    return os.environ.get("PALLADIUM_COMPILE_ISOLATED", "") not in ("", "0")


def _send(stream: Any, header: dict, payload: bytes) -> None:
    h = json.dumps(header).encode()
    stream.write(struct.pack(">I", len(h)) + h + payload)
    stream.flush()


def _recv(stream: Any) -> tuple[dict, bytes] | None:
    raw = stream.read(4)
    if len(raw) < 4:
        return None
    (n,) = struct.unpack(">I", raw)
    header = json.loads(stream.read(n).decode())
    size = int(header.get("size", 0))
    payload = stream.read(size) if size else b""
    return header, payload


class _Worker:
    def __init__(self) -> None:
        self.lock = threading.Lock()
        self.proc: subprocess.Popen | None = None

    def _start(self) -> subprocess.Popen:
        root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
        return subprocess.Popen([sys.executable, "-m", "palladium_amd.compile_worker"], stdin=subprocess.PIPE,
                                stdout=subprocess.PIPE, stderr=subprocess.PIPE, env=env)

    def compile(self, source: str, name: str, mode: int, arch: str) -> bytes:
        from palladium_amd.errors import CompileError

        with self.lock:
            if self.proc is None or self.proc.poll() is not None:
                self.proc = self._start()
            proc = self.proc
            src = source.encode()
            timeout = float(os.environ.get("PALLADIUM_COMPILE_TIMEOUT", "900"))
            try:
                _send(proc.stdin, {"name": name, "mode": int(mode), "arch": arch, "size": len(src)}, src)
                ready, _, _ = select.select([proc.stdout], [], [], timeout)
                if not ready:
                    proc.kill()
                    proc.wait()
                    self.proc = None
                    raise CompileError(f"compiling {name!r} took longer than {timeout:g} s "
                                       "(PALLADIUM_COMPILE_TIMEOUT); the compiler process was stopped")
                reply = _recv(proc.stdout)
            except (BrokenPipeError, OSError):
                reply = None
            if reply is None:
                proc.wait()
                tail = proc.stderr.read().decode(errors="replace").strip().splitlines()[-20:]
                self.proc = None
                raise CompileError(
                    f"the compiler process ended (exit {proc.returncode}) while compiling {name!r}:\n" + "\n".join(tail)
                )
            header, payload = reply
            if not header.get("ok"):
                raise CompileError(header.get("error", "compile failed"))
            return payload


_worker = _Worker()


def compile_isolated(source: str, name: str, mode: int, arch: str = "gfx950") -> bytes:
    """Code object for `source`, compiled in the helper process."""
    return _worker.compile(source, name, mode, arch)


def _serve() -> None:
    from palladium_amd import runtime as rt

    stdin, stdout = sys.stdin.buffer, sys.stdout.buffer
    while True:
        req = _recv(stdin)
        if req is None:
            return
        header, payload = req
        try:
            code = rt.compile_code_object(payload.decode(), header["name"], int(header["mode"]), header["arch"])
            _send(stdout, {"ok": True, "size": len(code)}, code)
        except Exception as e:  # noqa: BLE001 - every compile error goes back to the caller
            _send(stdout, {"ok": False, "error": str(e)}, b"")


if __name__ == "__main__":
    _serve()
