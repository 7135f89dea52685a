"""Out-of-process sampling worker and its client.

The evaluation harness of the reference runs the engine in a separate worker process: the
client spawns the worker, which holds the engine and the weights and answers ``sample``
requests; every message is a 4-byte length followed by a pickle, over the worker's stdin and
stdout (M1.md:55-72).  The harness's own message schema is not part of the reference, so the
one here is this module's:

Framing: a 4-byte unsigned big-endian length ``n``, then ``n`` bytes of pickle (protocol 4).

Requests are dicts with an ``"op"``:

- ``{"op": "ping"}`` -> ``{"ok": True, "ready": bool, "pid": int, "config": {...}}``;
  ``ready`` is False (with ``"error"``) when the engine could not be set up.
- ``{"op": "sample", "prefix_embs": [1, P, W], "noise": [1, H, A] or None, "seed": int,
  "prefix_pad": bool [P] or None, "graph": bool, "num_steps": int}`` ->
  ``{"ok": True, "actions": float32 [1, H, A], "ms": float}``.  ``graph`` (default True)
  runs the device loop (``PiZeroRunner.sample_graph``, ``num_denoise_steps`` steps);
  otherwise the host loop (``PiZeroRunner.sample``) of ``num_steps`` steps.
- ``{"op": "shutdown"}`` -> ``{"ok": True}``, then the worker exits with status 0.

A failed request is answered with ``{"ok": False, "error": "..."}`` and the worker keeps
serving.  Messages are unpickled with an allow-list: plain containers, numbers, strings and
numpy arrays / dtypes / scalars.  A message naming any other global is refused with an error
reply, so a peer cannot make the worker run code.  The worker writes only frames to its
stdout: its own output and that of the native library go to stderr.

Run as ``python -m mlc_vla.worker --config CONFIG.json (--checkpoint MODEL.safetensors |
--random-weights SEED)``; ``WorkerClient`` spawns and drives it.
"""

from __future__ import annotations

import argparse
import io
import json
import os
import pickle
import struct
import subprocess
import sys
import time
from typing import Any, BinaryIO, Dict, Optional

import numpy as np

_LEN = struct.Struct(">I")
MAX_FRAME = 1 << 31  # bytes of one message at most

# (module, name) pairs a message may name: what numpy arrays, dtypes and scalars pickle to
_ALLOWED = {
    ("numpy.core.multiarray", "_reconstruct"),
    ("numpy._core.multiarray", "_reconstruct"),
    ("numpy.core.multiarray", "scalar"),
    ("numpy._core.multiarray", "scalar"),
    ("numpy", "ndarray"),
    ("numpy", "dtype"),
    ("numpy.core.numeric", "_frombuffer"),
    ("numpy._core.numeric", "_frombuffer"),
}


class FrameError(RuntimeError):
    """A malformed, truncated or refused message."""


class WorkerError(RuntimeError):
    """The worker answered a request with an error."""


class _RestrictedUnpickler(pickle.Unpickler):
    def find_class(self, module: str, name: str):
        if (module, name) in _ALLOWED:
            return super().find_class(module, name)
        raise FrameError(f"message refers to {module}.{name}, which a message may not name")


def encode(obj: Any) -> bytes:
    """One frame: length prefix + pickle."""
    body = pickle.dumps(obj, protocol=4)
    if len(body) >= MAX_FRAME:
        raise FrameError(f"message of {len(body)} bytes is too large")
    return _LEN.pack(len(body)) + body


def decode(body: bytes) -> Any:
    """The object of one frame body, through the allow-list."""
    try:
        return _RestrictedUnpickler(io.BytesIO(body)).load()
    except FrameError:
        raise
    except Exception as e:  # a corrupt pickle
        raise FrameError(f"undecodable message: {e}") from e


def _read_exact(f: BinaryIO, n: int) -> Optional[bytes]:
    buf = bytearray()
    while len(buf) < n:
        chunk = f.read(n - len(buf))
        if not chunk:
            return None
        buf += chunk
    return bytes(buf)


def read_frame(f: BinaryIO) -> Optional[bytes]:
    """The body of the next frame; None at a clean end of stream (no partial header)."""
    head = f.read(_LEN.size)
    if not head:
        return None
    if len(head) < _LEN.size:
        rest = _read_exact(f, _LEN.size - len(head))
        if rest is None:
            raise FrameError("stream ended inside a frame header")
        head += rest
    (n,) = _LEN.unpack(head)
    if n >= MAX_FRAME:
        raise FrameError(f"frame length {n} is too large")
    body = _read_exact(f, n)
    if body is None:
        raise FrameError(f"stream ended inside a frame of {n} bytes")
    return body


def write_frame(f: BinaryIO, obj: Any) -> None:
    f.write(encode(obj))
    f.flush()


# ---------------------------------------------------------------------------------------
# worker side


def random_params(named_params, seed: int):
    """Synthetic weights: N(0, 0.02) in ``named_params`` order and dtypes (numpy's
    default_rng(seed)); integer parameters are zero."""
    rng = np.random.default_rng(seed)
    out = []
    for _, p in named_params:
        shape = tuple(int(s) for s in p.shape)
        dt = np.dtype(p.dtype)
        if np.issubdtype(dt, np.integer):
            out.append(np.zeros(shape, dt))
        else:
            out.append((0.02 * rng.standard_normal(shape, dtype=np.float32)).astype(dt))
    return out


class _Engine:
    """The runner and its bound weights."""

    def __init__(self, config_kwargs: Dict[str, Any], checkpoint: Optional[str], random_seed: Optional[int],
                 cuda_graph: bool):
        from .model.pi0 import Pi0Config
        from .sample import PiZeroRunner

        cfg = Pi0Config(**config_kwargs)
        self.runner = PiZeroRunner(cfg, "rocm", cuda_graph=cuda_graph)
        names = self.runner.named_params
        if checkpoint is not None:
            from .model.pi0.pi0_loader import load_params, load_safetensors

            built = load_params(cfg, load_safetensors(checkpoint), named_params=names)
            arrays = [built[n] for n, _ in names]
        else:
            arrays = random_params(names, int(random_seed or 0))
        self.params = self.runner.to_params(arrays)

    def sample(self, req: Dict[str, Any]) -> np.ndarray:
        prefix = np.asarray(req["prefix_embs"])
        noise = req.get("noise")
        pad = req.get("prefix_pad")
        seed = int(req.get("seed", 0))
        if req.get("graph", True):
            return self.runner.sample_graph(self.params, prefix, noise=noise, seed=seed, prefix_pad=pad)
        return self.runner.sample(self.params, prefix, noise=noise, num_steps=int(req.get("num_steps", 10)),
                                  seed=seed, prefix_pad=pad)


def serve(inp: BinaryIO, out: BinaryIO, engine: Optional[_Engine], setup_error: Optional[str],
          config_kwargs: Dict[str, Any]) -> int:
    """Answer requests until shutdown (0) or the end of the input stream (0)."""
    while True:
        try:
            body = read_frame(inp)
        except FrameError as e:
            print(f"worker: {e}; stopping", file=sys.stderr, flush=True)
            return 1
        if body is None:
            return 0
        try:
            req = decode(body)
            if not isinstance(req, dict) or "op" not in req:
                raise FrameError("a request is a dict with an 'op'")
            op = req["op"]
            if op == "ping":
                rep = {"ok": True, "ready": engine is not None, "pid": os.getpid(), "config": config_kwargs}
                if setup_error:
                    rep["error"] = setup_error
            elif op == "sample":
                if engine is None:
                    raise RuntimeError(f"the engine is not set up: {setup_error}")
                t0 = time.perf_counter()
                actions = np.asarray(engine.sample(req), dtype=np.float32)
                rep = {"ok": True, "actions": actions, "ms": (time.perf_counter() - t0) * 1e3}
            elif op == "shutdown":
                write_frame(out, {"ok": True})
                return 0
            else:
                raise FrameError(f"unknown op {op!r}")
        except Exception as e:  # answered, and the worker keeps serving
            rep = {"ok": False, "error": f"{type(e).__name__}: {e}"}
        write_frame(out, rep)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m mlc_vla.worker", description=__doc__.split("\n\n")[0])
    ap.add_argument("--config", required=True, help="JSON file of Pi0Config keyword arguments")
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--checkpoint", help="PI0Pytorch safetensors file")
    src.add_argument("--random-weights", type=int, metavar="SEED", help="N(0, 0.02) synthetic weights")
    ap.add_argument("--cuda-graph", action="store_true")
    args = ap.parse_args(argv)
    # frames own the real stdout; everything else printed (Python or native) goes to stderr
    out = os.fdopen(os.dup(1), "wb", buffering=0)
    os.dup2(2, 1)
    sys.stdout = sys.stderr
    inp = os.fdopen(os.dup(0), "rb", buffering=0)
    with open(args.config) as f:
        config_kwargs = json.load(f)
    for k in ("image_keys",):
        if isinstance(config_kwargs.get(k), list):
            config_kwargs[k] = tuple(config_kwargs[k])
    engine, err = None, None
    try:
        engine = _Engine(config_kwargs, args.checkpoint, args.random_weights, args.cuda_graph)
    except Exception as e:  # reported to the client by ping / sample
        err = f"{type(e).__name__}: {e}"
        print(f"worker: engine setup failed: {err}", file=sys.stderr, flush=True)
    return serve(inp, out, engine, err, config_kwargs)


# ---------------------------------------------------------------------------------------
# client side


class WorkerClient:
    """Spawns ``python -m mlc_vla.worker`` and sends it requests (one at a time)."""

    def __init__(self, config_kwargs: Dict[str, Any], config_path: str, checkpoint: Optional[str] = None,
                 random_weights: Optional[int] = None, cuda_graph: bool = False, python: str = sys.executable,
                 env: Optional[Dict[str, str]] = None):
        if (checkpoint is None) == (random_weights is None):
            raise ValueError("give exactly one of checkpoint and random_weights")
        cfg = dict(config_kwargs)
        for k, v in cfg.items():
            if isinstance(v, tuple):
                cfg[k] = list(v)
        with open(config_path, "w") as f:
            json.dump(cfg, f)
        cmd = [python, "-m", "mlc_vla.worker", "--config", config_path]
        cmd += ["--checkpoint", checkpoint] if checkpoint is not None else ["--random-weights", str(random_weights)]
        if cuda_graph:
            cmd.append("--cuda-graph")
        e = dict(os.environ if env is None else env)
        pkg_root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        e["PYTHONPATH"] = pkg_root + (os.pathsep + e["PYTHONPATH"] if e.get("PYTHONPATH") else "")
        self.proc = subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE, env=e)

    def request(self, msg: Dict[str, Any]) -> Dict[str, Any]:
        write_frame(self.proc.stdin, msg)
        body = read_frame(self.proc.stdout)
        if body is None:
            raise WorkerError(f"the worker exited (status {self.proc.poll()})")
        rep = decode(body)
        if not rep.get("ok", False):
            raise WorkerError(rep.get("error", "request failed"))
        return rep

    def ping(self) -> Dict[str, Any]:
        return self.request({"op": "ping"})

    def sample(self, prefix_embs: np.ndarray, noise: Optional[np.ndarray] = None, seed: int = 0,
               prefix_pad: Optional[np.ndarray] = None, graph: bool = True, num_steps: int = 10) -> np.ndarray:
        return self.request({"op": "sample", "prefix_embs": np.asarray(prefix_embs), "noise": noise, "seed": seed,
                             "prefix_pad": prefix_pad, "graph": graph, "num_steps": num_steps})["actions"]

    def close(self, timeout: float = 60.0) -> int:
        """Ask the worker to stop and wait for it; kill it if it does not stop in time."""
        if self.proc.poll() is None:
            try:
                self.request({"op": "shutdown"})
            except (WorkerError, FrameError, OSError):
                pass
            try:
                self.proc.wait(timeout=timeout)
            except subprocess.TimeoutExpired:
                self.proc.kill()
                self.proc.wait()
        for f in (self.proc.stdin, self.proc.stdout):
            if f:
                f.close()
        return self.proc.returncode

    def __enter__(self) -> "WorkerClient":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


if __name__ == "__main__":
    sys.exit(main())
