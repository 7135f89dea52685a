"""The sampling worker's wire protocol (mlc_vla/worker.py; the reference's evaluation worker,
M1.md:55-72: a 4-byte length + pickle per message over the worker's stdin / stdout), on the
CPU: framing round trips and truncation, the unpickling allow-list, the request loop with a
stand-in engine, and a real worker process, whose engine setup fails without a GPU -- it
reports that as an error reply and keeps serving.  The GPU test (test_gpu_worker.py) samples
through a worker against the in-process runner."""

from __future__ import annotations

import io
import pickle
import struct

import numpy as np
import pytest

from conftest import TINY_KWARGS
from mlc_vla import worker as W


def _frames(*objs) -> io.BytesIO:
    return io.BytesIO(b"".join(W.encode(o) for o in objs))


def _replies(buf: io.BytesIO):
    buf.seek(0)
    out = []
    while True:
        body = W.read_frame(buf)
        if body is None:
            return out
        out.append(W.decode(body))


def test_frame_round_trip():
    rng = np.random.default_rng(0)
    msg = {"op": "sample", "prefix_embs": rng.standard_normal((1, 5, 8)).astype(np.float16),
           "noise": rng.standard_normal((1, 4, 3)).astype(np.float32), "prefix_pad": np.array([True, False, True]),
           "seed": 3, "graph": False, "num_steps": 7, "nested": [1, 2.5, "x", None, (np.float32(1.5),)]}
    f = W.encode(msg)
    assert struct.unpack(">I", f[:4])[0] == len(f) - 4  # big-endian length prefix
    got = W.decode(f[4:])
    assert set(got) == set(msg)
    for k in ("prefix_embs", "noise", "prefix_pad"):
        assert got[k].dtype == msg[k].dtype
        np.testing.assert_array_equal(got[k], msg[k])
    assert got["nested"][:4] == [1, 2.5, "x", None] and got["nested"][4][0] == np.float32(1.5)


def test_read_frame_boundaries():
    buf = _frames({"a": 1}, {"b": 2})
    assert W.decode(W.read_frame(buf)) == {"a": 1}
    assert W.decode(W.read_frame(buf)) == {"b": 2}
    assert W.read_frame(buf) is None  # clean end of stream
    whole = W.encode({"op": "ping"})
    for cut in (2, 6, len(whole) - 1):  # inside the header, inside the body
        with pytest.raises(W.FrameError, match="stream ended"):
            W.read_frame(io.BytesIO(whole[:cut]))
    with pytest.raises(W.FrameError, match="too large"):
        W.read_frame(io.BytesIO(struct.pack(">I", 0xFFFFFFFF)))


def test_unpickling_allow_list_refuses_other_globals():
    # protocol-0 pickle whose GLOBAL opcode names os.system: refused at the opcode, before any call
    with pytest.raises(W.FrameError, match="os.system"):
        W.decode(b"cos\nsystem\n(S'true'\ntR.")
    with pytest.raises(W.FrameError, match="builtins.print"):
        W.decode(pickle.dumps(print))
    import collections
    with pytest.raises(W.FrameError, match="OrderedDict"):
        W.decode(pickle.dumps(collections.OrderedDict(a=1)))
    with pytest.raises(W.FrameError, match="undecodable"):
        W.decode(b"\x80\x04garbage")


class _Echo:
    """Stand-in engine for the request loop: 'actions' are the noise plus the seed."""

    def sample(self, req):
        return np.asarray(req["noise"], np.float32) + req.get("seed", 0)


def test_serve_request_loop():
    noise = np.arange(6, dtype=np.float32).reshape(1, 2, 3)
    inp = _frames({"op": "ping"}, {"op": "sample", "prefix_embs": np.zeros((1, 2, 2)), "noise": noise, "seed": 2},
                  {"op": "nope"}, "not a dict", {"op": "shutdown"}, {"op": "ping"})
    out = io.BytesIO()
    assert W.serve(inp, out, _Echo(), None, {"k": 1}) == 0
    r = _replies(out)
    assert len(r) == 5  # the ping after shutdown is not answered
    assert r[0]["ok"] and r[0]["ready"] and r[0]["config"] == {"k": 1}
    assert r[1]["ok"] and r[1]["actions"].dtype == np.float32
    np.testing.assert_array_equal(r[1]["actions"], noise + 2)
    assert not r[2]["ok"] and "unknown op" in r[2]["error"]
    assert not r[3]["ok"] and "dict with an 'op'" in r[3]["error"]
    assert r[4] == {"ok": True}


def test_serve_without_engine_reports_errors():
    inp = _frames({"op": "ping"}, {"op": "sample", "prefix_embs": np.zeros((1, 2, 2))})
    out = io.BytesIO()
    assert W.serve(inp, out, None, "RuntimeError: no GPU", {}) == 0  # end of stream
    r = _replies(out)
    assert r[0]["ok"] and not r[0]["ready"] and "no GPU" in r[0]["error"]
    assert not r[1]["ok"] and "not set up" in r[1]["error"]
    # a refused message is answered with an error and the loop goes on
    out = io.BytesIO()
    bad = pickle.dumps(print)
    assert W.serve(io.BytesIO(struct.pack(">I", len(bad)) + bad + W.encode({"op": "ping"})), out, None, None, {}) == 0
    r = _replies(out)
    assert not r[0]["ok"] and "may not name" in r[0]["error"]
    assert r[1]["ok"]


def test_worker_process_without_gpu(tmp_path):
    """A real worker process on this CPU-only machine: the engine cannot be set up (the HIP
    library finds no GPU), which ping reports; sample is refused; shutdown ends it with 0.
    Its stdout carries frames only (a stray print would break the next read)."""
    c = W.WorkerClient(TINY_KWARGS, str(tmp_path / "cfg.json"), random_weights=1)
    try:
        p = c.ping()
        assert p["config"]["action_horizon"] == TINY_KWARGS["action_horizon"]
        if p["ready"]:
            pytest.skip("a GPU is visible here; the GPU test covers this case")
        assert p["error"]
        with pytest.raises(W.WorkerError, match="not set up"):
            c.sample(np.zeros((1, 4, 4), np.float16))
        assert c.ping()["ok"]
    finally:
        rc = c.close()
    assert rc == 0
