"""Device tensors and the VM-style entry points of the M1 functions.

Mirrors the reference's runtime boundary: ``tvm.runtime.tensor(np, dev)`` builds
device tensors and ``relax.VirtualMachine(ex, dev)["<fn>"](*tensors, params)``
runs an exported function (python/mlc_vla/sample.py:95-105,128,158-160,184-186).
Here device memory and the current stream come from PyTorch-ROCm; every function
body is one call into ``libmlcvla_hip.so``.

Behaviour kept from the reference boundary:
  - arguments are checked against the exported signature (shape and dtype must
    match exactly, like Relax struct-info matching) before anything runs;
  - ``params`` is the last argument, a list in ``named_params`` order;
  - outputs are freshly allocated device tensors; ``prefill`` returns a 2-tuple.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _native as N
from .model.pi0.pi0_model import BACKBONE_FUNCS, get_default_spec

_TORCH = {"float16": torch.float16, "float32": torch.float32, "int32": torch.int32, "uint32": torch.int32}


class Device:
    """A HIP device (``tvm.device("rocm", i)``)."""

    def __init__(self, kind: str = "rocm", index: int = 0):
        self.kind = kind
        self.index = index

    @property
    def torch(self) -> torch.device:
        return torch.device("cuda", self.index)

    def sync(self) -> None:
        torch.cuda.synchronize(self.index)

    def __repr__(self) -> str:
        return f"{self.kind}({self.index})"


def device(kind: str = "rocm", index: int = 0) -> Device:
    if not torch.cuda.is_available():
        raise N.MlcvError("no HIP device visible: the gfx950 kernels are the only compute path")
    return Device(kind, index)


class Tensor:
    """Device tensor with a logical dtype string (uint32 is stored as int32 bits).  An output
    of a VM function carries its VM's ``check``: reading it on the host also reports a
    persistent step of that VM that ended early (``mlcv_sync``)."""

    __slots__ = ("torch", "dtype", "_check")

    def __init__(self, t: torch.Tensor, dtype: str, check=None):
        self.torch = t
        self.dtype = dtype
        self._check = check

    @property
    def shape(self):
        return tuple(self.torch.shape)

    def numpy(self) -> np.ndarray:
        if self._check is not None:
            self._check()
        a = self.torch.detach().cpu().numpy()
        return a.view(np.uint32) if self.dtype == "uint32" else a

    def data_ptr(self) -> int:
        return self.torch.data_ptr()

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape}, dtype={self.dtype})"


def tensor(arr, dev: Optional[Device] = None) -> Tensor:
    """Copy a numpy array to the device (``tvm.runtime.tensor``)."""
    dev = dev or device()
    a = np.ascontiguousarray(arr)
    dt = str(a.dtype)
    if dt not in _TORCH:
        raise TypeError(f"unsupported dtype {dt}")
    if dt == "uint32":
        a = a.view(np.int32)
    return Tensor(torch.from_numpy(a).to(dev.torch), dt)


def empty(shape, dtype: str, dev: Optional[Device] = None, check=None) -> Tensor:
    dev = dev or device()
    return Tensor(torch.empty(tuple(shape), dtype=_TORCH[dtype], device=dev.torch), dtype, check)


def as_tensor(x) -> Tensor:
    if isinstance(x, Tensor):
        return x
    if isinstance(x, torch.Tensor):
        inv = {torch.float16: "float16", torch.float32: "float32", torch.int32: "int32"}
        if x.dtype not in inv:
            raise TypeError(f"unsupported tensor dtype {x.dtype}")
        return Tensor(x, inv[x.dtype])
    raise TypeError(f"expected a device tensor, got {type(x).__name__}")


def _ptr(t: Tensor) -> ctypes.c_void_p:
    if not t.torch.is_cuda:
        raise ValueError("tensor is not on the HIP device")
    if not t.torch.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.torch.data_ptr())


def _check(name: str, arg: str, t: Tensor, shape, dtype) -> None:
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype:
        raise ValueError(f"{name}: argument {arg} expects {tuple(shape)} {dtype}, got {t.shape} {t.dtype}")


class Executable:
    """What ``compile_model`` returns: the configuration the kernels are planned for."""

    def __init__(self, config, functions: Sequence[str], named_params, quant: Optional[str] = None,
                 cuda_graph: bool = False, hoist_modulation: bool = True):
        self.config = config
        self.functions = tuple(functions)
        self.named_params = list(named_params)
        self.quant = quant
        self.cuda_graph = cuda_graph
        self.hoist_modulation = hoist_modulation

    def c_config(self) -> N.Config:
        c = self.config
        vlm, ae = c.vlm, c.action_expert
        return N.Config(
            vlm_width=vlm.width, vlm_mlp=vlm.mlp_dim, ae_width=ae.width, ae_mlp=ae.mlp_dim,
            depth=vlm.depth, num_heads=vlm.num_heads, num_kv_heads=vlm.num_kv_heads, head_dim=vlm.head_dim,
            prefix_len=c.prefix_len, suffix_len=c.suffix_len, action_dim=c.action_dim,
            num_steps=c.num_denoise_steps, rms_norm_eps=c.rms_norm_eps, rope_theta=c.rope_theta,
            dtype=N.MLCV_DTYPE_F32 if c.dtype == "float32" else N.MLCV_DTYPE_F16,
            quant=N.MLCV_QUANT_Q4F16_1 if self.quant == "q4f16_1" else N.MLCV_QUANT_NONE,
        )


class VirtualMachine:
    """``vm["embed_language" | "denoise_step" | "prefill" | "denoise_step_kv" | "denoise_loop_kv" |
    "chunk"](*tensors, params)``.  The backbone functions share one native context (created
    when any of them is compiled); ``embed_language`` is a stateless kernel over the
    ``embed_tokens`` table, the first parameter when it is compiled."""

    def __init__(self, ex: Executable, dev: Optional[Device] = None):
        self.ex = ex
        self.dev = dev or device()
        self._spec = get_default_spec(ex.config)
        names = [n for n, _ in ex.named_params]
        self._nvis = sum(1 for n in names if n.startswith("vision."))
        self._emb = "embed_tokens.weight" in names
        self._bb0 = self._nvis + (1 if self._emb else 0)  # first backbone parameter
        self._backbone = any(f in BACKBONE_FUNCS for f in ex.functions)
        self._vis_ws = None
        self._vis_key = None  # (ids of the last parameter list, its tensors, their pointer array)
        self._ctx = ctypes.c_void_p()
        self._bound = None
        if self._backbone:
            cfg = ex.c_config()
            h = ctypes.c_void_p()
            with torch.cuda.device(self.dev.index):
                N.call("mlcv_create", ctypes.byref(cfg), ctypes.byref(h))
            self._ctx = h
            self.set_graph(ex.cuda_graph)
            self.set_hoist(ex.hoist_modulation)

    def __del__(self):
        h = getattr(self, "_ctx", None)
        if h is not None and h.value:
            try:
                N.load().mlcv_destroy(h)
            except Exception:  # noqa: BLE001 -- interpreter shutdown
                pass
            self._ctx = None

    # options ---------------------------------------------------------------
    def set_graph(self, on: bool) -> None:
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_USE_GRAPH, int(bool(on)))

    def set_step_graph(self, on: bool) -> None:
        """denoise_step_kv as a captured hipGraph replay (off by default: direct launches, whose
        step ends sooner than a graph replay's; the loop and the chunk keep their graphs)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_STEP_GRAPH, int(bool(on)))

    def set_hoist(self, on: bool) -> None:
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_HOIST_MODULATION, int(bool(on)))

    def set_persist(self, on: bool) -> None:
        """Run each step as one persistent kernel (off by default; only for shapes it is built for)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_PERSIST, int(bool(on)))

    def set_xtp(self, on: bool) -> None:
        """Run the decoder layers tensor-parallel over the GPU's XCDs (on by default where the
        shape and the device allow it; an error elsewhere)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_XTP, int(bool(on)))

    def set_xtp_keep(self, on: bool) -> None:
        """Keep every layer's intermediates of the XCD step for probes (testing; slower)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_XTP_KEEP, int(bool(on)))

    def set_step_form(self, form: str) -> None:
        """The execution of denoise_step_kv: "chain" (one launch per operation), "persistent"
        (one launch per step) or "xtp" (two launches per layer over the XCDs)."""
        if form not in ("chain", "persistent", "xtp"):
            raise ValueError(f"unknown step form {form!r}")
        if form == "xtp":
            self.set_xtp(True)
        else:
            self.set_xtp(False)
            self.set_persist(form == "persistent")

    def set_sync_words(self, value: int) -> None:
        """Set the persistent step's progress words and the XCD step's barrier words (testing:
        a value just below 2**32 makes the next launches wrap them)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_SYNC_WORDS, int(value) & 0xFFFFFFFF)

    def set_mask_skip(self, on: bool) -> None:
        """Skip key chunks whose mask is entirely <= -1e9 in every attention (default; the
        results are bit-identical), or compute them (testing)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_MASK_SKIP, int(bool(on)))

    def set_persist_spin(self, polls: int) -> None:
        """Polls before a wait of the persistent or XCD step gives up."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_PERSIST_SPIN, int(polls))

    def set_meet_polls(self, polls: int) -> None:
        """Polls of a prefill split-K meeting before it gives up (the call's outputs are then
        invalid and reading them raises)."""
        N.call("mlcv_set_option", self._ctx, N.MLCV_OPT_MEET_POLLS, int(polls))

    def check(self) -> None:
        """Synchronize and raise if a bounded device-side wait of this VM gave up."""
        if self._ctx:
            N.call("mlcv_sync", self._ctx, self._stream())

    # the op codes of mlcv_bench_op (include/mlcvla.h)
    STEP_OPS = {"time_mod": 0, "modulation": 1, "qkv": 2, "attention": 3, "o_proj": 4, "gate_up": 5, "down": 6,
                "head": 7, "attention_only": 8, "action_in": 9}

    def run_op(self, op: str, layer: int = 0, keys=None, values=None) -> None:
        """Enqueue one operation of denoise_step_kv on this VM's current buffers (testing):
        the launch chain's kernels with the arguments the step gives them."""
        kp = _ptr(keys) if keys is not None else None
        vp = _ptr(values) if values is not None else None
        N.call("mlcv_bench_op", self._ctx, self.STEP_OPS[op], int(layer), 1, kp, vp, self._stream())

    def probe(self, what: str, layer: int, shape, dtype) -> np.ndarray:
        """An intermediate of the last step (testing): see mlcv_step_probe."""
        out = np.empty(shape, dtype)
        N.call("mlcv_step_probe", self._ctx, N.PROBES[what], int(layer), out.ctypes.data_as(ctypes.c_void_p),
               out.nbytes, self._stream())
        return out

    # plumbing --------------------------------------------------------------
    def _stream(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream(self.dev.index).cuda_stream)

    def _check_params(self, params: Sequence) -> List[Tensor]:
        specs = self.ex.named_params
        if len(params) != len(specs):
            raise ValueError(f"expected {len(specs)} params, got {len(params)}")
        ts: List[Tensor] = [as_tensor(p) for p in params]
        for (name, sp), t in zip(specs, ts):
            want = "int32" if sp.dtype == "uint32" and t.dtype == "int32" else sp.dtype
            _check("params", name, t, sp.shape, want)
        return ts

    def _bind(self, params: Sequence) -> None:
        if not self._backbone:
            raise KeyError("no backbone function is compiled in this executable")
        ts = self._check_params(params)[self._bb0:]
        key = tuple(t.torch.data_ptr() for t in ts)
        if key == self._bound:
            return
        arr = (ctypes.c_void_p * len(ts))(*[ctypes.c_void_p(k) for k in key])
        self._bound = None  # a failing bind leaves the context unbound
        N.call("mlcv_bind_params", self._ctx, arr, len(ts), self._stream())
        self._bound = key
        self._keep = ts  # the caller owns them; kept alive while bound

    def _args(self, fn: str, tensors) -> List[Tensor]:
        spec = self._spec[fn]
        if len(tensors) != len(spec):
            raise ValueError(f"{fn}: expected {len(spec)} tensors, got {len(tensors)}")
        out = []
        for (arg, sp), x in zip(spec.items(), tensors):
            t = as_tensor(x)
            _check(fn, arg, t, sp.shape, sp.dtype)
            out.append(t)
        return out

    def __getitem__(self, name: str):
        fns = {}
        if "embed_image" in self.ex.functions:
            fns["embed_image"] = self.embed_image
        if "embed_language" in self.ex.functions:
            fns["embed_language"] = self.embed_language
        if self._backbone:
            fns.update({"denoise_step": self.denoise_step, "prefill": self.prefill,
                        "denoise_step_kv": self.denoise_step_kv, "denoise_loop_kv": self.denoise_loop_kv,
                        "chunk": self.chunk})
        if name not in fns:
            raise KeyError(f"function {name!r} is not built (available: {sorted(fns)})")
        return fns[name]

    # exported functions ------------------------------------------------------
    def embed_language(self, input_ids, params):
        """[1, max_token_len] int32 -> [1, max_token_len, vlm_width]: the embed_tokens rows
        times sqrt(width) in the model dtype (pi0_model.py:101-104)."""
        table = self._check_params(params)[self._nvis]
        (ids,) = self._args("embed_language", (input_ids,))
        vocab, width = table.shape
        out = empty((1, ids.shape[1], width), self.ex.config.dtype, self.dev)
        N.call("mlcv_embed_language", _ptr(ids), ids.shape[1], _ptr(table), vocab, width, _ptr(out), self._stream())
        return out

    def embed_image(self, image, params):
        """[1, S, S, C] channels-last -> [1, num_patches, projection_dim]: the SigLIP tower and
        the PaliGemma projector (pi0_model.py:97-99, siglip.py:73-120)."""
        key = tuple(id(p) for p in params)
        if self._vis_key is None or self._vis_key[0] != key:  # validate once per parameter list
            vis = self._check_params(params)[: self._nvis]
            arr = (ctypes.c_void_p * len(vis))(*[ctypes.c_void_p(t.torch.data_ptr()) for t in vis])
            self._vis_key = (key, vis, arr)
        _, vis, arr = self._vis_key
        (img,) = self._args("embed_image", (image,))
        s = self.ex.config.siglip
        cfg = N.VisionConfig(image_size=s.image_size, patch_size=s.patch_size, num_channels=s.num_channels,
                             hidden_size=s.hidden_size, intermediate_size=s.intermediate_size,
                             num_hidden_layers=s.num_hidden_layers, num_attention_heads=s.num_attention_heads,
                             projection_dim=s.projection_dim, layer_norm_eps=s.layer_norm_eps)
        if self._vis_ws is None:
            nbytes = ctypes.c_size_t()
            N.call("mlcv_embed_image_workspace", ctypes.byref(cfg), ctypes.byref(nbytes))
            self._vis_ws = torch.empty(nbytes.value, dtype=torch.uint8, device=self.dev.torch)
        out = empty((1, s.num_patches, s.projection_dim), self.ex.config.dtype, self.dev)
        N.call("mlcv_embed_image", ctypes.byref(cfg), arr, len(vis), _ptr(img), _ptr(out),
               ctypes.c_void_p(self._vis_ws.data_ptr()), self._vis_ws.numel(), self._stream())
        return out

    def denoise_step(self, prefix_embs, x_t, time_emb, params):
        """The joint prefix + suffix velocity (Pi0Model.denoise_step, pi0_model.py:111-125):
        every prefix token valid, RoPE positions 0..P+T-1; returns v [1,T,A] f32."""
        self._bind(params)
        a = self._args("denoise_step", (prefix_embs, x_t, time_emb))
        v = empty(a[1].shape, "float32", self.dev, self.check)
        N.call("mlcv_denoise_step", self._ctx, *[_ptr(t) for t in a], _ptr(v), self._stream())
        return v

    def prefill(self, prefix_embs, prefix_mask, params):
        self._bind(params)
        pe, pm = self._args("prefill", (prefix_embs, prefix_mask))
        kvs = self._spec["denoise_step_kv"]["keys"].shape
        keys = empty(kvs, "float32", self.dev, self.check)
        values = empty(kvs, self.ex.config.dtype, self.dev, self.check)
        N.call("mlcv_prefill", self._ctx, _ptr(pe), _ptr(pm), _ptr(keys), _ptr(values), self._stream())
        return keys, values

    def denoise_step_kv(self, keys, values, x_t, time_emb, suffix_cos, suffix_sin, prefix_mask, params):
        self._bind(params)
        a = self._args("denoise_step_kv", (keys, values, x_t, time_emb, suffix_cos, suffix_sin, prefix_mask))
        v = empty(a[2].shape, "float32", self.dev, self.check)
        N.call("mlcv_denoise_step_kv", self._ctx, *[_ptr(t) for t in a], _ptr(v), self._stream())
        return v

    def denoise_loop_kv(self, keys, values, x0, time_embs, suffix_cos, suffix_sin, prefix_mask, params):
        self._bind(params)
        a = self._args("denoise_loop_kv", (keys, values, x0, time_embs, suffix_cos, suffix_sin, prefix_mask))
        x = empty(a[2].shape, "float32", self.dev, self.check)
        N.call("mlcv_denoise_loop_kv", self._ctx, *[_ptr(t) for t in a], _ptr(x), self._stream())
        return x

    def chunk(self, prefix_embs, prefix_mask, x0, time_embs, suffix_cos, suffix_sin, params):
        """prefill + denoise_loop_kv as one graph; returns the final actions [1,T,A] f32."""
        self._bind(params)
        pe, pm = self._args("prefill", (prefix_embs, prefix_mask))
        lk = self._spec["denoise_loop_kv"]
        x0t, te, c, s = (as_tensor(t) for t in (x0, time_embs, suffix_cos, suffix_sin))
        for arg, t in (("x0", x0t), ("time_embs", te), ("suffix_cos", c), ("suffix_sin", s)):
            _check("chunk", arg, t, lk[arg].shape, lk[arg].dtype)
        x = empty(x0t.shape, "float32", self.dev, self.check)
        N.call("mlcv_chunk", self._ctx, _ptr(pe), _ptr(pm), _ptr(x0t), _ptr(te), _ptr(c), _ptr(s), _ptr(x),
               self._stream())
        return x
