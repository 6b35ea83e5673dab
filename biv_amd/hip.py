"""Host side of the gfx950 MoE backend, over the C ABI of include/biv_hip.h.

This mirrors the interface biv's MoE path sits behind: a backend context
(Engine construction, engine/src/engine.rs:15-60), weights uploaded once
(Weight / Experts, engine/src/ops.rs:12-43, model.rs:190-217), a MoE layer
(struct Moe, model.rs:229-237) and `ffn(h, n)` (Model::ffn, model.rs:853-898)
returning the block's output for n tokens.  Errors come back as HipError with
the library's message, as biv's backends return Error::Backend(String)
(engine/src/error.rs:67-68).

The library is required: there is no CPU fallback.  If libbiv_hip.so is not
built, loading raises.
"""
import ctypes
import os

import numpy as np

from . import synth

HERE = os.path.dirname(os.path.abspath(__file__))
# BIV_HIP_LIB names another build of the library (a tuning variant from
# python -m biv_amd.build -D... -o PATH)
LIB_PATH = os.environ.get("BIV_HIP_LIB") or os.path.join(HERE, "libbiv_hip.so")

ADD = 1

# every symbol include/biv_hip.h declares
SYMBOLS = [
    "biv_hip_create", "biv_hip_destroy", "biv_hip_last_error", "biv_hip_set_stream", "biv_hip_sync",
    "biv_hip_upload_weight", "biv_hip_upload_experts", "biv_hip_moe_create", "biv_hip_moe_forward",
    "biv_hip_moe_forward_device", "biv_hip_moe_forward_device_noalloc", "biv_hip_moe_forward_taps", "biv_hip_malloc", "biv_hip_free",
    "biv_hip_memcpy_h2d", "biv_hip_memcpy_d2h", "biv_hip_numerics", "biv_hip_device_bytes",
    "biv_hip_set_timing", "biv_hip_stage_times", "biv_hip_time_stage", "biv_hip_rms_norm",
    "biv_hip_moe_ffn_step", "biv_hip_moe_from_gguf", "biv_hip_dense_create", "biv_hip_dense_forward",
    "biv_hip_dense_forward_device", "biv_hip_dense_from_gguf", "biv_gguf_read_dense_config",
    "biv_gguf_open", "biv_gguf_close", "biv_gguf_last_error", "biv_gguf_get_u64", "biv_gguf_get_f32",
    "biv_gguf_get_str", "biv_gguf_n_tensors", "biv_gguf_tensor_name", "biv_gguf_tensor", "biv_gguf_read_moe_config",
]

STAGES = ["router", "route_sort", "gate_up", "quant_act", "down", "combine"]


class HipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"biv_hip error {code}: {msg}")
        self.code = code


class Taps(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "ids", "weights", "logits", "shared_logit", "pair_token", "pair_expert", "gate_idots", "up_idots",
        "act_q", "act_d", "down_idots")]


_lib = None


def load():
    """The loaded libbiv_hip.so; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipError(-3, f"{LIB_PATH} is not built (python -m biv_amd.build)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    pp = ctypes.POINTER(ctypes.c_void_p)
    L.biv_hip_create.argtypes = [i, pp]
    L.biv_hip_destroy.argtypes = [vp]
    L.biv_hip_destroy.restype = None
    L.biv_hip_last_error.argtypes = [vp]
    L.biv_hip_last_error.restype = ctypes.c_char_p
    L.biv_hip_set_stream.argtypes = [vp, vp]
    L.biv_hip_sync.argtypes = [vp]
    L.biv_hip_upload_weight.argtypes = [vp, i, sz, sz, vp, pp]
    L.biv_hip_upload_experts.argtypes = [vp, i, sz, sz, sz, vp, sz, sz, pp]
    L.biv_hip_moe_create.argtypes = [vp] + [vp] * 8 + [i, pp]
    L.biv_hip_moe_forward.argtypes = [vp, vp, vp, i, vp, ctypes.c_uint]
    L.biv_hip_moe_forward_device.argtypes = [vp, vp, vp, i, vp, ctypes.c_uint]
    L.biv_hip_moe_forward_device_noalloc.argtypes = [vp, vp, vp, i, vp, ctypes.c_uint]
    L.biv_hip_moe_forward_taps.argtypes = [vp, vp, vp, i, vp, ctypes.c_uint, ctypes.POINTER(Taps)]
    L.biv_hip_malloc.argtypes = [vp, sz, pp]
    L.biv_hip_free.argtypes = [vp, vp]
    L.biv_hip_memcpy_h2d.argtypes = [vp, vp, vp, sz]
    L.biv_hip_memcpy_d2h.argtypes = [vp, vp, vp, sz]
    L.biv_hip_numerics.argtypes = [vp, ctypes.c_char_p, sz]
    L.biv_hip_device_bytes.argtypes = [vp]
    L.biv_hip_device_bytes.restype = sz
    L.biv_hip_set_timing.argtypes = [vp, i]
    L.biv_hip_stage_times.argtypes = [vp, ctypes.POINTER(ctypes.c_double), i, ctypes.POINTER(ctypes.c_int)]
    L.biv_hip_rms_norm.argtypes = [vp, vp, vp, i, i, ctypes.c_float]
    L.biv_hip_moe_ffn_step.argtypes = [vp, vp, vp, vp, ctypes.c_float, i]
    L.biv_hip_dense_create.argtypes = [vp, vp, vp, vp, pp]
    L.biv_hip_dense_forward.argtypes = [vp, vp, vp, i, vp, ctypes.c_uint]
    L.biv_hip_dense_forward_device.argtypes = [vp, vp, vp, i, vp, ctypes.c_uint]
    L.biv_hip_time_stage.argtypes = [vp, ctypes.POINTER(ctypes.c_void_p), i, vp, i, vp, i, i,
                                     ctypes.POINTER(ctypes.c_double)]
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data


class HipMoe:
    """A MoE layer on the device: the counterpart of model::Moe."""

    def __init__(self, ctx, handle, layer):
        self.ctx = ctx
        self.handle = handle
        self.n_embd = layer.n_embd
        self.n_expert = layer.n_expert
        self.k = layer.k
        self.n_ff = layer.n_ff
        self.has_shared = layer.shared is not None

    def ffn(self, h, n=None, out=None, add=False):
        """Model::ffn for a MoE layer (model.rs:853-898): the block's output for
        the n tokens of h [n x n_embd]; with add=True, out += the block."""
        h = np.ascontiguousarray(h, dtype=np.float32).reshape(-1, self.n_embd)
        n = h.shape[0] if n is None else n
        if out is None:
            out = np.zeros((n, self.n_embd), np.float32)
        self.ctx._check(self.ctx.L.biv_hip_moe_forward(self.ctx.h, self.handle, _ptr(h), n, _ptr(out),
                                                       ADD if add else 0))
        return out

    def ffn_taps(self, h, add=False, out=None, dots=True):
        """ffn with the debug taps: returns (out, dict of taps); dots=False
        skips the per-block int32 taps (large at prefill sizes)."""
        h = np.ascontiguousarray(h, dtype=np.float32).reshape(-1, self.n_embd)
        n, k, E, ff = h.shape[0], self.k, self.n_embd, self.n_ff
        P, R = n * k, n * k + n
        t = dict(
            ids=np.zeros((n, k), np.int32), weights=np.zeros((n, k), np.float32),
            logits=np.zeros((n, self.n_expert), np.float32), shared_logit=np.zeros(n, np.float32),
            pair_token=np.zeros(P, np.int32), pair_expert=np.zeros(P, np.int32),
            gate_idots=np.zeros((R, ff, E // 32), np.int32) if dots else None,
            up_idots=np.zeros((R, ff, E // 32), np.int32) if dots else None,
            act_q=np.zeros((R, ff), np.int8), act_d=np.zeros((R, ff // 32), np.float32),
            down_idots=np.zeros((R, E, ff // 32), np.int32) if dots else None)
        if not dots:
            for name in ("gate_idots", "up_idots", "down_idots"):
                t[name] = None
        taps = Taps(**{name: (arr.ctypes.data if arr is not None else None) for name, arr in t.items()})
        if out is None:
            out = np.zeros((n, E), np.float32)
        self.ctx._check(self.ctx.L.biv_hip_moe_forward_taps(self.ctx.h, self.handle, _ptr(h), n, _ptr(out),
                                                            ADD if add else 0, ctypes.byref(taps)))
        return out, t

    def ffn_step_device(self, x_dev, norm_dev, eps, n):
        """The feed-forward half of Model::layer (model.rs:788-790) in device
        memory: x += moe(rms_norm(x, norm, eps)) for n rows."""
        self.ctx._check(self.ctx.L.biv_hip_moe_ffn_step(self.ctx.h, self.handle, x_dev, norm_dev, eps, n))

    def forward_device(self, h_dev, n, out_dev, add=False):
        """encode_moe's counterpart: device pointers, queued on the context's stream."""
        self.ctx._check(self.ctx.L.biv_hip_moe_forward_device(self.ctx.h, self.handle, ctypes.c_void_p(h_dev), n,
                                                              ctypes.c_void_p(out_dev), ADD if add else 0))


    def forward_device_noalloc(self, h_dev, n, out_dev, add=False):
        """forward_device through the entry point that allocates nothing (its
        scratch is the library's fixed device buffer, shared by every call on
        the GPU)."""
        self.ctx._check(self.ctx.L.biv_hip_moe_forward_device_noalloc(
            self.ctx.h, self.handle, ctypes.c_void_p(h_dev), n, ctypes.c_void_p(out_dev), ADD if add else 0))


class HipDense:
    """A dense SwiGLU FFN layer on the device: the counterpart of
    Ffn::Dense (model.rs:239-246)."""

    def __init__(self, ctx, handle, n_embd, n_ff):
        self.ctx = ctx
        self.handle = handle
        self.n_embd = n_embd
        self.n_ff = n_ff

    def ffn(self, h, out=None, add=False):
        """dense_ffn (model.rs:1118-1126) of the rows of h: host arrays."""
        h = np.ascontiguousarray(h, dtype=np.float32).reshape(-1, self.n_embd)
        n = h.shape[0]
        if out is None:
            out = np.zeros((n, self.n_embd), np.float32)
        self.ctx._check(self.ctx.L.biv_hip_dense_forward(self.ctx.h, self.handle, _ptr(h), n, _ptr(out),
                                                         ADD if add else 0))
        return out

    def forward_device(self, h_dev, n, out_dev, add=False):
        self.ctx._check(self.ctx.L.biv_hip_dense_forward_device(self.ctx.h, self.handle, ctypes.c_void_p(h_dev), n,
                                                                ctypes.c_void_p(out_dev), ADD if add else 0))


class HipEngine:
    """A context on one GPU: owns the uploads, the scratch and the stream."""

    def __init__(self, device=0):
        self.L = load()
        h = ctypes.c_void_p()
        rc = self.L.biv_hip_create(device, ctypes.byref(h))
        if rc:
            raise HipError(rc, self.L.biv_hip_last_error(None).decode())
        self.h = h
        self._keep = []

    def _check(self, rc):
        if rc:
            raise HipError(rc, self.L.biv_hip_last_error(self.h).decode())

    def close(self):
        if self.h:
            self.L.biv_hip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload_weight(self, w):
        out = ctypes.c_void_p()
        self._check(self.L.biv_hip_upload_weight(self.h, w.ty, w.cols, w.rows, _ptr(w.data), ctypes.byref(out)))
        return out

    def upload_experts(self, x):
        out = ctypes.c_void_p()
        self._check(self.L.biv_hip_upload_experts(self.h, x.ty, x.cols, x.rows, x.n, _ptr(x.data), x.stride,
                                                  x.offset, ctypes.byref(out)))
        return out

    def moe(self, layer: "synth.MoeLayer"):
        """Upload a layer's parts and make the device MoE block."""
        router = self.upload_weight(layer.router)
        gate, up, down = (self.upload_experts(x) for x in (layer.gate, layer.up, layer.down))
        sh = [None] * 4
        if layer.shared is not None:
            sh = [self.upload_weight(w) for w in layer.shared]
        out = ctypes.c_void_p()
        self._check(self.L.biv_hip_moe_create(self.h, router, gate, up, down, *sh, layer.k, ctypes.byref(out)))
        return HipMoe(self, out, layer)

    def dense(self, layer: "synth.DenseLayer"):
        """Upload a dense FFN layer (gate, up, down) and create it."""
        g, u, d = (self.upload_weight(w) for w in (layer.gate, layer.up, layer.down))
        h = ctypes.c_void_p()
        self._check(self.L.biv_hip_dense_create(self.h, g, u, d, ctypes.byref(h)))
        return HipDense(self, h, layer.n_embd, layer.n_ff)

    def set_stream(self, stream_ptr):
        self._check(self.L.biv_hip_set_stream(self.h, ctypes.c_void_p(stream_ptr)))

    def sync(self):
        self._check(self.L.biv_hip_sync(self.h))

    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self._check(self.L.biv_hip_malloc(self.h, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, p):
        self._check(self.L.biv_hip_free(self.h, ctypes.c_void_p(p)))

    def h2d(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self._check(self.L.biv_hip_memcpy_h2d(self.h, ctypes.c_void_p(dst), _ptr(arr), arr.nbytes))

    def d2h(self, arr, src):
        self._check(self.L.biv_hip_memcpy_d2h(self.h, _ptr(arr), ctypes.c_void_p(src), arr.nbytes))
        return arr

    def numerics(self):
        buf = ctypes.create_string_buffer(512)
        self._check(self.L.biv_hip_numerics(self.h, buf, 512))
        return dict(kv.split("=", 1) for kv in buf.value.decode().split(";") if kv)

    def device_bytes(self):
        return self.L.biv_hip_device_bytes(self.h)

    def set_timing(self, enable):
        self._check(self.L.biv_hip_set_timing(self.h, 1 if enable else 0))

    def stage_times(self):
        """(summed ms per stage, number of forwards) since the last call."""
        ms = (ctypes.c_double * len(STAGES))()
        n = ctypes.c_int()
        self._check(self.L.biv_hip_stage_times(self.h, ms, len(STAGES), ctypes.byref(n)))
        return dict(zip(STAGES, list(ms))), n.value

    def rms_norm_device(self, x_dev, w_dev, rows, n, eps):
        """ops::rms_norm in place on device memory (queued on the stream)."""
        self._check(self.L.biv_hip_rms_norm(self.h, x_dev, w_dev, rows, n, eps))

    def rms_norm(self, x, w, eps):
        """ops::rms_norm of the host rows x [rows, n] by w [n]: a new array."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, n = x.shape
        xd, wd = self.malloc(x.nbytes), self.malloc(w.nbytes)
        try:
            self.h2d(xd, x)
            self.h2d(wd, w)
            self.rms_norm_device(xd, wd, rows, n, eps)
            out = np.empty_like(x)
            self.d2h(out, xd)
        finally:
            self.free(xd)
            self.free(wd)
        return out

    def time_stage(self, moes, h_dev, n, out_dev, stage, reps):
        """ms per launch of one stage (a name of STAGES) run alone, back to
        back, over the layers `moes` in turn (after one full forward of the
        first for the routing)."""
        arr = (ctypes.c_void_p * len(moes))(*[m.handle for m in moes])
        ms = ctypes.c_double()
        self._check(self.L.biv_hip_time_stage(self.h, arr, len(moes), h_dev, n, out_dev, STAGES.index(stage), reps,
                                              ctypes.byref(ms)))
        return ms.value
