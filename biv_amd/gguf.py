"""GGUF files for the MoE backend: a writer, and the library's reader and
layer loader over the C ABI (include/biv_hip.h, biv_gguf_*).

The reader is biv's (engine/src/gguf.rs) restated in the library: a GGUF or
the shards of a split one, memory-mapped, metadata key/values and the tensor
table; `moe_config` is the MoE part of Config (engine/src/model.rs:70-120)
and `HipEngine.moe_from_gguf` uploads one layer's MoE block as Loader::ffn
does (model.rs:386-421).

The writer produces the same container (version 3, little endian): it lets
tests and tools put synthetic qwen35moe layers in a file with the tensor
names biv's loader reads (engine/src/gguf/tensors.rs:115-131).
"""
import ctypes
import struct

import numpy as np

from . import hip, synth

# GGUF value types (gguf.rs:140-170)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}

E_INVALID, E_TYPE = -1, -2
E_FORMAT, E_IO, E_MISSING = -5, -6, -7


def _infer(v):
    if isinstance(v, bool):
        return BOOL
    if isinstance(v, int):
        return U32 if 0 <= v < 2 ** 32 else I64
    if isinstance(v, float):
        return F32
    if isinstance(v, str):
        return STRING
    if isinstance(v, (list, tuple)):
        return ARRAY
    raise TypeError(f"no GGUF type for {type(v)}")


def _pack_value(ty, v, elem_ty=None):
    if ty == STRING:
        b = v.encode()
        return struct.pack("<Q", len(b)) + b
    if ty == ARRAY:
        et = elem_ty if elem_ty is not None else (_infer(v[0]) if len(v) else U32)
        return struct.pack("<IQ", et, len(v)) + b"".join(_pack_value(et, x) for x in v)
    return struct.pack(_FMT[ty], v)


def write(path, kv, tensors, alignment=32, version=3):
    """Write a GGUF: kv is a list of (key, value) or (key, value, type) (the
    type inferred when absent; arrays take (key, list, ARRAY, elem_type)),
    tensors a list of (name, ggml_type, dims in ggml order, bytes)."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kv))
    body = []
    for item in kv:
        key, v = item[0], item[1]
        ty = item[2] if len(item) > 2 else _infer(v)
        et = item[3] if len(item) > 3 else None
        body.append(_pack_value(STRING, key) + struct.pack("<I", ty) + _pack_value(ty, v, et))
    offs, off = [], 0
    for name, ty, dims, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(bytes(data))
    for (name, ty, dims, data), o in zip(tensors, offs):
        body.append(_pack_value(STRING, name) + struct.pack("<I", len(dims)) +
                    b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, o))
    meta = head + b"".join(body)
    start = (len(meta) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(meta)
        f.write(b"\0" * (start - len(meta)))
        pos = 0
        for (name, ty, dims, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            b = bytes(data)
            f.write(b)
            pos = o + len(b)


def moe_layer_tensors(i, layer: "synth.MoeLayer"):
    """The tensors of blk.<i>'s MoE block, named and shaped as biv's loader
    reads them (model.rs:386-421); a fused gate_up stack (gate.offset == 0
    and up.offset > 0 in one buffer) is written as ffn_gate_up_exps."""
    p = f"blk.{i}."
    t = [(p + "ffn_gate_inp.weight", layer.router.ty, [layer.n_embd, layer.n_expert], layer.router.data)]
    g, u, d = layer.gate, layer.up, layer.down
    if u.offset > 0 and u.data is g.data:
        t.append((p + "ffn_gate_up_exps.weight", g.ty, [g.cols, 2 * g.rows, g.n], g.data))
    else:
        t.append((p + "ffn_gate_exps.weight", g.ty, [g.cols, g.rows, g.n], g.data[:g.nbytes]))
        t.append((p + "ffn_up_exps.weight", u.ty, [u.cols, u.rows, u.n], u.data[:u.nbytes]))
    t.append((p + "ffn_down_exps.weight", d.ty, [d.cols, d.rows, d.n], d.data[:d.nbytes]))
    if layer.shared is not None:
        sg, su, sd, gi = layer.shared
        t += [(p + "ffn_gate_shexp.weight", sg.ty, [sg.cols, sg.rows], sg.data),
              (p + "ffn_up_shexp.weight", su.ty, [su.cols, su.rows], su.data),
              (p + "ffn_down_shexp.weight", sd.ty, [sd.cols, sd.rows], sd.data),
              (p + "ffn_gate_inp_shexp.weight", gi.ty, [gi.cols], gi.data)]
    return t


def moe_kv(layers, eps=1e-6, arch="qwen35moe"):
    """The metadata Config reads for the MoE part (model.rs:70-120)."""
    l0 = layers[0]
    a = arch + "."
    return [("general.architecture", arch), (a + "block_count", len(layers)), (a + "embedding_length", l0.n_embd),
            (a + "expert_count", l0.n_expert), (a + "expert_used_count", l0.k),
            (a + "expert_feed_forward_length", l0.n_ff), (a + "expert_shared_feed_forward_length", l0.n_ff_sh),
            (a + "attention.layer_norm_rms_epsilon", float(eps))]


def write_moe(path, layers, eps=1e-6, alignment=32):
    """A GGUF holding the MoE blocks of `layers` as blk.0.., with their config."""
    tensors = [t for i, layer in enumerate(layers) for t in moe_layer_tensors(i, layer)]
    write(path, moe_kv(layers, eps), tensors, alignment=alignment)


def dense_layer_tensors(i, layer: "synth.DenseLayer"):
    """The tensors of blk.<i>'s dense FFN as Loader::ffn reads them
    (model.rs:381-386): gate and up [n_embd, n_ff], down [n_ff, n_embd]."""
    p = f"blk.{i}."
    return [(p + "ffn_" + name + ".weight", w.ty, [w.cols, w.rows], w.data)
            for name, w in (("gate", layer.gate), ("up", layer.up), ("down", layer.down))]


def dense_kv(layers, eps=1e-6, arch="qwen35"):
    """The metadata Config reads for a dense model's FFN (model.rs:70-131)."""
    l0 = layers[0]
    a = arch + "."
    return [("general.architecture", arch), (a + "block_count", len(layers)), (a + "embedding_length", l0.n_embd),
            (a + "feed_forward_length", l0.n_ff), (a + "attention.layer_norm_rms_epsilon", float(eps))]


def write_dense(path, layers, eps=1e-6, alignment=32):
    """A GGUF holding the dense FFNs of `layers` as blk.0.., with their config."""
    tensors = [t for i, layer in enumerate(layers) for t in dense_layer_tensors(i, layer)]
    write(path, dense_kv(layers, eps), tensors, alignment=alignment)


class DenseConfig(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_char * 32), ("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int),
                ("n_ff", ctypes.c_int), ("eps", ctypes.c_float)]


class MoeConfig(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_char * 32), ("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int),
                ("n_expert", ctypes.c_int), ("n_expert_used", ctypes.c_int), ("n_ff_exp", ctypes.c_int),
                ("n_ff_shexp", ctypes.c_int), ("eps", ctypes.c_float)]


def _lib():
    L = hip.load()
    if getattr(L, "_gguf_typed", False):
        return L
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.biv_gguf_open.argtypes = [ctypes.POINTER(ctypes.c_char_p), i, ctypes.POINTER(vp)]
    L.biv_gguf_close.argtypes = [vp]
    L.biv_gguf_close.restype = None
    L.biv_gguf_last_error.argtypes = [vp]
    L.biv_gguf_last_error.restype = ctypes.c_char_p
    L.biv_gguf_get_u64.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]
    L.biv_gguf_get_f32.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]
    L.biv_gguf_get_str.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, sz]
    L.biv_gguf_n_tensors.argtypes = [vp]
    L.biv_gguf_tensor_name.argtypes = [vp, i]
    L.biv_gguf_tensor_name.restype = ctypes.c_char_p
    L.biv_gguf_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(i), ctypes.POINTER(i),
                                  ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(vp), ctypes.POINTER(sz)]
    L.biv_gguf_read_moe_config.argtypes = [vp, ctypes.POINTER(MoeConfig)]
    L.biv_hip_moe_from_gguf.argtypes = [vp, vp, i, ctypes.POINTER(vp)]
    L.biv_gguf_read_dense_config.argtypes = [vp, ctypes.POINTER(DenseConfig)]
    L.biv_hip_dense_from_gguf.argtypes = [vp, vp, i, ctypes.POINTER(vp)]
    L._gguf_typed = True
    return L


class Gguf:
    """A GGUF (or its shards, in order) opened by the library: Gguf::from_shards."""

    def __init__(self, paths):
        self.L = _lib()
        if isinstance(paths, str):
            paths = [paths]
        arr = (ctypes.c_char_p * len(paths))(*[p.encode() for p in paths])
        h = ctypes.c_void_p()
        rc = self.L.biv_gguf_open(arr, len(paths), ctypes.byref(h))
        if rc:
            raise hip.HipError(rc, self.L.biv_gguf_last_error(None).decode())
        self.h = h

    def _check(self, rc):
        if rc:
            raise hip.HipError(rc, self.L.biv_gguf_last_error(self.h).decode())

    def close(self):
        if self.h:
            self.L.biv_gguf_close(self.h)
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

    def get_u64(self, key):
        v = ctypes.c_uint64()
        self._check(self.L.biv_gguf_get_u64(self.h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_f32(self, key):
        v = ctypes.c_float()
        self._check(self.L.biv_gguf_get_f32(self.h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_str(self, key, maxlen=4096):
        buf = ctypes.create_string_buffer(maxlen)
        self._check(self.L.biv_gguf_get_str(self.h, key.encode(), buf, maxlen))
        return buf.value.decode()

    def tensor_names(self):
        return [self.L.biv_gguf_tensor_name(self.h, i).decode() for i in range(self.L.biv_gguf_n_tensors(self.h))]

    def tensor(self, name):
        """(ggml type, dims, the mapped bytes as a read-only uint8 array)."""
        ty, nd = ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_uint64 * 4)()
        data, nb = ctypes.c_void_p(), ctypes.c_size_t()
        self._check(self.L.biv_gguf_tensor(self.h, name.encode(), ctypes.byref(ty), ctypes.byref(nd), dims,
                                           ctypes.byref(data), ctypes.byref(nb)))
        buf = (ctypes.c_uint8 * nb.value).from_address(data.value) if nb.value else (ctypes.c_uint8 * 0)()
        arr = np.frombuffer(buf, dtype=np.uint8)
        arr.flags.writeable = False
        return ty.value, list(dims[:nd.value]), arr

    def moe_config(self):
        cfg = MoeConfig()
        self._check(self.L.biv_gguf_read_moe_config(self.h, ctypes.byref(cfg)))
        return cfg


    def dense_config(self):
        cfg = DenseConfig()
        self._check(self.L.biv_gguf_read_dense_config(self.h, ctypes.byref(cfg)))
        return cfg


class _LayerShape:
    """The shape facts HipMoe keeps, from a GGUF's MoE config."""

    def __init__(self, cfg):
        self.n_embd, self.n_expert, self.k = cfg.n_embd, cfg.n_expert, cfg.n_expert_used
        self.n_ff = cfg.n_ff_exp
        self.shared = True if cfg.n_ff_shexp else None


def moe_from_gguf(engine: "hip.HipEngine", g: Gguf, layer: int) -> "hip.HipMoe":
    """Loader::ffn for MoE layer `layer` of the file, uploaded to the engine's GPU."""
    _lib()
    out = ctypes.c_void_p()
    engine._check(engine.L.biv_hip_moe_from_gguf(engine.h, g.h, layer, ctypes.byref(out)))
    return hip.HipMoe(engine, out, _LayerShape(g.moe_config()))


def dense_from_gguf(engine: "hip.HipEngine", g: Gguf, layer: int) -> "hip.HipDense":
    """Loader::ffn for dense layer `layer` of the file, uploaded to the engine's GPU."""
    _lib()
    cfg = g.dense_config()
    out = ctypes.c_void_p()
    engine._check(engine.L.biv_hip_dense_from_gguf(engine.h, g.h, layer, ctypes.byref(out)))
    return hip.HipDense(engine, out, cfg.n_embd, cfg.n_ff)
