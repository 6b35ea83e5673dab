"""Synthetic qwen35moe MoE layers: seeded N(0, std) weights quantised to ggml
blocks, and hidden-state inputs.

The containers mirror biv's weight views: `Weight` is ops::Weight
(engine/src/ops.rs:12-43), `Experts` is model::Experts (model.rs:190-217),
`MoeLayer` is model::Moe with its SharedExpert (model.rs:219-237).  Byte
layouts are ggml's (engine/src/quant.rs:50-68, dequantize_row 156-349).

biv only dequantises; it has no weight quantiser.  The quantisers here are
simple ones of our own: any valid block is a valid test input, because the
GPU and the CPU oracle read the same bytes.
"""
import os
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np

F32, F16, Q8_0, Q4K, Q6K, BF16 = 0, 1, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4K: (256, 144), Q6K: (256, 210)}
NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q8_0: "Q8_0", Q4K: "Q4_K", Q6K: "Q6_K"}


def row_size(ty, n):
    be, bb = BLOCK[ty]
    assert n % be == 0
    return n // be * bb


@dataclass
class Weight:
    ty: int
    cols: int
    rows: int
    data: np.ndarray  # uint8, rows * row_size(cols)


@dataclass
class Experts:
    ty: int
    cols: int
    rows: int
    n: int
    data: np.ndarray  # uint8
    stride: int       # bytes from an expert's matrix to the next
    offset: int = 0   # bytes from an expert's matrix to these rows

    def expert(self, e):
        start = e * self.stride + self.offset
        return self.data[start:start + self.rows * row_size(self.ty, self.cols)]

    @property
    def nbytes(self):
        return self.n * self.rows * row_size(self.ty, self.cols)


@dataclass
class MoeLayer:
    n_embd: int
    n_expert: int
    k: int
    n_ff: int
    n_ff_sh: int
    router: Weight
    gate: Experts
    up: Experts
    down: Experts
    shared: Optional[Tuple[Weight, Weight, Weight, Weight]]  # gate, up, down, gate_inp


def _round_away(x):
    """Round half away from zero (to within f32 rounding of x + 0.5: any
    nearby integer makes a valid block, so this need not be exact)."""
    x = np.asarray(x, dtype=np.float32)
    return np.trunc(x + np.copysign(np.float32(0.5), x))


def _f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def quantize_q8_0(x):
    """[rows, cols] f32 -> [rows, cols/32*34] uint8 (ggml's quantize_row_q8_0 method)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    nb = cols // 32
    xb = x.reshape(rows, nb, 32)
    amax = np.abs(xb).max(-1)
    d = (amax / np.float32(127)).astype(np.float32)
    safe = np.where(d != 0, d, np.float32(1))
    inv = np.where(d != 0, np.float32(1) / safe, np.float32(0)).astype(np.float32)
    q = np.clip(_round_away((xb * inv[..., None]).astype(np.float32)), -127, 127).astype(np.int8)
    out = np.empty((rows, nb, 34), np.uint8)
    out[..., 0:2] = _f16(d).view(np.uint8).reshape(rows, nb, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(rows, nb * 34)


def quantize_q4k(x):
    """[rows, cols] f32 -> [rows, cols/256*144] uint8: 8 sub-blocks of 32 with
    6-bit scales and mins under f16 d and dmin (layout of quant.rs:268-285)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    nsb = cols // 256
    xs = x.reshape(rows, nsb, 8, 32)
    mn = np.minimum(xs.min(-1), 0.0)
    mx = xs.max(-1)
    scale = (mx - mn) / np.float32(15)
    mins = -mn
    d16 = _f16(scale.max(-1) / np.float32(63))
    dm16 = _f16(mins.max(-1) / np.float32(63))
    df, dmf = d16.astype(np.float32), dm16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[..., None] > 0, np.clip(_round_away(scale / df[..., None]), 0, 63), 0).astype(np.uint8)
        m = np.where(dmf[..., None] > 0, np.clip(_round_away(mins / dmf[..., None]), 0, 63), 0).astype(np.uint8)
        eff_d = df[..., None] * sc.astype(np.float32)
        eff_m = dmf[..., None] * m.astype(np.float32)
        q = np.where(eff_d[..., None] > 0,
                     np.clip(_round_away((xs + eff_m[..., None]) / eff_d[..., None]), 0, 15), 0).astype(np.uint8)
    out = np.empty((rows, nsb, 144), np.uint8)
    out[..., 0:2] = d16.view(np.uint8).reshape(rows, nsb, 2)
    out[..., 2:4] = dm16.view(np.uint8).reshape(rows, nsb, 2)
    s = out[..., 4:16]
    for j in range(4):
        s[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        s[..., j + 4] = (m[..., j] & 63) | ((m[..., j + 4] >> 4) << 6)
        s[..., j + 8] = (sc[..., j + 4] & 0xF) | ((m[..., j + 4] & 0xF) << 4)
    for j in range(4):
        out[..., 16 + 32 * j:16 + 32 * j + 32] = q[..., 2 * j, :] | (q[..., 2 * j + 1, :] << 4)
    return out.reshape(rows, nsb * 144)


def quantize_q6k(x):
    """[rows, cols] f32 -> [rows, cols/256*210] uint8: 16 sub-blocks of 16 with
    int8 scales under an f16 d, 6-bit values (layout of quant.rs:327-346)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    nsb = cols // 256
    xs = x.reshape(rows, nsb, 16, 16)
    scale = np.abs(xs).max(-1) / np.float32(31)
    d16 = _f16(scale.max(-1) / np.float32(127))
    df = d16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[..., None] > 0, np.clip(_round_away(scale / df[..., None]), -128, 127), 0).astype(np.int8)
        eff = df[..., None] * sc.astype(np.float32)
        q = np.where(eff[..., None] != 0, np.clip(_round_away(xs / eff[..., None]), -32, 31), 0).astype(np.int16)
    v = (q + 32).astype(np.uint8).reshape(rows, nsb, 2, 128)
    out = np.empty((rows, nsb, 210), np.uint8)
    for n in range(2):
        h = v[:, :, n, :]
        ql = out[..., 64 * n:64 * n + 64]
        ql[..., 0:32] = (h[..., 0:32] & 0xF) | ((h[..., 64:96] & 0xF) << 4)
        ql[..., 32:64] = (h[..., 32:64] & 0xF) | ((h[..., 96:128] & 0xF) << 4)
        out[..., 128 + 32 * n:160 + 32 * n] = ((h[..., 0:32] >> 4) | ((h[..., 32:64] >> 4) << 2)
                                               | ((h[..., 64:96] >> 4) << 4) | ((h[..., 96:128] >> 4) << 6))
    out[..., 192:208] = sc.view(np.uint8)
    out[..., 208:210] = d16.view(np.uint8).reshape(rows, nsb, 2)
    return out.reshape(rows, nsb * 210)


def to_bf16(x):
    """f32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def quantize(ty, x):
    x = np.asarray(x, dtype=np.float32)
    if ty == Q8_0:
        return quantize_q8_0(x)
    if ty == Q4K:
        return quantize_q4k(x)
    if ty == Q6K:
        return quantize_q6k(x)
    if ty == BF16:
        return to_bf16(x).view(np.uint8).reshape(x.shape[0], -1)
    if ty == F32:
        return np.ascontiguousarray(x).view(np.uint8).reshape(x.shape[0], -1)
    raise ValueError(f"no quantiser for type {ty}")


def _normal(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def make_experts(rng, ty, cols, rows, n, std=0.02):
    """n matrices; expert e is drawn from its own stream spawned from rng, so
    the bytes do not depend on how many threads quantise them."""
    from concurrent.futures import ThreadPoolExecutor
    rb = row_size(ty, cols)
    data = np.empty(n * rows * rb, np.uint8)
    seeds = rng.spawn(n)

    def one(e):
        data[e * rows * rb:(e + 1) * rows * rb] = quantize(ty, _normal(seeds[e], (rows, cols), std)).reshape(-1)

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(one, range(n)))
    return Experts(ty, cols, rows, n, data, rows * rb, 0)


def make_weight(rng, ty, cols, rows, std=0.02):
    return Weight(ty, cols, rows, quantize(ty, _normal(rng, (rows, cols), std)).reshape(-1))


def fuse_gate_up(gate, up):
    """One ffn_gate_up_exps stack: per expert the gate rows then the up rows
    (model.rs:389-399); returns the (gate, up) views with stride and offset."""
    rb = row_size(gate.ty, gate.cols)
    half = gate.rows * rb
    both = np.empty(gate.n * 2 * half, np.uint8)
    for e in range(gate.n):
        both[2 * e * half:(2 * e + 1) * half] = gate.expert(e)
        both[(2 * e + 1) * half:(2 * e + 2) * half] = up.expert(e)
    g = Experts(gate.ty, gate.cols, gate.rows, gate.n, both, 2 * half, 0)
    u = Experts(up.ty, up.cols, up.rows, up.n, both, 2 * half, half)
    return g, u


def make_layer(seed, n_embd=2048, n_expert=256, k=8, n_ff=512, n_ff_sh=512, types=(Q8_0, Q8_0, Q8_0),
               shared=True, shared_types=None, fused_gate_up=False, std=0.02):
    """A MoE layer with weights ~N(0, std) from `seed`: router and gate_inp in
    F32, experts quantised to types = (gate, up, down)."""
    rng = np.random.default_rng(seed)
    gty, uty, dty = types
    router = Weight(F32, n_embd, n_expert, _normal(rng, (n_expert, n_embd), std).view(np.uint8).reshape(-1))
    gate = make_experts(rng, gty, n_embd, n_ff, n_expert, std)
    up = make_experts(rng, uty, n_embd, n_ff, n_expert, std)
    down = make_experts(rng, dty, n_ff, n_embd, n_expert, std)
    if fused_gate_up:
        gate, up = fuse_gate_up(gate, up)
    sh = None
    if shared:
        sg_t, su_t, sd_t = shared_types or types
        sh = (make_weight(rng, sg_t, n_embd, n_ff_sh, std), make_weight(rng, su_t, n_embd, n_ff_sh, std),
              make_weight(rng, sd_t, n_ff_sh, n_embd, std),
              Weight(F32, n_embd, 1, _normal(rng, (1, n_embd), std).view(np.uint8).reshape(-1)))
    return MoeLayer(n_embd, n_expert, k, n_ff, n_ff_sh if shared else 0, router, gate, up, down, sh)


@dataclass(frozen=True)
class DenseLayer:
    """Ffn::Dense of a qwen35 layer (model.rs:239-246)."""
    n_embd: int
    n_ff: int
    gate: Weight
    up: Weight
    down: Weight


def make_dense(seed, n_embd=2048, n_ff=3584, types=(Q8_0, Q8_0, Q8_0), std=0.02):
    """A dense SwiGLU FFN with weights ~N(0, std) from `seed`, quantised to
    types = (gate, up, down)."""
    rng = np.random.default_rng(seed)
    gty, uty, dty = types
    return DenseLayer(n_embd, n_ff, make_weight(rng, gty, n_embd, n_ff, std), make_weight(rng, uty, n_embd, n_ff, std),
                      make_weight(rng, dty, n_ff, n_embd, std))


def make_tokens(seed, T, n_embd=2048, offsets=False):
    """Hidden states ~N(0, 1), [T x n_embd] f32; with offsets, each token also
    gets a seeded offset vector of its own so tokens route to distinct experts."""
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((T, n_embd), dtype=np.float32)
    if offsets:
        h += np.float32(0.5) * rng.standard_normal((T, n_embd), dtype=np.float32)
    return h.astype(np.float32)


def zipf_bias_tokens(layer, seed, T, s=1.1, scale=0.13):
    """Hidden states whose router logits carry a per-expert bias
    b_e = -scale * s * ln(rank_e) (a Zipf(s) popularity over a seeded ranking;
    scale 0.13 puts ~60 of the 512 tokens on the hottest expert):
    h = z + mu with router . mu = b (least squares), so every token shares the
    bias and expert loads are skewed."""
    rng = np.random.default_rng(seed)
    ne, E = layer.n_expert, layer.n_embd
    rank = rng.permutation(ne) + 1
    b = (-scale * s * np.log(rank)).astype(np.float64)
    b -= b.mean()
    W = layer.router.data.view(np.float32).reshape(ne, E).astype(np.float64)
    mu, *_ = np.linalg.lstsq(W, b, rcond=None)
    z = rng.standard_normal((T, E), dtype=np.float32)
    return (z + mu.astype(np.float32)[None, :]).astype(np.float32)
