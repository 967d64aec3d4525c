"""Seeded synthetic inputs and work counts for the attention path.

Shapes are TinyLlama's (n_head 32, n_head_kv 4, head_dim 64, RoPE theta 1e4).
Inputs come from numpy's PCG64 generator (`standard_normal`, float32), seeded
from a fixed base and the workload id, so the host side of a test, the
golden-vector script and bench.py all see the same numbers.

Workloads (one new token per (sequence, layer) unless stated):
    decode_single   1 layer, position 127, cache rows 0..126 filled
    decode_model    22 layers, context 2048 (position 2047)
    decode_ragged   64 sequences, positions uniform in [255, 2047], 22 layers
    prefill         512-token prompt, 22 layers, RoPE in-kernel
    decode_long     16384 context, batch 8, 22 layers, K,V ~ N(0, 0.5^2) with
                    1% of (position, kv head) key rows scaled x8
"""
from __future__ import annotations

import hashlib

import numpy as np

SEED_BASE = 0x7A11A

N_HEAD, N_HEAD_KV, HEAD_DIM = 32, 4, 64
Q_DIM, KV_DIM = N_HEAD * HEAD_DIM, N_HEAD_KV * HEAD_DIM
FREQ_BASE = 10000.0

WORKLOAD_IDS = {"decode_single": 1, "decode_model": 2, "decode_ragged": 3, "prefill": 4,
                "decode_long": 5, "weights": 6, "block": 7}


def rng(workload: str | int, salt: int = 0) -> np.random.Generator:
    wid = WORKLOAD_IDS[workload] if isinstance(workload, str) else int(workload)
    return np.random.default_rng([SEED_BASE, wid, salt])


def normal(g: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    x = g.standard_normal(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    if std != 1.0:
        x *= np.float32(std)
    return x


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ---- algorithmic work --------------------------------------------------------

def decode_bytes(length: int, n_head=N_HEAD, n_head_kv=N_HEAD_KV, head_dim=HEAD_DIM) -> int:
    """HBM bytes one (sequence, layer) decode step must move at L = pos+1.

    K and V read once (not once per q head) + q in + out + new k,v in +
    appended k,v out.  For TinyLlama: 2048*L + 20480.
    """
    kv = n_head_kv * head_dim * 4
    qd = n_head * head_dim * 4
    return 2 * length * kv + 2 * qd + 4 * kv


def prefill_flops(n_tok: int, n_head=N_HEAD, head_dim=HEAD_DIM, pos0: int = 0) -> int:
    """Exact causal flops of QK^T plus PV: token t sees pos0+t+1 keys."""
    keys = n_tok * pos0 + n_tok * (n_tok + 1) // 2
    return 2 * 2 * n_head * head_dim * keys


# ---- decode inputs -----------------------------------------------------------

class DecodeCase:
    """Host arrays for n_seq sequences x n_layers layers, one new token each.

    cache rows 0..pos-1 of every (sequence, layer) are filled; row pos and
    later are zero (the new token is appended at pos).
    """

    def __init__(self, n_seq, n_layers, n_ctx, pos, q, k, v, kc, vc, n_head=N_HEAD,
                 n_head_kv=N_HEAD_KV):
        self.n_seq, self.n_layers, self.n_ctx = n_seq, n_layers, n_ctx
        self.n_head, self.n_head_kv = n_head, n_head_kv
        self.pos = np.asarray(pos, np.int32)
        self.q, self.k, self.v = q, k, v   # [n_seq, n_layers, heads*64]
        self.kc, self.vc = kc, vc          # [n_seq, n_layers, n_ctx, kv heads*64]

    @property
    def algorithmic_bytes(self) -> int:
        return int(sum(decode_bytes(int(p) + 1) for p in self.pos) * self.n_layers)


def make_decode(workload: str | int, n_seq: int, n_layers: int, n_ctx: int, pos,
                kv_std: float = 1.0, peaked_frac: float = 0.0, peaked_scale: float = 8.0,
                salt: int = 0, n_head: int = N_HEAD, n_head_kv: int = N_HEAD_KV) -> DecodeCase:
    g = rng(workload, salt)
    q_dim, kv_dim = n_head * HEAD_DIM, n_head_kv * HEAD_DIM
    pos = np.broadcast_to(np.asarray(pos, np.int32), (n_seq,)).copy()
    q = normal(g, (n_seq, n_layers, q_dim))
    k = normal(g, (n_seq, n_layers, kv_dim))
    v = normal(g, (n_seq, n_layers, kv_dim))
    kc = np.zeros((n_seq, n_layers, n_ctx, kv_dim), np.float32)
    vc = np.zeros_like(kc)
    for s in range(n_seq):
        n = int(pos[s])
        if n == 0:
            continue
        kc[s, :, :n] = normal(g, (n_layers, n, kv_dim), kv_std)
        vc[s, :, :n] = normal(g, (n_layers, n, kv_dim), kv_std)
        if peaked_frac > 0:
            rows = kc[s, :, :n].reshape(n_layers, n, n_head_kv, HEAD_DIM)
            hit = g.random((n_layers, n, n_head_kv)) < peaked_frac
            rows[hit] *= np.float32(peaked_scale)
    return DecodeCase(n_seq, n_layers, n_ctx, pos, q, k, v, kc, vc, n_head, n_head_kv)


def decode_single() -> DecodeCase:
    return make_decode("decode_single", 1, 1, 128, 127)


def decode_model(n_layers: int = 22, n_ctx: int = 2048, salt: int = 0) -> DecodeCase:
    return make_decode("decode_model", 1, n_layers, n_ctx, n_ctx - 1, salt=salt)


def ragged_positions(n_seq: int = 64, lo: int = 256, hi: int = 2048) -> np.ndarray:
    """Context lengths uniform in [lo, hi] from the seed; returns pos = L - 1."""
    g = rng("decode_ragged", 1000)
    return (g.integers(lo, hi + 1, size=n_seq) - 1).astype(np.int32)


def decode_ragged(n_seq: int = 64, n_layers: int = 22, n_ctx: int = 2048) -> DecodeCase:
    return make_decode("decode_ragged", n_seq, n_layers, n_ctx, ragged_positions(n_seq))


def decode_long(n_seq: int = 8, n_layers: int = 22, n_ctx: int = 16384) -> DecodeCase:
    return make_decode("decode_long", n_seq, n_layers, n_ctx, n_ctx - 1, kv_std=0.5,
                       peaked_frac=0.01)


# The long-context workloads are timed with one layer's data in every layer
# (the byte stream per layer is the same, and host generation stays a few
# seconds): these are the one-layer cases, replicated by replicate_layers()
# or, on the device, copied into every layer's slice of the cache.

def decode_long_layer(n_seq: int = 8, n_ctx: int = 16384) -> DecodeCase:
    """Context 16384, batch 8, peaked keys: one layer."""
    return decode_long(n_seq=n_seq, n_layers=1, n_ctx=n_ctx)


def decode_sweep_layer(n_ctx: int) -> DecodeCase:
    """Batch 1, new token at the last position of an n_ctx cache: one layer."""
    return make_decode("decode_model", 1, 1, n_ctx, n_ctx - 1, salt=n_ctx)


def replicate_layers(one: DecodeCase, n_layers: int) -> DecodeCase:
    """A one-layer case with its inputs repeated for n_layers layers (host
    arrays, n_layers times the one layer's memory)."""
    rep = lambda a: np.ascontiguousarray(np.repeat(a, n_layers, axis=1))  # noqa: E731
    return DecodeCase(one.n_seq, n_layers, one.n_ctx, one.pos, rep(one.q), rep(one.k), rep(one.v),
                      rep(one.kc), rep(one.vc), one.n_head, one.n_head_kv)


# ---- prefill inputs -------------------------------------------------------------

class PrefillCase:
    def __init__(self, n_layers, n_tok, pos0, q, k, v, n_head=N_HEAD, n_head_kv=N_HEAD_KV):
        self.n_layers, self.n_tok, self.pos0 = n_layers, n_tok, pos0
        self.n_head, self.n_head_kv = n_head, n_head_kv
        self.q, self.k, self.v = q, k, v   # [n_layers, n_tok, dim]

    @property
    def algorithmic_flops(self) -> int:
        return prefill_flops(self.n_tok, n_head=self.n_head, pos0=self.pos0) * self.n_layers


def make_prefill(n_layers: int = 22, n_tok: int = 512, pos0: int = 0, salt: int = 0,
                 n_head: int = N_HEAD, n_head_kv: int = N_HEAD_KV) -> PrefillCase:
    g = rng("prefill", salt)
    q = normal(g, (n_layers, n_tok, n_head * HEAD_DIM))
    k = normal(g, (n_layers, n_tok, n_head_kv * HEAD_DIM))
    v = normal(g, (n_layers, n_tok, n_head_kv * HEAD_DIM))
    return PrefillCase(n_layers, n_tok, pos0, q, k, v, n_head, n_head_kv)


# ---- weights in the reference's GGUF formats ---------------------------------
# Type ids: ggml_type (src/gguf.h:23-32); block layouts src/gguf.h:56-135.
W_F32, W_F16, W_Q4_0, W_Q8_0, W_Q6_K = 0, 1, 2, 8, 14
W_NAMES = {W_F32: "f32", W_F16: "f16", W_Q4_0: "q4_0", W_Q8_0: "q8_0", W_Q6_K: "q6_k"}


def weight_row_bytes(wtype: int, cols: int) -> int:
    return {W_F32: 4 * cols, W_F16: 2 * cols, W_Q8_0: 34 * (cols // 32),
            W_Q4_0: 18 * (cols // 32), W_Q6_K: 210 * (cols // 256)}[wtype]


def _f16_bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, np.float16).view(np.uint8).reshape(*np.shape(a), 2)


def make_weights(wtype: int, rows: int, cols: int, salt: int = 0) -> np.ndarray:
    """Seeded random weights as the raw bytes (uint8, [rows * row_bytes]) of a
    row-major [rows][cols] matrix.  Scales are chosen so W.x with x ~ N(0,1)
    stays O(1) per row at cols = 2048."""
    g = rng("weights", salt * 64 + wtype)
    if wtype == W_F32:
        return normal(g, (rows, cols), 0.02).view(np.uint8).reshape(-1)
    if wtype == W_F16:
        return _f16_bits(normal(g, (rows, cols), 0.02)).reshape(-1)
    if wtype == W_Q8_0:
        nb = cols // 32
        blk = np.empty((rows, nb, 34), np.uint8)
        blk[..., 0:2] = _f16_bits(g.uniform(0.0002, 0.0003, (rows, nb)))
        blk[..., 2:34] = g.integers(-128, 128, (rows, nb, 32)).astype(np.int8).view(np.uint8)
        return blk.reshape(-1)
    if wtype == W_Q4_0:
        nb = cols // 32
        blk = np.empty((rows, nb, 18), np.uint8)
        blk[..., 0:2] = _f16_bits(g.uniform(0.003, 0.006, (rows, nb)))
        blk[..., 2:18] = g.integers(0, 256, (rows, nb, 16)).astype(np.uint8)
        return blk.reshape(-1)
    if wtype == W_Q6_K:
        nb = cols // 256
        blk = np.empty((rows, nb, 210), np.uint8)
        blk[..., 0:192] = g.integers(0, 256, (rows, nb, 192)).astype(np.uint8)
        blk[..., 192:208] = g.integers(-32, 32, (rows, nb, 16)).astype(np.int8).view(np.uint8)
        blk[..., 208:210] = _f16_bits(g.uniform(0.0001, 0.0002, (rows, nb)))
        return blk.reshape(-1)
    raise ValueError(wtype)


# ---- a whole model with seeded random weights ----------------------------------
# Tensor names and shapes as the reference's forward() reads them from a GGUF
# file (src/forward.cpp:167-266); dims are GGUF order (ne0 = columns).

class ModelSpec:
    def __init__(self, n_layers, n_embd, n_head, n_head_kv, n_ff, n_vocab, n_ctx,
                 rope_freq_base=FREQ_BASE, rms_norm_eps=1e-5):
        self.n_layers, self.n_embd, self.n_head, self.n_head_kv = n_layers, n_embd, n_head, n_head_kv
        self.n_ff, self.n_vocab, self.n_ctx = n_ff, n_vocab, n_ctx
        self.rope_freq_base, self.rms_norm_eps = rope_freq_base, rms_norm_eps

    @property
    def head_dim(self):
        return self.n_embd // self.n_head

    @property
    def kv_dim(self):
        return self.n_head_kv * self.head_dim


def tinyllama_spec(n_ctx: int = 2048) -> ModelSpec:
    return ModelSpec(22, 2048, 32, 4, 5632, 32000, n_ctx)


def make_model(spec: ModelSpec, wtype: int = W_Q8_0, salt: int = 0, embd_type: int | None = None,
               output_type: int | None = W_Q6_K, norm_scale: float = 1.0,
               overrides: dict | None = None):
    """{name: (dims, ggml type, raw bytes)} for every tensor forward() reads.
    Weights come from make_weights (seeded per tensor), norms are F32 in
    [0.5, 1.5) * norm_scale.  output_type None ties the classifier to
    token_embd.weight (no output.weight tensor), as TinyLlama files do.
    overrides maps a tensor-name suffix ("attn_v.weight") to another type."""
    e, kv, ff = spec.n_embd, spec.kv_dim, spec.n_ff
    g = rng("weights", 100000 + salt)
    t = {}
    overrides = overrides or {}

    def weight(name, rows, cols, ty, s):
        for suffix, oty in overrides.items():
            if name.endswith(suffix):
                ty = oty
        t[name] = ((cols, rows), ty, make_weights(ty, rows, cols, salt=salt * 4096 + s))

    def norm(name):
        v = (g.uniform(0.5, 1.5, e) * norm_scale).astype(np.float32)
        t[name] = ((e,), W_F32, v.view(np.uint8))

    weight("token_embd.weight", spec.n_vocab, e, wtype if embd_type is None else embd_type, 1)
    for l in range(spec.n_layers):
        p = f"blk.{l}."
        s = 16 * (l + 1)
        norm(p + "attn_norm.weight")
        weight(p + "attn_q.weight", e, e, wtype, s + 1)
        weight(p + "attn_k.weight", kv, e, wtype, s + 2)
        weight(p + "attn_v.weight", kv, e, wtype, s + 3)
        weight(p + "attn_output.weight", e, e, wtype, s + 4)
        norm(p + "ffn_norm.weight")
        weight(p + "ffn_gate.weight", ff, e, wtype, s + 5)
        weight(p + "ffn_up.weight", ff, e, wtype, s + 6)
        weight(p + "ffn_down.weight", e, ff, wtype, s + 7)
    norm("output_norm.weight")
    if output_type is not None:
        weight("output.weight", spec.n_vocab, e, output_type, 2)
    return t
