"""ctypes loaders for the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package: to check the HIP results, or as the CPU baseline.  The HIP product
(tinyllama-engine_amd/) never imports or links anything here.

Two libraries:
  liboracle.so         plain-C restatement of the reference's rope / softmax /
                       attention (tl_oracle.c, see its header for citations)
  _ref/libref_ops.so   the reference's own src/ops.cpp, compiled by
                       oracle/Makefile where /root/reference exists; optional.
  _ref/libref_forward.so  the reference's forward pass and GGUF loader
                       (forward.cpp, gguf_model.cpp, tokenizer.cpp, ops.cpp),
                       same origin; optional.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref_ops.so")
REF_FWD_SO = os.path.join(HERE, "_ref", "libref_forward.so")
REF_SRC = "/root/reference/src"

_fp = C.POINTER(C.c_float)
_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int)


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_fp)


def dptr(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_dp)


def iptr(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_ip)


def build(with_ref: bool | None = None) -> None:
    """Compile liboracle.so, and _ref/libref_ops.so when the reference tree exists."""
    targets = ["all"]
    if with_ref is None:
        with_ref = os.path.isdir(REF_SRC)
    if with_ref:
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


_oracle = None
_ref = None


def oracle() -> C.CDLL:
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            build(with_ref=False)
        lib = C.CDLL(ORACLE_SO)
        lib.oracle_fault.argtypes = [C.c_int]
        lib.oracle_rope.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        lib.oracle_rope_table.argtypes = [_fp, C.c_int, C.c_int, C.c_float]
        lib.oracle_softmax.argtypes = [_fp, C.c_int]
        lib.oracle_attention.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp,
                                         C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
        lib.oracle_attention_f64.argtypes = [_dp, _fp, _fp, _fp, C.c_int, C.c_int,
                                             C.c_int, C.c_int, C.c_int, C.c_int]
        lib.oracle_prefill.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        lib.oracle_decode_units_mt.argtypes = [C.c_int, C.c_int, _fp, _fp, _fp, _fp, _fp, _fp,
                                               C.c_size_t, _ip, C.c_int, C.c_int, C.c_int,
                                               C.c_int, C.c_float, C.c_int]
        lib.oracle_decode_units_mt.restype = C.c_int
        lib.oracle_fp16_to_f32.argtypes = [C.c_uint16]
        lib.oracle_fp16_to_f32.restype = C.c_float
        lib.oracle_row_bytes.argtypes = [C.c_int, C.c_int]
        lib.oracle_row_bytes.restype = C.c_longlong
        lib.oracle_matmul.argtypes = [_fp, C.c_void_p, _fp, C.c_int, C.c_int, C.c_int]
        lib.oracle_matmul.restype = C.c_int
        lib.oracle_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        lib.oracle_vec_add.argtypes = [_fp, _fp, C.c_int]
        lib.oracle_silu.argtypes = [_fp, C.c_int]
        lib.oracle_elementwise_mul.argtypes = [_fp, _fp, C.c_int]
        lib.oracle_ffn_swiglu.argtypes = [_fp, _fp, _fp, _fp, C.c_void_p, C.c_void_p, C.c_void_p,
                                          C.c_int, C.c_int, C.c_int]
        lib.oracle_ffn_swiglu.restype = C.c_int
        lib.oracle_embed.argtypes = [_fp, C.c_void_p, C.c_int, C.c_int, C.c_int]
        lib.oracle_embed.restype = C.c_int
        lib.oracle_argmax.argtypes = [_fp, C.c_int]
        lib.oracle_argmax.restype = C.c_int
        lib.oracle_forward.argtypes = [C.c_void_p, _fp, _fp, _fp, C.c_int, C.c_int, _fp]
        lib.oracle_forward.restype = C.c_int
        _oracle = lib
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref() -> C.CDLL:
    """The compiled reference; raises if oracle/_ref was never built."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_SO):
            raise FileNotFoundError(REF_SO)
        lib = C.CDLL(REF_SO)
        lib.ref_rope.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        lib.ref_softmax.argtypes = [_fp, C.c_int]
        lib.ref_attention.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, C.c_int, C.c_int,
                                      C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
        lib.ref_decode_units_mt.argtypes = [C.c_int, C.c_int, _fp, _fp, _fp, _fp, _fp, _fp,
                                            C.c_size_t, _ip, C.c_int, C.c_int, C.c_int,
                                            C.c_int, C.c_float, C.c_int]
        lib.ref_decode_units_mt.restype = C.c_int
        lib.ref_prefill.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, C.c_int, C.c_int, C.c_int,
                                    C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        lib.ref_matmul.argtypes = [_fp, C.c_void_p, _fp, C.c_int, C.c_int, C.c_int]
        lib.ref_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        lib.ref_vec_add.argtypes = [_fp, _fp, C.c_int]
        lib.ref_fp16_to_f32.argtypes = [C.c_uint16]
        lib.ref_fp16_to_f32.restype = C.c_float
        lib.ref_silu.argtypes = [_fp, C.c_int]
        lib.ref_elementwise_mul.argtypes = [_fp, _fp, C.c_int]
        lib.ref_ffn_swiglu.argtypes = [_fp, _fp, _fp, _fp, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_int, C.c_int, C.c_int]
        lib.ref_argmax.argtypes = [_fp, C.c_int]
        lib.ref_argmax.restype = C.c_int
        _ref = lib
    return _ref


# ---- numpy-level helpers (same calling convention as the reference) -------

class Shape:
    """TinyLlama attention shape: llama_config_t fields src/gguf.h:139-168."""

    def __init__(self, n_head=32, n_head_kv=4, head_dim=64, n_ctx=2048, n_layers=1,
                 freq_base=10000.0):
        self.n_head, self.n_head_kv, self.head_dim = n_head, n_head_kv, head_dim
        self.n_ctx, self.n_layers, self.freq_base = n_ctx, n_layers, freq_base

    @property
    def kv_dim(self):
        return self.n_head_kv * self.head_dim

    @property
    def q_dim(self):
        return self.n_head * self.head_dim


def rope(q, k, pos, s: Shape, lib=None):
    """In-place rope on copies; returns (q', k')."""
    q = np.ascontiguousarray(q, dtype=np.float32).copy()
    k = np.ascontiguousarray(k, dtype=np.float32).copy()
    if lib is None:
        oracle().oracle_rope(fptr(q), fptr(k), pos, s.head_dim, s.n_head, s.n_head_kv, s.freq_base)
    else:
        lib.ref_rope(fptr(q), fptr(k), pos, s.head_dim, s.n_head, s.n_head_kv, s.freq_base)
    return q, k


def softmax(x, lib=None):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    (oracle().oracle_softmax if lib is None else lib.ref_softmax)(fptr(x), x.size)
    return x


def attention(q, k, v, kc, vc, layer, pos, s: Shape, lib=None):
    """attention() on the given caches (mutated in place: append at pos)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(s.q_dim, np.float32)
    att = np.zeros(s.n_ctx, np.float32)
    if lib is None:
        oracle().oracle_attention(fptr(out), fptr(q), fptr(k), fptr(v), fptr(kc), fptr(vc),
                                  fptr(att), layer, pos, s.n_head, s.n_head_kv, s.head_dim,
                                  s.n_ctx)
    else:
        lib.ref_attention(fptr(out), fptr(q), fptr(k), fptr(v), fptr(kc), fptr(vc), fptr(att),
                          layer, pos, s.n_layers, s.n_head, s.n_head_kv, s.head_dim, s.n_ctx)
    return out


def attention_f64(q, kc, vc, layer, pos, s: Shape):
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(s.q_dim, np.float64)
    oracle().oracle_attention_f64(dptr(out), fptr(q), fptr(kc), fptr(vc), layer, pos,
                                  s.n_head, s.n_head_kv, s.head_dim, s.n_ctx)
    return out


def prefill(q, k, v, kc, vc, layer, pos0, s: Shape, lib=None):
    """Token-by-token prompt loop; q [T, q_dim], k/v [T, kv_dim] raw.  With
    lib = ref(), the reference's own rope() + attention() do the loop."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    t = q.shape[0]
    out = np.zeros((t, s.q_dim), np.float32)
    fn = oracle().oracle_prefill if lib is None else lib.ref_prefill
    fn(fptr(out), fptr(q), fptr(k), fptr(v), fptr(kc), fptr(vc), layer, pos0, t, s.n_head,
       s.n_head_kv, s.head_dim, s.n_ctx, s.freq_base)
    return out


def rope_table(n_pos, head_dim=64, freq_base=10000.0):
    cs = np.zeros((n_pos, head_dim // 2, 2), np.float32)
    oracle().oracle_rope_table(fptr(cs), n_pos, head_dim, freq_base)
    return cs


def decode_units_mt(n_threads, q, k, v, kc, vc, pos, s: Shape, rotate=True, lib=None):
    """n_units independent decode steps; kc/vc [n_units, n_ctx, kv_dim] (mutated)."""
    n_units = q.shape[0]
    out = np.zeros((n_units, s.q_dim), np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    stride = s.n_ctx * s.kv_dim
    args = (n_threads, n_units, fptr(out), fptr(np.ascontiguousarray(q, np.float32)),
            fptr(np.ascontiguousarray(k, np.float32)), fptr(np.ascontiguousarray(v, np.float32)),
            fptr(kc), fptr(vc), stride, iptr(pos), s.n_head, s.n_head_kv, s.head_dim, s.n_ctx,
            s.freq_base, int(rotate))
    rc = (oracle().oracle_decode_units_mt if lib is None else lib.ref_decode_units_mt)(*args)
    assert rc == 0
    return out


# ---- projections either side of the attention block -----------------------
# Weight type ids are the reference's ggml_type values (src/gguf.h:23-32).
F32, F16, Q4_0, Q8_0, Q6_K = 0, 1, 2, 8, 14
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q6_K: 256}


def row_bytes(wtype: int, cols: int) -> int:
    return int(oracle().oracle_row_bytes(wtype, cols))


def matmul(W: np.ndarray, x: np.ndarray, rows: int, cols: int, wtype: int, lib=None) -> np.ndarray:
    """out[rows] = W . x with W the raw bytes (uint8) of a [rows][cols] matrix
    of type wtype; lib=ref() runs the reference's own matmul()."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert W.size == rows * row_bytes(wtype, cols)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(rows, np.float32)
    if lib is None:
        assert oracle().oracle_matmul(fptr(out), W.ctypes.data, fptr(x), rows, cols, wtype) == 0
    else:
        lib.ref_matmul(fptr(out), W.ctypes.data, fptr(x), rows, cols, wtype)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, lib=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    (oracle().oracle_rmsnorm if lib is None else lib.ref_rmsnorm)(fptr(out), fptr(x), fptr(w),
                                                                   x.size, eps)
    return out


def vec_add(out: np.ndarray, x: np.ndarray, lib=None) -> np.ndarray:
    out = np.ascontiguousarray(out, dtype=np.float32).copy()
    x = np.ascontiguousarray(x, dtype=np.float32)
    (oracle().oracle_vec_add if lib is None else lib.ref_vec_add)(fptr(out), fptr(x), out.size)
    return out


# ---- FFN, embedding, whole forward pass ------------------------------------

def silu(x: np.ndarray, lib=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    (oracle().oracle_silu if lib is None else lib.ref_silu)(fptr(x), x.size)
    return x


def ffn_swiglu(x, w_gate, w_up, w_down, n_ff, n_embd, wtype, lib=None):
    """(out, hb, hb2) of ffn_swiglu(); weights are raw bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(n_embd, np.float32)
    hb, hb2 = np.zeros(n_ff, np.float32), np.zeros(n_ff, np.float32)
    ws = [np.ascontiguousarray(w, np.uint8) for w in (w_gate, w_up, w_down)]
    f = oracle().oracle_ffn_swiglu if lib is None else lib.ref_ffn_swiglu
    rc = f(fptr(out), fptr(x), fptr(hb), fptr(hb2), ws[0].ctypes.data, ws[1].ctypes.data,
           ws[2].ctypes.data, n_ff, n_embd, wtype)
    assert lib is not None or rc == 0
    return out, hb, hb2


def embed(table, token: int, n_embd: int, wtype: int) -> np.ndarray:
    out = np.zeros(n_embd, np.float32)
    table = np.ascontiguousarray(table, np.uint8)
    assert oracle().oracle_embed(fptr(out), table.ctypes.data, token, n_embd, wtype) == 0
    return out


class _Layer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("wq", C.c_void_p), ("wk", C.c_void_p),
                ("wv", C.c_void_p), ("wo", C.c_void_p), ("type_q", C.c_int), ("type_k", C.c_int),
                ("type_v", C.c_int), ("type_o", C.c_int), ("ffn_norm", C.c_void_p),
                ("w_gate", C.c_void_p), ("w_up", C.c_void_p), ("w_down", C.c_void_p),
                ("type_ffn", C.c_int)]


class _Model(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int),
                ("n_head_kv", C.c_int), ("n_ff", C.c_int), ("n_vocab", C.c_int), ("n_ctx", C.c_int),
                ("rope_freq_base", C.c_float), ("rms_norm_eps", C.c_float),
                ("token_embd", C.c_void_p), ("type_embd", C.c_int), ("output_norm", C.c_void_p),
                ("output", C.c_void_p), ("type_output", C.c_int), ("layers", C.POINTER(_Layer))]


class Model:
    """The oracle's forward() over a model given as {name: (dims, type, raw
    bytes)} (workloads.make_model); keeps its own KV cache, like a RunState."""

    def __init__(self, spec, tensors):
        self.spec, self.t = spec, {k: (d, ty, np.ascontiguousarray(r, np.uint8))
                                   for k, (d, ty, r) in tensors.items()}
        ptr = lambda n: self.t[n][2].ctypes.data  # noqa: E731
        ty = lambda n: self.t[n][1]  # noqa: E731
        L = (_Layer * spec.n_layers)()
        for l in range(spec.n_layers):
            p = f"blk.{l}."
            L[l] = _Layer(ptr(p + "attn_norm.weight"), ptr(p + "attn_q.weight"),
                          ptr(p + "attn_k.weight"), ptr(p + "attn_v.weight"),
                          ptr(p + "attn_output.weight"), ty(p + "attn_q.weight"),
                          ty(p + "attn_k.weight"), ty(p + "attn_v.weight"),
                          ty(p + "attn_output.weight"), ptr(p + "ffn_norm.weight"),
                          ptr(p + "ffn_gate.weight"), ptr(p + "ffn_up.weight"),
                          ptr(p + "ffn_down.weight"), ty(p + "ffn_gate.weight"))
        out_name = "output.weight" if "output.weight" in self.t else "token_embd.weight"
        self._layers = L
        self._m = _Model(spec.n_layers, spec.n_embd, spec.n_head, spec.n_head_kv, spec.n_ff,
                         spec.n_vocab, spec.n_ctx, spec.rope_freq_base, spec.rms_norm_eps,
                         ptr("token_embd.weight"), ty("token_embd.weight"),
                         ptr("output_norm.weight"), ptr(out_name), ty(out_name), L)
        cache = spec.n_layers * spec.n_ctx * spec.kv_dim
        self.kc, self.vc = np.zeros(cache, np.float32), np.zeros(cache, np.float32)
        self.scratch = np.zeros(5 * spec.n_embd + 2 * spec.kv_dim + spec.n_ctx + 2 * spec.n_ff,
                                np.float32)

    def forward(self, token: int, pos: int) -> np.ndarray:
        logits = np.zeros(self.spec.n_vocab, np.float32)
        rc = oracle().oracle_forward(C.addressof(self._m), fptr(self.kc), fptr(self.vc),
                                     fptr(self.scratch), token, pos, fptr(logits))
        assert rc == 0
        return logits

    def tokens(self, tokens) -> np.ndarray:
        """Logits [n][n_vocab] of forward() at positions 0..n-1."""
        return np.stack([self.forward(int(t), i) for i, t in enumerate(tokens)])

    def greedy(self, prompt, n_gen: int):
        """The prompt loop, then argmax decoding (src/generate.cpp:56-100)."""
        pos = 0
        for t in prompt:
            logits = self.forward(int(t), pos)
            pos += 1
        out = []
        nxt = int(oracle().oracle_argmax(fptr(logits), logits.size))
        for i in range(n_gen):
            out.append(nxt)
            if i + 1 == n_gen:
                break
            logits = self.forward(nxt, pos)
            pos += 1
            nxt = int(oracle().oracle_argmax(fptr(logits), logits.size))
        return out


_ref_fwd = None


def ref_forward_available() -> bool:
    return os.path.exists(REF_FWD_SO)


def ref_forward():
    """The reference's own forward pass over a GGUF file (oracle/_ref)."""
    global _ref_fwd
    if _ref_fwd is None:
        lib = C.CDLL(REF_FWD_SO)
        lib.ref_forward_error.restype = C.c_char_p
        lib.ref_forward_tokens.argtypes = [C.c_char_p, _ip, C.c_int, _fp, _ip]
        lib.ref_forward_tokens.restype = C.c_int
        lib.ref_generate_greedy.argtypes = [C.c_char_p, _ip, C.c_int, C.c_int, _ip]
        lib.ref_generate_greedy.restype = C.c_int
        lib.ref_bench_trial.argtypes = [C.c_char_p, _ip, C.c_int, C.c_int, C.c_int, _dp, _dp]
        lib.ref_bench_trial.restype = C.c_int
        _ref_fwd = lib
    return _ref_fwd


def ref_forward_tokens(path: str, tokens, n_vocab: int) -> np.ndarray:
    lib = ref_forward()
    toks = np.ascontiguousarray(tokens, np.int32)
    logits = np.zeros((toks.size, n_vocab), np.float32)
    nv = np.zeros(1, np.int32)
    rc = lib.ref_forward_tokens(path.encode(), iptr(toks), toks.size, fptr(logits), iptr(nv))
    assert rc == 0, lib.ref_forward_error()
    assert nv[0] == n_vocab
    return logits


def ref_generate_greedy(path: str, prompt, n_gen: int):
    lib = ref_forward()
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.zeros(n_gen, np.int32)
    rc = lib.ref_generate_greedy(path.encode(), iptr(p), p.size, n_gen, iptr(out))
    assert rc == 0, lib.ref_forward_error()
    return out.tolist()


def ref_bench_trial(path: str, prompt, n_decode: int, threads: int):
    """(prefill ms, decode ms) of one trial of the reference's benchmark loop."""
    lib = ref_forward()
    p = np.ascontiguousarray(prompt, np.int32)
    a, b = np.zeros(1), np.zeros(1)
    rc = lib.ref_bench_trial(path.encode(), iptr(p), p.size, n_decode, threads, dptr(a), dptr(b))
    assert rc == 0, lib.ref_forward_error()
    return float(a[0]), float(b[0])
