"""MI355X grouped-query attention path of the TinyLlama engine.

Python view of the C ABI in include/tla_attention.h (libtla.so, built for
gfx950 by __graft_entry__.build()).  The product is the shared library; this
module is the ctypes binding the tests and bench.py drive it through.  There
is no CPU fallback: if libtla.so is missing, importing `lib()` raises.

Interfaces mirrored (reference files):
    Engine.rope        rope()       src/ops.h:175-176
    Engine.softmax     softmax()    src/ops.h:107
    Engine.attention   attention()  src/ops.h:204-206
    Engine.rope_attention   the block of forward() src/forward.cpp:192-208
    Engine.decode      batched / multi-layer decode (one attention() per
                       (sequence, layer))
    Engine.prefill     the prompt loop src/generate.cpp:56-59, batched
    Engine.kv_cache    RunState::key_cache / value_cache src/run_state.h:93-101
    Engine.matmul / rmsnorm / vec_add / silu / elementwise_mul / ffn_swiglu
                       the ops of src/ops.h:64-66, 95-96, 118, 131, 143, 232-235
    Engine.attn_qkv / attn_out / ffn_block
                       the halves of a layer src/forward.cpp:180-228
    Engine.embed       embed_token() src/forward.cpp:17-134
    Engine.argmax      sample_argmax() src/ops.h:249
    Engine.forward     forward() src/forward.cpp:167-266 (DeviceModel weights)
    Engine.generate_greedy  the generation loop src/generate.cpp:56-100 at
                       temperature 0
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtla.so")
HOST_LIB_PATH = os.path.join(HERE, "libtla_host.so")

TLA_OK = 0
TLA_ERR_INVALID_ARGUMENT = 1
TLA_ERR_OUT_OF_RANGE = 2
TLA_ERR_UNSUPPORTED = 3
TLA_ERR_DEVICE = 4
TLA_ERR_OUT_OF_MEMORY = 5
TLA_ROTATE = 1
TLA_BATCH_PROMPT = 2
TLA_KV_IN_CACHE = 4

KERNEL_DECODE, KERNEL_PREFILL, KERNEL_APPEND, KERNEL_GEMV = range(4)
# weight formats: the reference's ggml_type ids (src/gguf.h:23-32)
W_F32, W_F16, W_Q4_0, W_Q8_0, W_Q6_K = 0, 1, 2, 8, 14
OPT_DECODE_SPLIT, OPT_DECODE_PLAN, OPT_DECODE_GROUP = 0, 1, 2
OPT_STREAM_TILES = 3
OPT_SPLIT_ROWS = 4
OPT_SPLIT_K = 5
PLAN_AUTO, PLAN_ALIGNED, PLAN_BALANCED = 0, 1, 2
READ_GLOBAL, READ_GLOBAL_NT, READ_BUFFER, READ_BUFFER_NT = 0, 1, 2, 3


class TlaError(RuntimeError):
    def __init__(self, code: int, what: str, msg: str):
        super().__init__(f"{what} failed (status {code}): {msg}")
        self.code = code


class Config(C.Structure):
    """tla_config: the llama_config_t fields the path uses (src/gguf.h:139-168)."""

    _fields_ = [("n_layers", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int),
                ("n_head_kv", C.c_int), ("n_ctx", C.c_int), ("rope_freq_base", C.c_float)]

    @classmethod
    def tinyllama(cls, n_layers=22, n_ctx=2048):
        return cls(n_layers, 2048, 32, 4, n_ctx, 10000.0)

    @property
    def head_dim(self):
        return self.n_embd // self.n_head

    @property
    def kv_dim(self):
        return self.n_head_kv * self.head_dim


_vp = C.c_void_p
_lib = None


class LayerWeights(C.Structure):
    """tla_layer_weights: one layer's device tensors and ggml types."""

    _fields_ = [("attn_norm", _vp), ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wo", _vp),
                ("type_q", C.c_int), ("type_k", C.c_int), ("type_v", C.c_int), ("type_o", C.c_int),
                ("ffn_norm", _vp), ("w_gate", _vp), ("w_up", _vp), ("w_down", _vp),
                ("type_ffn", C.c_int)]


class Model(C.Structure):
    """tla_model: the weights forward() reads (src/forward.cpp:167-266)."""

    _fields_ = [("n_ff", C.c_int), ("n_vocab", C.c_int), ("rms_norm_eps", C.c_float),
                ("token_embd", _vp), ("type_embd", C.c_int), ("output_norm", _vp),
                ("output", _vp), ("type_output", C.c_int), ("layers", C.POINTER(LayerWeights))]

# name -> (restype, argtypes); every symbol declared in include/tla_attention.h
SIGNATURES = {
    "tla_last_error": (C.c_char_p, []),
    "tla_abi_version": (C.c_int, []),
    "tla_engine_create": (C.c_int, [C.POINTER(Config), C.c_int, C.POINTER(_vp)]),
    "tla_engine_destroy": (C.c_int, [_vp]),
    "tla_synchronize": (C.c_int, [_vp]),
    "tla_alloc": (C.c_int, [_vp, C.c_size_t, C.POINTER(_vp)]),
    "tla_free": (C.c_int, [_vp, _vp]),
    "tla_kv_cache_alloc": (C.c_int, [_vp, C.c_int, C.POINTER(_vp), C.POINTER(_vp)]),
    "tla_memcpy_h2d": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "tla_memcpy_d2h": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "tla_memcpy_d2d": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "tla_rope": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
    "tla_softmax": (C.c_int, [_vp, _vp, C.c_int]),
    "tla_matmul": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int]),
    "tla_matmul_batch": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tla_rmsnorm": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_float]),
    "tla_vec_add": (C.c_int, [_vp, _vp, _vp, C.c_int]),
    "tla_attn_qkv": (C.c_int, [_vp, C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp,
                               C.c_int]),
    "tla_attn_out": (C.c_int, [_vp, C.c_int, _vp, _vp, _vp, C.c_int]),
    "tla_silu": (C.c_int, [_vp, _vp, C.c_int]),
    "tla_elementwise_mul": (C.c_int, [_vp, _vp, _vp, C.c_int]),
    "tla_ffn_swiglu": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int,
                                 C.c_int]),
    "tla_ffn_block": (C.c_int, [_vp, C.c_int, _vp, _vp, C.c_float, _vp, _vp, _vp, C.c_int,
                                C.c_int, _vp]),
    "tla_embed": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tla_argmax": (C.c_int, [_vp, _vp, C.c_int, C.POINTER(C.c_int)]),
    "tla_matmul_argmax": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "tla_forward": (C.c_int, [_vp, C.POINTER(Model), _vp, _vp, C.c_int, C.c_int, _vp]),
    "tla_prefill_forward": (C.c_int, [_vp, C.POINTER(Model), _vp, _vp, C.POINTER(C.c_int), C.c_int,
                                      C.c_int, _vp]),
    "tla_generate_greedy": (C.c_int, [_vp, C.POINTER(Model), _vp, _vp, C.POINTER(C.c_int), C.c_int,
                                      C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "tla_attention": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int]),
    "tla_rope_attention": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int]),
    "tla_rope_attention_host": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int]),
    "tla_host_alloc": (C.c_int, [_vp, C.c_size_t, C.POINTER(_vp)]),
    "tla_host_free": (C.c_int, [_vp, _vp]),
    "tla_decode": (C.c_int, [_vp, C.c_int, C.POINTER(C.c_int), C.c_int, C.c_int, C.c_int,
                             _vp, _vp, _vp, _vp, _vp, _vp, C.c_size_t]),
    "tla_decode_noalloc": (C.c_int, [_vp, C.c_int, C.POINTER(C.c_int), C.c_int, C.c_int, C.c_int,
                                     _vp, _vp, _vp, _vp, _vp, _vp, C.c_size_t]),
    "tla_prefill": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                              _vp, _vp, _vp, _vp, _vp, _vp]),
    "tla_profile_enable": (C.c_int, [_vp, C.c_int]),
    "tla_profile_read": (C.c_int, [_vp, C.c_int, C.POINTER(C.c_double),
                                   C.POINTER(C.c_longlong)]),
    "tla_event_record": (C.c_int, [_vp, C.c_int]),
    "tla_event_elapsed": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "tla_set_option": (C.c_int, [_vp, C.c_int, C.c_longlong]),
    "tla_read_floor": (C.c_int, [_vp, _vp, C.c_size_t, C.c_int, C.c_int, C.c_int, _vp]),
    "tla_mfma_floor": (C.c_int, [_vp, C.c_int, C.c_int, _vp]),
}


def lib() -> C.CDLL:
    """Load libtla.so (raises if it was never built -- no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build the HIP extension first (__graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().tla_last_error().decode()


def _check(rc: int, what: str):
    if rc != TLA_OK:
        raise TlaError(rc, what, last_error())


class DeviceArray:
    """A device allocation with a numpy-like shape and dtype (float32/int32)."""

    def __init__(self, engine: "Engine", shape, dtype=np.float32, ptr=None, owner=True):
        self.engine = engine
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.owner = owner
        if ptr is None:
            p = _vp()
            _check(lib().tla_alloc(engine.h, max(self.nbytes, 4), C.byref(p)), "tla_alloc")
            ptr = p.value
        self.ptr = ptr

    def upload(self, host: np.ndarray):
        host = np.ascontiguousarray(host, dtype=self.dtype)
        assert host.nbytes == self.nbytes, (host.shape, self.shape)
        _check(lib().tla_memcpy_h2d(self.engine.h, self.ptr, host.ctypes.data, self.nbytes),
               "tla_memcpy_h2d")
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _check(lib().tla_memcpy_d2h(self.engine.h, out.ctypes.data, self.ptr, self.nbytes),
               "tla_memcpy_d2h")
        return out

    def at(self, byte_offset: int) -> int:
        return self.ptr + byte_offset

    def free(self):
        if self.owner and self.ptr:
            _check(lib().tla_free(self.engine.h, self.ptr), "tla_free")
        self.ptr = None


class Engine:
    """One tla_engine: device, stream, RoPE table, split-KV workspace."""

    def __init__(self, cfg: Config, device: int = 0):
        self.cfg = cfg
        h = _vp()
        _check(lib().tla_engine_create(C.byref(cfg), device, C.byref(h)), "tla_engine_create")
        self.h = h.value

    def close(self):
        if self.h:
            lib().tla_engine_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- memory -------------------------------------------------------------
    def array(self, host_or_shape, dtype=np.float32) -> DeviceArray:
        if isinstance(host_or_shape, np.ndarray):
            a = DeviceArray(self, host_or_shape.shape, host_or_shape.dtype)
            return a.upload(host_or_shape)
        return DeviceArray(self, host_or_shape, dtype)

    def kv_cache(self, n_seq: int = 1):
        """(key_cache, value_cache) device arrays [n_seq, n_layers, n_ctx, kv_dim], zeroed."""
        k, v = _vp(), _vp()
        _check(lib().tla_kv_cache_alloc(self.h, n_seq, C.byref(k), C.byref(v)),
               "tla_kv_cache_alloc")
        shape = (n_seq, self.cfg.n_layers, self.cfg.n_ctx, self.cfg.kv_dim)
        return DeviceArray(self, shape, ptr=k.value), DeviceArray(self, shape, ptr=v.value)

    def copy(self, dst: int, src: int, nbytes: int):
        _check(lib().tla_memcpy_d2d(self.h, dst, src, nbytes), "tla_memcpy_d2d")

    def synchronize(self):
        _check(lib().tla_synchronize(self.h), "tla_synchronize")

    # ---- operators --------------------------------------------------------------
    def rope(self, q: int, k: int, pos: int, head_dim=64, n_head=32, n_head_kv=4,
             freq_base=10000.0):
        _check(lib().tla_rope(self.h, q, k, pos, head_dim, n_head, n_head_kv, freq_base),
               "tla_rope")

    def softmax(self, x: int, size: int):
        _check(lib().tla_softmax(self.h, x, size), "tla_softmax")

    def attention(self, out: int, q: int, k: int, v: int, key_cache: int, value_cache: int,
                  layer: int, pos: int, att: int = 0):
        _check(lib().tla_attention(self.h, out, q, k, v, key_cache, value_cache, att or None,
                                   layer, pos), "tla_attention")

    def rope_attention_host(self, out_host: int, qkv_host: int, qkv_dev: int, out_dev: int,
                            key_cache: int, value_cache: int, layer: int, pos: int):
        _check(lib().tla_rope_attention_host(self.h, out_host, qkv_host, qkv_dev, out_dev, key_cache,
                                             value_cache, layer, pos), "tla_rope_attention_host")

    def host_alloc(self, nbytes: int) -> int:
        p = _vp()
        _check(lib().tla_host_alloc(self.h, nbytes, C.byref(p)), "tla_host_alloc")
        return p.value

    def host_free(self, ptr: int):
        _check(lib().tla_host_free(self.h, ptr), "tla_host_free")

    def rope_attention(self, out: int, q: int, k: int, v: int, key_cache: int,
                       value_cache: int, layer: int, pos: int):
        _check(lib().tla_rope_attention(self.h, out, q, k, v, key_cache, value_cache, layer, pos),
               "tla_rope_attention")

    def decode(self, pos, layer0: int, n_step_layers: int, out: int, q: int, k: int, v: int,
               key_cache: int, value_cache: int, seq_stride: int = 0, rotate: bool = True,
               kv_in_cache: bool = False):
        pos = np.ascontiguousarray(pos, dtype=np.int32).reshape(-1)
        flags = (TLA_ROTATE if rotate else 0) | (TLA_KV_IN_CACHE if kv_in_cache else 0)
        _check(lib().tla_decode(self.h, int(pos.size), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                layer0, n_step_layers, flags, out, q, k, v,
                                key_cache, value_cache, seq_stride), "tla_decode")

    def prefill(self, pos0: int, n_tok: int, layer0: int, n_step_layers: int, out: int, q: int,
                k: int, v: int, key_cache: int, value_cache: int, rotate: bool = True):
        _check(lib().tla_prefill(self.h, pos0, n_tok, layer0, n_step_layers,
                                 TLA_ROTATE if rotate else 0, out, q, k, v, key_cache,
                                 value_cache), "tla_prefill")

    # ---- projections either side of the attention block -------------------------
    def matmul(self, out: int, w: int, x: int, rows: int, cols: int, wtype: int):
        _check(lib().tla_matmul(self.h, out, w, x, rows, cols, wtype), "tla_matmul")

    def rmsnorm(self, out: int, x: int, weight: int, size: int, eps: float):
        _check(lib().tla_rmsnorm(self.h, out, x, weight, size, eps), "tla_rmsnorm")

    def vec_add(self, out: int, x: int, size: int):
        _check(lib().tla_vec_add(self.h, out, x, size), "tla_vec_add")

    def attn_qkv(self, n_seq: int, q: int, k: int, v: int, x: int, norm_w: int | None, eps: float,
                 wq: int, wk: int, wv: int, wtype: int):
        _check(lib().tla_attn_qkv(self.h, n_seq, q, k, v, x, norm_w, eps, wq, wk, wv, wtype),
               "tla_attn_qkv")

    def attn_out(self, n_seq: int, x: int, wo: int, xb2: int, wtype: int):
        _check(lib().tla_attn_out(self.h, n_seq, x, wo, xb2, wtype), "tla_attn_out")

    def matmul_batch(self, out: int, w: int, x: int, rows: int, cols: int, n_tok: int, wtype: int):
        _check(lib().tla_matmul_batch(self.h, out, w, x, rows, cols, n_tok, wtype), "tla_matmul_batch")

    def silu(self, x: int, size: int):
        _check(lib().tla_silu(self.h, x, size), "tla_silu")

    def elementwise_mul(self, a: int, b: int, size: int):
        _check(lib().tla_elementwise_mul(self.h, a, b, size), "tla_elementwise_mul")

    def ffn_swiglu(self, out: int, inp: int, hb: int, hb2: int, w_gate: int, w_up: int,
                   w_down: int, n_ff: int, n_embd: int, wtype: int):
        _check(lib().tla_ffn_swiglu(self.h, out, inp, hb, hb2, w_gate, w_up, w_down, n_ff, n_embd,
                                    wtype), "tla_ffn_swiglu")

    def ffn_block(self, n_seq: int, x: int, norm_w: int, eps: float, w_gate: int, w_up: int,
                  w_down: int, n_ff: int, wtype: int, hb: int):
        _check(lib().tla_ffn_block(self.h, n_seq, x, norm_w, eps, w_gate, w_up, w_down, n_ff, wtype,
                                   hb), "tla_ffn_block")

    def embed(self, out: int, table: int, token: int, n_embd: int, n_vocab: int, wtype: int):
        _check(lib().tla_embed(self.h, out, table, token, n_embd, n_vocab, wtype), "tla_embed")

    def argmax(self, logits: int, n_vocab: int) -> int:
        t = C.c_int()
        _check(lib().tla_argmax(self.h, logits, n_vocab, C.byref(t)), "tla_argmax")
        return t.value

    def matmul_argmax(self, out: int, w: int, x: int, rows: int, cols: int, wtype: int) -> int:
        t = C.c_int()
        _check(lib().tla_matmul_argmax(self.h, out, w, x, rows, cols, wtype, C.byref(t)),
               "tla_matmul_argmax")
        return t.value

    def forward(self, model: "DeviceModel", kc: int, vc: int, token: int, pos: int, logits: int):
        _check(lib().tla_forward(self.h, C.byref(model.c), kc, vc, token, pos, logits),
               "tla_forward")

    def prefill_forward(self, model: "DeviceModel", kc: int, vc: int, tokens, pos0: int, logits: int):
        p = (C.c_int * len(tokens))(*[int(t) for t in tokens])
        _check(lib().tla_prefill_forward(self.h, C.byref(model.c), kc, vc, p, len(tokens), pos0,
                                         logits), "tla_prefill_forward")

    def generate_greedy(self, model: "DeviceModel", kc: int, vc: int, prompt, n_gen: int,
                        batch_prompt: bool = False):
        p = (C.c_int * len(prompt))(*[int(t) for t in prompt])
        out = (C.c_int * n_gen)()
        _check(lib().tla_generate_greedy(self.h, C.byref(model.c), kc, vc, p, len(prompt), n_gen,
                                         TLA_BATCH_PROMPT if batch_prompt else 0, out),
               "tla_generate_greedy")
        return list(out)

    # ---- measurement --------------------------------------------------------------
    def set_option(self, option: int, value: int):
        _check(lib().tla_set_option(self.h, option, value), "tla_set_option")

    def profile(self, enable: bool):
        _check(lib().tla_profile_enable(self.h, int(enable)), "tla_profile_enable")

    def profile_read(self, kernel_id: int):
        ms, n = C.c_double(), C.c_longlong()
        _check(lib().tla_profile_read(self.h, kernel_id, C.byref(ms), C.byref(n)),
               "tla_profile_read")
        return ms.value, n.value

    def read_floor(self, src: int, nbytes: int, n_workgroups: int, sink: int,
                   kind: int = READ_GLOBAL, depth: int = 8):
        _check(lib().tla_read_floor(self.h, src, nbytes, n_workgroups, kind, depth, sink),
               "tla_read_floor")

    def mfma_floor(self, n_workgroups: int, iters: int, sink: int):
        _check(lib().tla_mfma_floor(self.h, n_workgroups, iters, sink), "tla_mfma_floor")

    def event(self, slot: int):
        _check(lib().tla_event_record(self.h, slot), "tla_event_record")

    def elapsed(self, a: int, b: int) -> float:
        ms = C.c_float()
        _check(lib().tla_event_elapsed(self.h, a, b, C.byref(ms)), "tla_event_elapsed")
        return ms.value


class DeviceModel:
    """A model's tensors copied to the device unchanged and described as a
    tla_model.  `tensors` maps GGUF tensor names to (dims, ggml type, raw
    bytes), the names forward() looks up (src/forward.cpp:167-266);
    output.weight falls back to token_embd.weight (tied embeddings)."""

    def __init__(self, engine: Engine, tensors: dict, n_ff: int, n_vocab: int, eps: float):
        self.engine = engine
        self.arrays = {}
        for name, (dims, ty, raw) in tensors.items():
            self.arrays[name] = engine.array(np.ascontiguousarray(raw, np.uint8))
        ptr = lambda n: self.arrays[n].ptr  # noqa: E731
        ty = lambda n: tensors[n][1]  # noqa: E731
        n_layers = engine.cfg.n_layers
        self.layers = (LayerWeights * n_layers)()
        for l in range(n_layers):
            p = f"blk.{l}."
            self.layers[l] = LayerWeights(
                ptr(p + "attn_norm.weight"), ptr(p + "attn_q.weight"), ptr(p + "attn_k.weight"),
                ptr(p + "attn_v.weight"), ptr(p + "attn_output.weight"), ty(p + "attn_q.weight"),
                ty(p + "attn_k.weight"), ty(p + "attn_v.weight"), ty(p + "attn_output.weight"),
                ptr(p + "ffn_norm.weight"), ptr(p + "ffn_gate.weight"), ptr(p + "ffn_up.weight"),
                ptr(p + "ffn_down.weight"), ty(p + "ffn_gate.weight"))
        out = "output.weight" if "output.weight" in tensors else "token_embd.weight"
        self.c = Model(n_ff, n_vocab, eps, ptr("token_embd.weight"), ty("token_embd.weight"),
                       ptr("output_norm.weight"), ptr(out), ty(out), self.layers)
        self.weight_bytes = sum(a.nbytes for a in self.arrays.values())

    def free(self):
        for a in self.arrays.values():
            a.free()
        self.arrays = {}
