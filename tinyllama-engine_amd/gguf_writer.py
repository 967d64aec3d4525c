"""Writes a GGUF (version 3) file: the header, metadata key/values, tensor
infos and aligned tensor data, per the published GGUF format (little endian:
magic "GGUF", u32 version, u64 tensor count, u64 kv count; strings are u64
length + bytes; tensor info = name, u32 n_dims, u64 dims (ne0 first), u32
ggml type, u64 offset from the aligned start of the data section).

Synthetic model files: the seeded random models of workloads.make_model
written in the layout the reference's GGUF loader reads (src/gguf_model.cpp),
so that the reference's own programs -- its forward pass, its `engine` and
`benchmark`, and those programs built on the drop-in attention path -- can
load the same weights the device path takes as pointers.  No compute."""
import struct

import numpy as np

GGUF_UINT32, GGUF_FLOAT32, GGUF_STRING, GGUF_ARRAY = 4, 6, 8, 9


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def byte_vocab(n_vocab: int) -> list:
    """A vocabulary the reference's tokenizer can load and encode any text
    with: its three special tokens (src/tokenizer.cpp:25-27), the 256 byte
    tokens "<0xNN>" of its byte fallback (src/tokenizer.cpp:153-160), then
    filler pieces up to n_vocab."""
    assert n_vocab >= 259
    toks = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    return toks + [f"\u2581w{i}" for i in range(n_vocab - len(toks))]


def write_gguf(path, spec, tensors, alignment: int = 32, vocab=None):
    """vocab: None, or token strings written as tokenizer.ggml.tokens (with
    zero tokenizer.ggml.scores), which the reference's loader reads into its
    tokenizer (src/gguf_model.cpp:414-460)."""
    kv = [
        ("general.architecture", GGUF_STRING, _str("llama")),
        ("general.alignment", GGUF_UINT32, struct.pack("<I", alignment)),
        ("llama.block_count", GGUF_UINT32, struct.pack("<I", spec.n_layers)),
        ("llama.embedding_length", GGUF_UINT32, struct.pack("<I", spec.n_embd)),
        ("llama.attention.head_count", GGUF_UINT32, struct.pack("<I", spec.n_head)),
        ("llama.attention.head_count_kv", GGUF_UINT32, struct.pack("<I", spec.n_head_kv)),
        ("llama.feed_forward_length", GGUF_UINT32, struct.pack("<I", spec.n_ff)),
        ("llama.rope.dimension_count", GGUF_UINT32, struct.pack("<I", spec.head_dim)),
        ("llama.rope.freq_base", GGUF_FLOAT32, struct.pack("<f", spec.rope_freq_base)),
        ("llama.context_length", GGUF_UINT32, struct.pack("<I", spec.n_ctx)),
        ("llama.attention.layer_norm_rms_epsilon", GGUF_FLOAT32,
         struct.pack("<f", spec.rms_norm_eps)),
    ]
    if vocab is not None:
        kv.append(("tokenizer.ggml.tokens", GGUF_ARRAY,
                   struct.pack("<IQ", GGUF_STRING, len(vocab)) + b"".join(_str(t) for t in vocab)))
        kv.append(("tokenizer.ggml.scores", GGUF_ARRAY,
                   struct.pack("<IQ", GGUF_FLOAT32, len(vocab)) + b"\0" * (4 * len(vocab))))
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv)))
    for key, ty, val in kv:
        head += _str(key) + struct.pack("<I", ty) + val
    offsets, off = {}, 0
    for name, (dims, ty, raw) in tensors.items():
        offsets[name] = off
        off += (len(raw) + alignment - 1) // alignment * alignment
    for name, (dims, ty, raw) in tensors.items():
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, offsets[name])
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for name, (dims, ty, raw) in tensors.items():
            raw = np.ascontiguousarray(raw, np.uint8).tobytes()
            f.write(raw + b"\0" * ((-len(raw)) % alignment))
