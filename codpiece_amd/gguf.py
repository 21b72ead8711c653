"""The model file.

Reading goes through the library's reader: `scan` for the structure, and
`hparams` for the qwen35 hyper-parameters (no GPU needed for either).
`codpiece_amd.model.Model.from_gguf` loads a whole model.

Writing is a small GGUF v3 writer (little-endian; typed metadata, a tensor
directory, then the data section at 32-byte alignment, ggml dimension order).
It has one use here: `write_seeded_model` produces a random-init qwen35-layout
model in the layout the reference loads (crates/codpiece-model/src/qwen35.rs:
75-130 for the keys, :159-183 and mtp_graph.rs for the tensor names), with
all-attention layers (full_attention_interval = 1) and one nextn (MTP) layer.
"""
import ctypes
import struct

import numpy as np

from . import _lib

GGUF_MAGIC = 0x46554747
F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

# metadata value types
_U32, _I32, _F32, _BOOL, _STR, _ARR, _U64 = 4, 5, 6, 7, 8, 9, 10


def scan(path):
    """GgufFile::open of the library's reader: a dict of the header facts."""
    lib = _lib.load()
    info = _lib.GgufInfo()
    err = ctypes.create_string_buffer(512)
    st = lib.cpv_gguf_scan(str(path).encode(), ctypes.byref(info), err, len(err))
    if st != _lib.CPV_OK:
        raise _lib.CpvError(st, err.value.decode())
    return {k: getattr(info, k) for k, _ in _lib.GgufInfo._fields_}


def hparams(path):
    """Hparams::from_gguf of the library's reader, as a cpv_hparams structure."""
    lib = _lib.load()
    hp = _lib.Hparams()
    err = ctypes.create_string_buffer(512)
    st = lib.cpv_gguf_hparams(str(path).encode(), ctypes.byref(hp), err, len(err))
    if st != _lib.CPV_OK:
        raise _lib.CpvError(st, err.value.decode())
    return hp


class Writer:
    """Collects metadata and tensors, then writes a GGUF v3 file."""

    def __init__(self, alignment=32):
        self.alignment = alignment
        self.kvs = []        # (key, type, payload bytes)
        self.tensors = []    # (name, ggml type, dims, bytes)

    @staticmethod
    def _str(s):
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def add_u32(self, key, v):
        self.kvs.append((key, _U32, struct.pack("<I", v)))

    def add_f32(self, key, v):
        self.kvs.append((key, _F32, struct.pack("<f", v)))

    def add_str(self, key, v):
        self.kvs.append((key, _STR, self._str(v)))

    def add_i32_array(self, key, vals):
        self.kvs.append((key, _ARR, struct.pack("<IQ", _I32, len(vals)) + struct.pack(f"<{len(vals)}i", *vals)))

    def add_str_array(self, key, vals):
        self.kvs.append((key, _ARR, struct.pack("<IQ", _STR, len(vals)) + b"".join(self._str(v) for v in vals)))

    def add_tensor(self, name, gtype, dims, data):
        """dims in ggml order (ne0 = row length first); data: the ggml bytes."""
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        blk, size = BLOCK[gtype]
        n = int(np.prod(dims))
        if n % blk or data.size != n // blk * size:
            raise ValueError(f"{name}: {data.size} bytes for {dims} of type {gtype}")
        self.tensors.append((name, gtype, list(dims), data))

    def write(self, path):
        a = self.alignment
        head = [struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kvs))]
        for key, t, payload in self.kvs:
            head.append(self._str(key) + struct.pack("<I", t) + payload)
        off = 0
        for name, gtype, dims, data in self.tensors:
            head.append(self._str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                        struct.pack("<IQ", gtype, off))
            off = (off + data.size + a - 1) // a * a
        hb = b"".join(head)
        with open(path, "wb") as f:
            f.write(hb)
            f.write(b"\0" * ((-len(hb)) % a))
            for name, gtype, dims, data in self.tensors:
                f.write(data.tobytes())
                f.write(b"\0" * ((-data.size) % a))


def _f16_bytes(x):
    return np.asarray(x, dtype=np.float16).view(np.uint8).reshape(-1, 2)


def random_blocks(gtype, n_rows, k, rng):
    """Random ggml blocks with plausible scales (weights roughly N(0, 0.02)-sized)."""
    blk, size = BLOCK[gtype]
    nb = n_rows * (k // blk)
    raw = rng.integers(0, 256, size=(nb, size), dtype=np.uint8)
    u = rng.random(nb)
    if gtype == Q8_0:
        raw[:, 0:2] = _f16_bytes(1.5e-4 + 1e-4 * u)                 # d; 32 int8 codes follow
    elif gtype == Q4_K:
        raw[:, 0:2] = _f16_bytes(1.5e-4 + 1e-4 * u)                 # d
        raw[:, 2:4] = _f16_bytes(1.2e-3 + 6e-4 * u)                 # dmin
    elif gtype == Q6_K:
        raw[:, 208:210] = _f16_bytes(1.2e-5 + 6e-6 * u)             # d (the 16 scales are int8)
    else:
        raise ValueError(f"type {gtype}")
    return raw.reshape(-1)


def seeded_tensors(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, seed=0, qtype=Q8_0,
                   head_type=None, has_mtp=True, mtp_shared=False):
    """name -> (ggml type, [ne0, ne1], bytes) of a random-init qwen35 model: linear
    weights of `qtype` (the embedding and output of `head_type`, default `qtype`),
    norm weights 1 + N(0, 0.1) (distinct per tensor).  The query projection
    carries the output gate (2 * n_head * head_dim rows), as the qwen35 graph
    expects.  The nextn layer has its own embedding and head only with
    `mtp_shared` (otherwise it uses the trunk's)."""
    rng = np.random.default_rng(seed)
    head_type = qtype if head_type is None else head_type
    E, H, Hkv, hd, F, V = n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab
    out = {}

    def lin(name, gtype, k, rows):
        out[name] = (gtype, [k, rows], random_blocks(gtype, rows, k, rng))

    def norm(name, n):
        out[name] = (F32, [n, 1], (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32).view(np.uint8))

    lin("token_embd.weight", head_type, E, V)
    for il in range(n_layer + (1 if has_mtp else 0)):
        p = f"blk.{il}."
        norm(p + "attn_norm.weight", E)
        norm(p + "post_attention_norm.weight", E)
        norm(p + "attn_q_norm.weight", hd)
        norm(p + "attn_k_norm.weight", hd)
        lin(p + "attn_q.weight", qtype, E, 2 * H * hd)
        lin(p + "attn_k.weight", qtype, E, Hkv * hd)
        lin(p + "attn_v.weight", qtype, E, Hkv * hd)
        lin(p + "attn_output.weight", qtype, H * hd, E)
        lin(p + "ffn_gate.weight", qtype, E, F)
        lin(p + "ffn_up.weight", qtype, E, F)
        lin(p + "ffn_down.weight", qtype, F, E)
    if has_mtp:
        p = f"blk.{n_layer}.nextn."
        lin(p + "eh_proj.weight", qtype, 2 * E, E)
        norm(p + "enorm.weight", E)
        norm(p + "hnorm.weight", E)
        if mtp_shared:
            lin(p + "embed_tokens.weight", head_type, E, V)
            norm(p + "shared_head_norm.weight", E)
            lin(p + "shared_head_head.weight", head_type, E, V)
    norm("output_norm.weight", E)
    lin("output.weight", head_type, E, V)
    return out


def write_seeded_model(path, n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_rot=None,
                       rope_sections=(0, 0, 0, 0), rms_eps=1e-6, freq_base=1e6, seed=0, qtype=Q8_0,
                       head_type=None, has_mtp=True, mtp_shared=False, context_length=32768):
    """Write a seeded random-init qwen35 model and return its tensors (as
    `seeded_tensors`), so that a caller can load the same bytes directly."""
    tensors = seeded_tensors(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, seed, qtype,
                             head_type, has_mtp, mtp_shared)
    w = Writer()
    w.add_str("general.architecture", "qwen35")
    w.add_u32("qwen35.block_count", n_layer + (1 if has_mtp else 0))
    w.add_u32("qwen35.nextn_predict_layers", 1 if has_mtp else 0)
    w.add_u32("qwen35.context_length", context_length)
    w.add_u32("qwen35.embedding_length", n_embd)
    w.add_u32("qwen35.feed_forward_length", n_ff)
    w.add_u32("qwen35.attention.head_count", n_head)
    w.add_u32("qwen35.attention.head_count_kv", n_head_kv)
    w.add_u32("qwen35.attention.key_length", head_dim)
    w.add_u32("qwen35.attention.value_length", head_dim)
    w.add_f32("qwen35.attention.layer_norm_rms_epsilon", rms_eps)
    w.add_u32("qwen35.rope.dimension_count", head_dim if n_rot is None else n_rot)
    w.add_i32_array("qwen35.rope.dimension_sections", list(rope_sections))
    w.add_f32("qwen35.rope.freq_base", freq_base)
    w.add_u32("qwen35.full_attention_interval", 1)
    w.add_str_array("tokenizer.ggml.tokens", [f"<t{i}>" for i in range(n_vocab)])
    for name, (gtype, dims, data) in tensors.items():
        w.add_tensor(name, gtype, dims, data)
    w.write(path)
    return tensors
