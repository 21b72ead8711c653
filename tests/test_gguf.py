"""The GGUF reader (cpv_gguf_scan / cpv_gguf_hparams) on the CPU, and the
seeded-model writer.

The first three tests re-express the reference reader's own tests
(crates/codpiece-gguf/src/lib.rs:484-550): the minimal v3 file (2 keys, one
F32 [4, 2] tensor), a bad magic, and block sizing (Q8_0 32 -> 34 bytes, 33
elements rejected, Q6_K 512 -> 420).  The others cover the reader's other
checks and the qwen35 hyper-parameter mapping (Hparams::from_gguf,
crates/codpiece-model/src/qwen35.rs:75-130).
"""
import struct

import numpy as np
import pytest

from codpiece_amd import _lib, gguf

MAGIC = 0x46554747


def s8(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def raw_file(tensors, kvs, version=3, pad_data=True, alignment=32):
    """tensors: (name, dims, type, offset); kvs: (key, type id, payload).  The data
    section holds enough zero bytes for every tensor."""
    wide = version >= 3
    L = (lambda n: struct.pack("<Q", n)) if wide else (lambda n: struct.pack("<I", n))
    S = (lambda s: L(len(s.encode())) + s.encode())
    b = struct.pack("<II", MAGIC, version) + L(len(tensors)) + L(len(kvs))
    for k, t, payload in kvs:
        b += S(k) + struct.pack("<I", t) + payload
    for name, dims, t, off in tensors:
        b += S(name) + struct.pack("<I", len(dims)) + b"".join(L(d) for d in dims) + struct.pack("<IQ", t, off)
    b += b"\0" * ((-len(b)) % alignment)
    return b


def scan_bytes(tmp_path, data, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return gguf.scan(p)


def test_reference_mini_file(tmp_path):
    kvs = [("general.architecture", 8, s8("testarch")), ("test.layers", 4, struct.pack("<I", 7))]
    data = raw_file([("t0", [4, 2], 0, 0)], kvs) + b"\0" * 32
    info = scan_bytes(tmp_path, data)
    assert info["version"] == 3 and info["n_tensors"] == 1 and info["n_kv"] == 2
    assert info["tensor_bytes"] == 32
    # 24 header + 48 + 27 key bytes + 42 directory bytes = 141, aligned to 32
    assert info["data_start"] == 160 and info["alignment"] == 32
    with pytest.raises(_lib.CpvError) as e:
        gguf.hparams(tmp_path / "f.gguf")
    assert e.value.status == _lib.CPV_EUNSUPPORTED and "testarch" in str(e.value)


def test_reference_bad_magic(tmp_path):
    with pytest.raises(_lib.CpvError) as e:
        scan_bytes(tmp_path, b"NOPE0000")
    assert "not a GGUF file" in str(e.value)


def test_reference_block_sizing(tmp_path):
    kvs = [("general.architecture", 8, s8("t"))]
    ok = raw_file([("a", [32, 1], 8, 0), ("b", [512, 1], 14, 64)], kvs) + b"\0" * (64 + 420)
    assert scan_bytes(tmp_path, ok)["tensor_bytes"] == 34 + 420
    bad = raw_file([("a", [33, 1], 8, 0)], kvs) + b"\0" * 64
    with pytest.raises(_lib.CpvError):
        scan_bytes(tmp_path, bad, "bad.gguf")


def test_version_2_counts_are_u32(tmp_path):
    kvs = [("general.architecture", 8, struct.pack("<I", 1) + b"x")]
    data = raw_file([("t0", [8], 0, 0)], kvs, version=2) + b"\0" * 32
    info = scan_bytes(tmp_path, data)
    assert info["version"] == 2 and info["tensor_bytes"] == 32


def test_layout_checks(tmp_path):
    kvs = [("general.architecture", 8, s8("t"))]
    # a tensor past the end of the file
    with pytest.raises(_lib.CpvError) as e:
        scan_bytes(tmp_path, raw_file([("t0", [16], 0, 0)], kvs) + b"\0" * 32, "a.gguf")
    assert "of a data section that holds" in str(e.value)
    # an offset off the alignment
    with pytest.raises(_lib.CpvError) as e:
        scan_bytes(tmp_path, raw_file([("t0", [4], 0, 8)], kvs) + b"\0" * 64, "b.gguf")
    assert "not aligned" in str(e.value)
    # overlapping tensors
    with pytest.raises(_lib.CpvError) as e:
        scan_bytes(tmp_path, raw_file([("t0", [16], 0, 32), ("t1", [8], 0, 32)], kvs) + b"\0" * 128, "c.gguf")
    assert "overlaps" in str(e.value)
    # an alignment that is not a power of two
    kv0 = kvs + [("general.alignment", 4, struct.pack("<I", 24))]
    with pytest.raises(_lib.CpvError) as e:
        scan_bytes(tmp_path, raw_file([], kv0) + b"\0" * 32, "d.gguf")
    assert "alignment" in str(e.value)
    # a truncated directory
    with pytest.raises(_lib.CpvError):
        scan_bytes(tmp_path, raw_file([("t0", [4], 0, 0)], kvs)[:40], "e.gguf")
    # an unknown metadata type
    with pytest.raises(_lib.CpvError) as e:
        scan_bytes(tmp_path, raw_file([], [("k", 99, b"")]), "f.gguf")
    assert "unknown metadata value type" in str(e.value)


SMALL = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=1000, n_rot=64,
             rope_sections=(11, 11, 10, 0), rms_eps=1e-6, freq_base=1e6)


def test_seeded_model_roundtrip(tmp_path):
    p = tmp_path / "m.gguf"
    tensors = gguf.write_seeded_model(p, seed=3, qtype=gguf.Q4_K, head_type=gguf.Q6_K, **SMALL)
    info = gguf.scan(p)
    assert info["n_tensors"] == len(tensors)
    assert info["tensor_bytes"] == sum(d.size for _, _, d in tensors.values())
    hp = gguf.hparams(p)
    for k in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab", "n_rot"):
        assert getattr(hp, k) == SMALL[k], k
    assert list(hp.rope_sections) == list(SMALL["rope_sections"])
    assert hp.has_mtp == 1
    assert np.float32(hp.rms_eps) == np.float32(1e-6) and hp.freq_base == 1e6
    # the bytes in the file are the tensors' bytes, at data_start + offset
    raw = p.read_bytes()
    off = info["data_start"]
    for name, (t, dims, data) in tensors.items():
        assert raw[off:off + data.size] == data.tobytes(), name
        off += (data.size + 31) // 32 * 32


def test_hparams_mapping_rules(tmp_path):
    def write(extra, drop=()):
        w = gguf.Writer()
        w.add_str("general.architecture", "qwen35")
        keys = {"qwen35.block_count": 3, "qwen35.embedding_length": 512, "qwen35.attention.head_count": 8,
                "qwen35.attention.head_count_kv": 2, "qwen35.feed_forward_length": 1536,
                "qwen35.full_attention_interval": 1, "qwen35.nextn_predict_layers": 1}
        keys.update(extra)
        for k, v in keys.items():
            if k not in drop:
                w.add_u32(k, v)
        w.add_str_array("tokenizer.ggml.tokens", ["a", "b", "c"])
        p = tmp_path / f"h{len(list(tmp_path.iterdir()))}.gguf"
        w.write(p)
        return p
    hp = gguf.hparams(write({}))
    # defaults: head dim from n_embd / n_head, rope over the whole head, eps 1e-6, base 10000
    assert (hp.n_layer, hp.head_dim, hp.n_rot, hp.n_vocab, hp.has_mtp) == (2, 64, 64, 3, 1)
    assert np.float32(hp.rms_eps) == np.float32(1e-6) and hp.freq_base == 10000.0
    with pytest.raises(_lib.CpvError) as e:
        gguf.hparams(write({"qwen35.full_attention_interval": 4}))
    assert e.value.status == _lib.CPV_EUNSUPPORTED
    with pytest.raises(_lib.CpvError) as e:
        gguf.hparams(write({}, drop=("qwen35.feed_forward_length",)))
    assert "feed_forward_length" in str(e.value)
    with pytest.raises(_lib.CpvError) as e:
        gguf.hparams(write({}, drop=("qwen35.full_attention_interval",)))   # default 4: recurrent layers
    assert e.value.status == _lib.CPV_EUNSUPPORTED
